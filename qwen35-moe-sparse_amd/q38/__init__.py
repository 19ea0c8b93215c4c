"""MI355X-native Q38 MoE feed-forward prefill (gfx950 HIP kernels behind a C ABI).

Package layout mirrors the reference's ``q38`` package where the MoE path lives:
``q38.models.qwen3_8_moe`` (drop-in MoE modules), ``q38.inference`` (experts-implementation
registration), ``q38.hip`` (ctypes binding of libq38moe.so) and ``q38.workloads`` (seeded
synthetic inputs of the benchmark configurations).
"""
