"""Benchmark: Q38 MoE-layer forward (one Qwen3_8MoeSparseMoeBlock) on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2] [--no-cpu-baseline] [--backward]

A step is one fused block forward (router, permutation, grouped gate/up + SwiGLU, grouped down x
routing weight, shared expert, gated combine) over the workload's packed tokens, inputs resident in
HBM. Prints ONE JSON line: whole-job tokens/s, the roofline of the dominant kernel (per-kernel
durations measured here with HIP events on the launch stream), and the reference's CPU block
forward timed on this host on a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "qwen35-moe-sparse_amd"))
sys.path.insert(0, str(REPO))

METRIC = "MoE-layer tokens/sec at 16K tokens bf16 (1 GPU) + % MFMA peak"
PEAK_BF16 = 2.5e15   # dense bf16 MFMA, MI355X datasheet
PEAK_FP8 = 5.0e15    # dense fp8 MFMA, MI355X datasheet
PEAK_HBM = 8.0e12    # HBM3E bytes/s
PEAK_FP32 = 157.3e12  # dense fp32 MFMA, MI355X datasheet


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def time_stream(fn, iters, stream):
    """Seconds per launch of `fn` (stage kernels relaunched back to back on `stream`). A GPU spin
    queued first keeps the device busy while the host enqueues every launch, so the events time the
    kernels back to back, not the host's per-call work (output allocation, argument checks)."""
    import torch
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        # about 2 ms of spinning at the MI355X clock, and 125 us more per launch beyond 16 (the
        # slowest host call, the route's, takes well under that)
        torch.cuda._sleep(4_000_000 + 250_000 * max(0, iters - 16))
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters * 1e-3  # seconds per launch


def kernel_breakdown(wl, x, d, bias, iters, stream):
    """Average duration of each stage kernel, launched alone back to back on `stream`. fp32
    workloads: the route stage is the fp32 block's three launches (router logits GEMM, shared gate
    logit GEMM, selection)."""
    import torch
    from q38.hip import ops
    T, h, E, k, I, Is = wl.tokens, wl.hidden, wl.experts, wl.topk, wl.inter, wl.shared_inter
    P = T * k
    f32 = x.dtype == torch.float32
    esz = 4 if f32 else 2
    peak_mfma = PEAK_FP32 if f32 else PEAK_BF16

    def route_fn():
        return ops.route(x, d["gate.weight"], k, w_shared_gate=d["shared_expert_gate.weight"], logit_bias=bias,
                         want_hist=True)
    logits, idx, w, gate, hist = route_fn()
    fused = I == Is
    srows = T if fused else 0
    counts, starts, perm, inv, tiles, tcount = ops.permute(idx, hist, E, shared_rows=srows)
    sh_w = (d["shared_expert.gate_proj.weight"], d["shared_expert.up_proj.weight"])
    H = ops.gate_up(x, d["experts.gate_up_proj"], perm, tiles, tcount, k, shared_weights=sh_w, shared_rows=srows)
    Y = ops.down(H, d["experts.down_proj"], tiles, tcount, T, k, w_shared_down=d["shared_expert.down_proj.weight"],
                 shared_rows=srows)
    sh = Y[P:] if fused else ops.shared_expert(x, *sh_w, d["shared_expert.down_proj.weight"])
    torch.cuda.synchronize()
    fl = wl.flops()
    sh_fl = fl["shared"] if fused else 0
    # The small-tile GEMMs (few rows per expert) stream each routed expert's weights once: their
    # bound is HBM, the algorithmic bytes those weights plus the rows read and written.
    small = not f32 and ops.gemm_tiling(T, h, E, k, I, srows) == "small"
    used = int((counts > 0).sum())
    rows = P + srows
    gu_bound, gu_work = ("hbm", (used * 2 * I * h + (2 * I * h if fused else 0) + rows * (h + I)) * esz) \
        if small else ("mfma", fl["gate_up"] + sh_fl * 2 // 3)
    dn_bound, dn_work = ("hbm", (used * h * I + (h * I if fused else 0) + rows * (I + h)) * esz) \
        if small else ("mfma", fl["down"] + sh_fl // 3)
    stages = {
        "route": (route_fn, "hbm",
                  # x read + router weights + idx/w/gate/hist written
                  (T * h + (E + 1) * h + T) * esz + P * (4 + esz)),
        "permute": (lambda: ops.permute(idx, hist, E, shared_rows=srows), "hbm", P * 4 * 3),
        # gate/up: routed pairs (+ the shared expert's gate/up when it runs in the same launch)
        "gate_up": (lambda: ops.gate_up(x, d["experts.gate_up_proj"], perm, tiles, tcount, k, shared_weights=sh_w,
                                        shared_rows=srows), gu_bound, gu_work),
        "down": (lambda: ops.down(H, d["experts.down_proj"], tiles, tcount, T, k,
                                  w_shared_down=d["shared_expert.down_proj.weight"], shared_rows=srows), dn_bound,
                 dn_work),
        # combine reads k bf16 rows + the shared row, writes one row per token
        "combine": (lambda: ops.combine(Y, inv, w, E, shared_out=sh, shared_gate_logit=gate), "hbm",
                    T * h * esz * (k + 2)),
    }
    if not fused:
        stages["shared_expert"] = (lambda: ops.shared_expert(x, *sh_w, d["shared_expert.down_proj.weight"]), "mfma",
                                   fl["shared"])
    out = {}
    for name, (fn, bound, work) in stages.items():
        fn()
        dt = time_stream(fn, iters, stream)
        if bound == "mfma":
            achieved, peak, unit = work / dt / 1e12, peak_mfma / 1e12, "TFLOP/s"
        else:
            achieved, peak, unit = work / dt / 1e9, PEAK_HBM / 1e9, "GB/s"
        out[name] = dict(us=round(dt * 1e6, 2), bound=bound, work=work, achieved=round(achieved, 2),
                         peak=peak, unit=unit, frac=round(achieved / peak, 4))
    for name in ("gate_up", "down"):
        out[name]["tiling"] = "fp32" if f32 else ("small" if small else "persistent")
    return out


def kernel_breakdown_fp8(wl, x, d, wq, bias, iters, stream):
    """Per-stage durations of the fp8 block (e4m3 experts), each stage relaunched alone."""
    import torch
    from q38.hip import ops
    T, h, E, k, I = wl.tokens, wl.hidden, wl.experts, wl.topk, wl.inter
    P = T * k
    logits, idx, w, gate, hist = ops.route(x, d["gate.weight"], k, w_shared_gate=d["shared_expert_gate.weight"],
                                           logit_bias=bias, want_hist=True)
    xq, sx = ops.quantize_rows(x)
    counts, starts, perm, inv, tiles, tcount = ops.permute(idx, hist, E, shared_rows=T)
    row_scale = torch.cat([sx[perm.long() // k], sx])
    H = ops.gate_up_fp8(xq, row_scale, wq, perm, tiles, tcount, k, shared_rows=T)
    Hq, sH = ops.quantize_rows(H)
    Y = ops.down_fp8(Hq, sH, wq, tiles, tcount, T, k, shared_rows=T)
    torch.cuda.synchronize()
    fl = wl.flops()
    # The e4m3 small tiles (few rows per expert) stream each routed expert's codes and scales once:
    # their bound is HBM, the algorithmic bytes those weights (shared expert included) plus the rows
    # (codes and row scale in, bf16 out).
    small = ops.gemm_tiling(T, h, E, k, I, T, fp8=True) == "small"
    used = int((counts > 0).sum()) + 1
    rows = P + T
    gu_bound, gu_work = ("hbm", used * 2 * I * (h + 4) + rows * (h + 4 + I * 2)) if small else \
        ("mfma", fl["gate_up"] + fl["shared"] * 2 // 3)
    dn_bound, dn_work = ("hbm", used * h * (I + 4) + rows * (I + 4 + h * 2)) if small else \
        ("mfma", fl["down"] + fl["shared"] // 3)
    stages = {
        "route": (lambda: ops.route(x, d["gate.weight"], k, w_shared_gate=d["shared_expert_gate.weight"],
                                    logit_bias=bias, want_hist=True), "hbm",
                  T * h * 2 + (E + 1) * h * 2 + P * 6 + T * 2),
        # x read (bf16) + e4m3 codes and scales written
        "quant_x": (lambda: ops.quantize_rows(x), "hbm", T * h * 3 + T * 4),
        "permute": (lambda: ops.permute(idx, hist, E, shared_rows=T), "hbm", P * 4 * 3),
        "gate_up": (lambda: ops.gate_up_fp8(xq, row_scale, wq, perm, tiles, tcount, k, shared_rows=T), gu_bound,
                    gu_work),
        "quant_h": (lambda: ops.quantize_rows(H), "hbm", (P + T) * I * 3 + (P + T) * 4),
        "down": (lambda: ops.down_fp8(Hq, sH, wq, tiles, tcount, T, k, shared_rows=T), dn_bound, dn_work),
        "combine": (lambda: ops.combine(Y, inv, w, E, shared_out=Y[P:], shared_gate_logit=gate), "hbm",
                    T * h * 2 * (k + 2)),
    }
    out = {}
    for name, (fn, bound, work) in stages.items():
        fn()
        dt = time_stream(fn, iters, stream)
        if bound == "mfma":
            achieved, peak, unit = work / dt / 1e12, PEAK_FP8 / 1e12, "TFLOP/s"
        else:
            achieved, peak, unit = work / dt / 1e9, PEAK_HBM / 1e9, "GB/s"
        out[name] = dict(us=round(dt * 1e6, 2), bound=bound, work=work, achieved=round(achieved, 2),
                         peak=peak, unit=unit, frac=round(achieved / peak, 4))
    for name in ("gate_up", "down"):
        out[name]["tiling"] = "small" if small else "persistent"
    return out


def _time_cpu_block(wl, dtype, experts, budget_s, max_runs=400):
    """Median seconds of the reference block's op sequence (oracle.reference_block_forward) on this
    host's CPU in `dtype` with the given experts implementation: 1 warmup, then runs over a sample
    of the workload's tokens (all of them unless one run would exceed a third of the budget) until
    about `budget_s` seconds of work are done, at least 3."""
    import torch
    from oracle import moe_oracle
    from q38 import workloads
    x_all, params, bias = workloads.make(wl, dtype=dtype)
    tokens = min(1024, wl.tokens)
    with torch.inference_mode():
        t0 = time.perf_counter()
        moe_oracle.reference_block_forward(x_all[:tokens], params, wl.topk, logit_bias=bias, experts=experts)
        per_tok = (time.perf_counter() - t0) / tokens
        tokens = int(max(min(1024, wl.tokens), min(wl.tokens, budget_s / 3 / max(per_tok, 1e-9))))
        x = x_all[:tokens]
        moe_oracle.reference_block_forward(x, params, wl.topk, logit_bias=bias, experts=experts)  # warmup
        times = []
        start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < max_runs):
            t0 = time.perf_counter()
            moe_oracle.reference_block_forward(x, params, wl.topk, logit_bias=bias, experts=experts)
            times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return dict(tokens=tokens, runs=len(times), seconds_total=round(sum(times), 2), seconds_median=round(med, 5),
                value=round(tokens / med, 1))


def _host_cpu():
    """Model name, family/model/stepping and core counts of this host (lscpu / cpuinfo)."""
    import subprocess
    import torch
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip() in ("Model name", "CPU family", "Model", "Stepping", "Socket(s)", "Core(s) per socket",
                               "Thread(s) per core"):
                info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return dict(cpu_model=info.get("Model name", ""), lscpu=info, os_cpu_count=os.cpu_count(),
                torch_threads=torch.get_num_threads(), torch_cpu_capability=torch.backends.cpu.get_cpu_capability())


def cpu_baseline(wl, budget_s=8.0):
    """The reference block on this host's CPU (BASELINE plan): the primary figure is the eager
    experts loop (the module's own forward, modeling_qwen3_8_moe.py:769-793) in the workload's
    dtype over the workload's tokens; `variants` adds transformers' grouped_mm experts (the
    presets' configured implementation, integrations/moe.py:377-478) on the same tokens, and, for
    the bf16 workloads, configuration 1 (fp32, h=256) with both implementations."""
    import torch
    from q38 import workloads
    torch.set_num_threads(os.cpu_count() or 1)
    bf = torch.float32 if wl.dtype == "fp32" else torch.bfloat16
    dname = "fp32" if bf == torch.float32 else "bf16"
    runs = {f"eager_{dname}_{wl.name}": (wl, bf, "eager", budget_s),
            f"grouped_mm_{dname}_{wl.name}": (wl, bf, "grouped_mm", budget_s * 0.75)}
    if wl.name != "c1":
        c1 = workloads.get("c1")
        runs["eager_fp32_c1"] = (c1, torch.float32, "eager", budget_s * 0.4)
        runs["grouped_mm_fp32_c1"] = (c1, torch.float32, "grouped_mm", budget_s * 0.4)
    variants = {}
    for name, (w_, dt, ex, bud) in runs.items():
        r = _time_cpu_block(w_, dt, ex, bud)
        r.update(unit="tokens/s", workload=w_.name, dtype="fp32" if dt == torch.float32 else "bf16", experts=ex)
        variants[name] = r
        log(f"[bench] cpu {name}: {r['value']} tokens/s ({r['runs']} runs over {r['tokens']} tokens)")
    prim = variants[f"eager_{dname}_{wl.name}"]
    host = _host_cpu()
    return dict(value=prim["value"], unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"{prim['runs']} block forwards over {prim['tokens']} of the {wl.tokens} tokens of {wl.name} "
                       f"(h={wl.hidden}, E={wl.experts}, k={wl.topk}, I={wl.inter}), {prim['seconds_total']:.1f} s of "
                       f"CPU work; {dname} torch CPU running the reference op sequence with the eager experts loop "
                       f"(modeling_qwen3_8_moe.py:769-793,805-813,824-835); value = tokens / median run after one "
                       f"warmup; variants: grouped_mm experts (transformers integrations/moe.py:377-478) and "
                       f"configuration 1 in fp32, same protocol",
                runs=prim["runs"], seconds_total=prim["seconds_total"], seconds_median=prim["seconds_median"],
                variants=variants, **host)


# Kernel symbol of each stage, as rocprofv3 names it (the committed PMC byte counts are keyed by stage
# and record the full kernel name they were read from): bf16 gate/up runs the four-wave kernel where
# its shape rule allows, the eight-wave grouped kernel otherwise (fp8, narrow K or N).
KERNEL_SYMBOLS = {
    "route": ("q38::route_kernel",),
    "permute": ("q38::permute_kernel",),
    "gate_up": ("gemm4w_gate_up_kernel", "q38::grouped_gemm_kernel<0,"),
    "down": ("q38::grouped_gemm_kernel<1,",),
    "combine": ("q38::combine_kernel",),
}
TRAFFIC_FILE = REPO / "profiles" / "hbm_traffic.json"


def hbm_traffic(workload, stage):
    """HBM bytes per launch of `stage` from the committed rocprofv3 PMC summary: the read requests that
    leave L2 weighted by their size (TCC_EA0_RDREQ_32B/64B/128B) plus WRITE_SIZE, each scaled by the
    factor a plain 256 MiB copy gives the same counters. None when no summary for this workload and
    stage exists."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    entry = data.get("workloads", {}).get(workload, {}).get(stage)
    return entry.get("hbm_bytes") if entry else None


MFMA_FILE = REPO / "profiles" / "mfma_busy.json"


def mfma_busy(workload, stage):
    """(MFMA busy %, engine clock GHz) of `stage` from the committed rocprofv3 PMC summary
    (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE per XCD x 1024 SIMDs; clock = GRBM_GUI_ACTIVE per
    XCD / dispatch duration), or None when no summary for this workload and stage exists."""
    try:
        entry = json.loads(MFMA_FILE.read_text())["workloads"][workload][stage]
    except (OSError, ValueError, KeyError):
        return None
    return {"mfma_busy_pct": entry["mfma_busy_pct"], "clock_ghz": entry["clock_ghz"],
            "source": "profiles/mfma_busy.json"}


def copy_probe(mib):
    """One device-to-device copy of `mib` MiB: the known-size reference for the FETCH_SIZE and
    WRITE_SIZE counters in a PMC run of this script."""
    import torch
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy probe: {mib} MiB read, {mib} MiB written")


def prefill_bench(args):
    """Workload c5: the packed no-cache prefill of a 12-layer random-init Q38 model (q38.prefill)
    on 4 x 4096 tokens, the fused HIP MoE block in every layer; the token mixers are torch code.
    Reports whole-model tokens/s, the share of the 12 MoE blocks, and a bounded CPU sample of the
    same restatement (CPU oracle in place of the HIP blocks)."""
    import torch
    from q38 import prefill as P

    cfg = P.c5_config()
    dev = torch.device("cuda:0")
    batch, seq = 4, 4096
    t0 = time.time()
    params = P.init_params(cfg, 0)
    model = P.Q38Prefill(cfg).load_params(params).to(device=dev, dtype=torch.bfloat16)
    ids = P.make_ids(batch, seq, cfg).to(dev)
    log(f"[bench] c5 prefill model built in {time.time() - t0:.1f} s")
    stream = torch.cuda.current_stream(dev)
    with torch.inference_mode():
        for _ in range(args.warmup):
            model(ids)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(args.steps):
            model(ids)
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / args.steps
        log(f"[bench] timed {args.steps} prefill steps: {ms:.2f} ms/step")
        # One MoE block on a layer-shaped input, as inside the prefill (T = batch * seq tokens).
        blk = model.model.layers[0].mlp
        xb = torch.randn(batch, seq, cfg.hidden, device=dev).to(torch.bfloat16)
        for _ in range(3):
            blk(xb)
        start.record(stream)
        for _ in range(20):
            blk(xb)
        end.record(stream)
        torch.cuda.synchronize()
        moe_ms = start.elapsed_time(end) / 20
    T = batch * seq
    res = {
        "metric": "Q38 packed no-cache prefill tokens/sec (config 5, 1 GPU)",
        "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded random-init parameters, uniform token ids with EOS about every 1000)",
        "config": {"workload": f"c5: 12-layer Q38 packed prefill, {batch}x{seq} tokens", "layers": cfg.layers,
                   "hidden": cfg.hidden, "experts": cfg.experts, "top_k": cfg.topk, "vocab": cfg.vocab,
                   "parallelism": "single GPU"},
        "roofline": None,
        "moe": {"ms_per_block": round(moe_ms, 4), "blocks": cfg.layers,
                "share_of_step": round(cfg.layers * moe_ms / ms, 4),
                "mfma_frac_block": round(moe_block_flops(cfg, T) / (moe_ms * 1e-3) / PEAK_BF16, 4)},
    }
    if not args.no_cpu_baseline:
        import oracle.moe_oracle as O

        def cpu_moe(block, x):
            w = {n: q for n, q in block.named_parameters()}
            B, S, h = x.shape
            return O.reference_block_forward(x.reshape(-1, h), w, block.gate.top_k).view(B, S, h)

        cpu = P.Q38Prefill(cfg, moe_forward=cpu_moe).load_params(params).to(dtype=torch.bfloat16)
        sample = P.make_ids(1, 1024, cfg)
        t = time.time()
        cpu(sample)
        sec = time.time() - t
        res["cpu_baseline"] = {"value": round(1024 / sec, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
                               "kind": "port", "sample": "one 1024-token sequence through the same 12-layer "
                               "restatement in bf16 torch on the host cores, CPU oracle MoE blocks"}
    print(json.dumps(res), flush=True)


def backward_bench(args):
    """Routed experts forward + backward (q38.hip.autograd.experts, the differentiable counterpart
    of the reference's padded experts path) on the workload's tokens: gradients of x,
    top_k_weights, gate_up_proj and down_proj. Reports tokens/s of the training step and each
    backward kernel's average duration, relaunched alone on the stream."""
    import torch
    from q38 import workloads
    from q38.hip import autograd, ops

    wl = workloads.get(args.workload, batch=1, seq=args.tokens) if args.tokens else workloads.get(args.workload)
    dev = torch.device("cuda:0")
    f32 = wl.dtype == "fp32"
    dt = torch.float32 if f32 else torch.bfloat16
    x, params, bias = workloads.make(wl, device="cpu", dtype=dt)
    x = x.to(dev)
    d = {n: p.to(dev).contiguous() for n, p in params.items()}
    T, h, E, k, I = wl.tokens, wl.hidden, wl.experts, wl.topk, wl.inter
    P = T * k
    with torch.inference_mode():
        _, idx, w, _, _ = ops.route(x, d["gate.weight"], k, w_shared_gate=d["shared_expert_gate.weight"],
                                    logit_bias=bias, want_hist=True)
    idx, w = idx.clone(), w.clone()
    leaves = [x.clone().requires_grad_(True), w.requires_grad_(True),
              d["experts.gate_up_proj"].clone().requires_grad_(True), d["experts.down_proj"].clone().requires_grad_(True)]
    dout = (torch.randn(T, h, device=dev) * 0.05).to(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)

    def step():
        for t in leaves:
            t.grad = None
        out = autograd.experts(leaves[0], idx, *leaves[1:])
        out.backward(dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    log(f"[bench] timed {args.steps} forward+backward steps: {ms:.4f} ms/step")

    # Backward stages alone, on the saved forward state.
    with torch.no_grad():
        xb, wb, wgu, wdn = (t.detach() for t in leaves)
        hist = ops.histogram(idx, E)
        counts, starts, perm, inv, tiles, tcount = ops.permute(idx, hist, E)
        H, GU = ops.gate_up_save(xb, wgu, perm, tiles, tcount, k)
        Y = ops.down(H, wdn, tiles, tcount, T, k)
        d_raw = ops.gather_rows(dout, perm, starts, counts, k, w=wb)
        dH = ops.down_kn(d_raw, wdn, tiles, tcount, T, k)
        dGU = ops.swiglu_backward(dH, GU)
        dxp = ops.down_kn(dGU, wgu, tiles, tcount, T, k)
        ones = torch.ones_like(wb)
        xs = ops.gather_rows(xb, perm, starts, counts, k)
        it = args.kernel_iters
        fl = lambda n: {"work": n, "unit": "TFLOP/s", "peak": PEAK_BF16 / 1e12, "bound": "mfma"}
        by = lambda n: {"work": n, "unit": "GB/s", "peak": PEAK_HBM / 1e9, "bound": "hbm"}
        stages = {
            "pair_dots_rows": (lambda: ops.pair_dots(dout, Y, inv, idx, E, w=wb), by(2 * (T * h + 2 * P * h) + 4 * P)),
            "dH_down_kn": (lambda: ops.down_kn(d_raw, wdn, tiles, tcount, T, k), fl(2 * P * h * I)),
            "fwd_gate_up_save": (lambda: ops.gate_up_save(xb, wgu, perm, tiles, tcount, k), fl(2 * P * h * 2 * I)),
            "fwd_gate_up": (lambda: ops.gate_up(xb, wgu, perm, tiles, tcount, k), fl(2 * P * h * 2 * I)),
            "swiglu_backward": (lambda: ops.swiglu_backward(dH, GU), by(2 * (P * I + 2 * P * 2 * I))),
            "dx_down_kn": (lambda: ops.down_kn(dGU, wgu, tiles, tcount, T, k), fl(2 * P * 2 * I * h)),
            "dx_combine": (lambda: ops.combine(dxp, inv, ones, E, idx=idx), by(2 * (P * h + T * h))),
            "wgrad_gate_up": (lambda: ops.expert_wgrad(dGU, xb, starts, counts, k, perm=perm), fl(2 * P * 2 * I * h)),
            "wgrad_gate_up_presorted": (lambda: ops.expert_wgrad(dGU, xs, starts, counts, k), fl(2 * P * 2 * I * h)),
            "wgrad_down": (lambda: ops.expert_wgrad(d_raw, H, starts, counts, k), fl(2 * P * h * I)),
        }
        kernels = {}
        for name, (fn, meta) in stages.items():
            fn()
            sec = time_stream(fn, it, stream)
            scale = 1e12 if meta["unit"] == "TFLOP/s" else 1e9
            ach = meta["work"] / sec / scale
            kernels[name] = {"us": round(sec * 1e6, 2), "bound": meta["bound"], "achieved": round(ach, 1),
                             "peak": meta["peak"], "unit": meta["unit"], "frac": round(ach / meta["peak"], 4),
                             "work": meta["work"]}
    log("[bench] backward kernels: " + ", ".join(f"{n} {v['us']}us" for n, v in kernels.items()))
    # Algorithmic FLOPs: forward 6 P h I (gate/up 4, down 2) + backward 12 P h I (dH 2, dx rows 4,
    # gate_up_proj gradient 4, down_proj gradient 2); the forward keeps [g | u], nothing is recomputed.
    flops = 18 * P * h * I
    res = {
        "metric": "routed-experts forward+backward tokens/sec (1 GPU)",
        "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights, N(0,0.05) output gradient)",
        "config": {"workload": f"{wl.name}: routed experts forward+backward, {wl.batch}x{wl.seq} packed tokens",
                   "tokens": T, "hidden": h, "experts": E, "top_k": k, "expert_inter": I,
                   "parallelism": "single GPU"},
        "mfma_frac_step": round(flops / (ms * 1e-3) / PEAK_BF16, 4),
        "kernels": kernels,
    }
    print(json.dumps(res), flush=True)


def moe_block_flops(cfg, T):
    """MoE block FLOPs for T tokens: routed experts, shared expert, router (flops.py:25, 38-40)."""
    h, I, Is, E, k = cfg.hidden, cfg.moe_ffn, cfg.shared_ffn, cfg.experts, cfg.topk
    return 2 * T * k * h * 3 * I + 6 * T * h * Is + 2 * T * h * E


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c2")
    ap.add_argument("--graph", action="store_true",
                    help="time replays of the block captured as one HIP graph (q38.hip.graph.BlockGraph) "
                         "instead of eager calls")
    ap.add_argument("--tokens", type=int, default=0,
                    help="run the workload's shapes on this many tokens (one sequence) instead of its own "
                         "batch x seq: decode and short-chunk sizes, where the small-tile GEMMs run")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--backward", action="store_true",
                    help="time the routed experts forward + backward (training step) instead")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="end with one copy of this many MiB (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this benchmark measures one GPU only; the MoE block is data-parallel "
                                   "across GPUs with no exchange, run one process per GPU", "n_gpus": args.gpus}))
        sys.exit(2)

    if args.workload == "c5":
        prefill_bench(args)
        return
    if args.backward:
        backward_bench(args)
        return
    import torch
    from q38 import workloads
    from q38.hip import ops

    wl = workloads.get(args.workload, batch=1, seq=args.tokens) if args.tokens else workloads.get(args.workload)
    dev = torch.device("cuda:0")
    log(f"[bench] workload {wl.name}: T={wl.tokens} h={wl.hidden} E={wl.experts} k={wl.topk} I={wl.inter} "
        f"Is={wl.shared_inter}")
    f32 = wl.dtype == "fp32"
    dt = torch.float32 if f32 else torch.bfloat16
    x, params, bias = workloads.make(wl, device="cpu", dtype=dt)
    x = x.to(dev)
    d = {n: p.to(dev).contiguous() for n, p in params.items()}
    if bias is not None:
        bias = bias.to(dev)
    T, h = x.shape
    k = wl.topk
    ws = torch.empty(ops.block_workspace_bytes(T, h, wl.experts, k, wl.inter, wl.shared_inter, dtype=dt),
                     dtype=torch.uint8, device=dev)
    out = torch.empty(T, h, dtype=dt, device=dev)
    weights = [d[n] for n in workloads.PARAM_ORDER]
    stream = torch.cuda.current_stream(dev)
    fp8 = wl.dtype == "fp8"
    if fp8:
        # e4m3 expert weights with per-output-channel scales, quantised once before timing (load time).
        wq = ops.quantize_weights_fp8(d)
        ws = torch.empty(ops.block_fp8_workspace_bytes(T, h, wl.experts, k, wl.inter), dtype=torch.uint8,
                         device=dev)

    graph = None
    if args.graph and not fp8:
        from q38.hip.graph import BlockGraph
        graph = BlockGraph(weights, k, T, logit_bias=bias)
        graph.x.copy_(x)

    def step():
        if graph is not None:
            graph.replay()
        elif fp8:
            ops.block_forward_fp8(x, d["gate.weight"], wq, d["shared_expert_gate.weight"], k, logit_bias=bias,
                                  workspace=ws, out=out)
        else:
            ops.block_forward(x, *weights, k, logit_bias=bias, workspace=ws, out=out)

    with torch.inference_mode():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        log(f"[bench] warmup {args.warmup} done")
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            step()
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / args.steps
        log(f"[bench] timed {args.steps} steps: {ms:.4f} ms/step")
        kernels = (kernel_breakdown_fp8(wl, x, d, wq, bias, args.kernel_iters, stream) if fp8 else
                   kernel_breakdown(wl, x, d, bias, args.kernel_iters, stream))
        log(f"[bench] kernels: " + ", ".join(f"{n} {v['us']}us" for n, v in kernels.items()))

    fl = wl.flops()
    peak_mfma = PEAK_FP8 if fp8 else (PEAK_FP32 if f32 else PEAK_BF16)
    # MFMA counters were collected at the workloads' own sizes only.
    counters = (lambda n: None) if args.tokens else (lambda n: mfma_busy(wl.name, n))
    for name in ("gate_up", "down"):
        kernels[name]["mfma_counters"] = counters(name)
    dom = max(kernels, key=lambda n: kernels[n]["us"])
    dk = kernels[dom]
    expert_us = kernels["gate_up"]["us"] + kernels["down"]["us"]
    # routed + shared expert FLOPs of the two grouped launches (the shared expert runs inside them
    # when its width equals the routed experts')
    expert_fl = fl["experts"] + (fl["shared"] if fp8 or wl.inter == wl.shared_inter else 0)
    res = {
        "metric": METRIC,
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8 e4m3 experts (fp32 accumulate), bf16 router/activations" if fp8 else ("fp32" if f32 else "bf16"),
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights; no checkpoint)",
        "config": {"workload": f"{wl.name}: one Q38 MoE block forward, {wl.batch}x{wl.seq} packed tokens",
                   "tokens": T, "hidden": h, "experts": wl.experts, "top_k": k, "expert_inter": wl.inter,
                   "shared_inter": wl.shared_inter, "routing_skew": wl.zipf_s, "parallelism": "single GPU",
                   "gemm_tiling": kernels["gate_up"].get("tiling", "persistent"),
                   "launch": "hip_graph" if graph is not None else "eager"},
        "roofline": {"kernel": dom, "bound": dk["bound"], "achieved": dk["achieved"], "peak": dk["peak"],
                     "unit": dk["unit"], "frac": dk["frac"],
                     "traffic": None if args.tokens else hbm_traffic(wl.name, dom),
                     "work_per_launch": dk["work"], "mfma_counters": counters(dom)},
        # Routed + shared expert GEMM FLOPs over the two grouped launches that compute them.
        "mfma_frac_expert_gemms": round(expert_fl / (expert_us * 1e-6) / peak_mfma, 4),
        "mfma_frac_block": round(fl["block"] / (ms * 1e-3) / peak_mfma, 4),
        "kernels": kernels,
    }
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU baseline")
        res["cpu_baseline"] = cpu_baseline(wl)
        log(f"[bench] cpu baseline: {res['cpu_baseline']['value']} tokens/s")
    if args.copy_probe_mib > 0:
        copy_probe(args.copy_probe_mib)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
