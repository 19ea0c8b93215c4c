"""q38moe_block_forward_noalloc (static per-GPU scratch, nothing allocated inside the call)
against q38moe_block_forward (caller workspace), through the C ABI: the same kernels on the same
inputs, so outputs, logits, routing indices and weights are bit-identical. Two calls in a row, the
second smaller and on other tokens, so that anything read from the previous call's scratch would
show; the fused shared expert (Is == I), the separate one (Is != I), the skew bias and token counts
on the small-tile side of the GEMM tiling rule; shapes beyond the scratch are refused with the
library's message."""
import pytest
import torch

pytestmark = pytest.mark.gpu

NAMES = ("gate.weight", "experts.gate_up_proj", "experts.down_proj", "shared_expert.gate_proj.weight",
         "shared_expert.up_proj.weight", "shared_expert.down_proj.weight", "shared_expert_gate.weight")


def _weights(wl, gpu):
    from q38 import workloads
    x, params, bias = workloads.make(wl, tokens=2048)
    return x.to(gpu), [params[n].to(gpu) for n in NAMES], (None if bias is None else bias.to(gpu))


LARGE = ((0, 2048, "persistent"), (1200, 1900, "persistent"))


@pytest.mark.parametrize("name,Is,spans", [
    ("c2", None, LARGE),
    ("c3", None, LARGE),
    ("c2", 128, LARGE),
    ("c2", None, ((0, 300, "small"), (500, 517, "small"))),
])
def test_noalloc_matches_block_forward(gpu, name, Is, spans):
    from q38 import workloads
    from q38.hip import ops
    wl = workloads.get(name) if Is is None else workloads.get(name, shared_inter=Is)
    x, W, bias = _weights(wl, gpu)
    k = wl.topk
    for lo, hi, want_kind in spans:  # second call: fewer tokens, other tokens
        xs = x[lo:hi].contiguous()
        T = xs.shape[0]
        kind = ops.gemm_tiling(T, wl.hidden, wl.experts, k, wl.inter, T if wl.shared_inter == wl.inter else 0)
        print(f"noalloc {name} Is={wl.shared_inter} T={T} {kind} tiles", flush=True)
        assert kind == want_kind
        ref = ops.block_forward(xs, *W, k, logit_bias=bias, return_router=True)
        E = W[0].shape[0]
        logits = torch.empty(T, E, dtype=torch.bfloat16, device=gpu)
        idx = torch.empty(T, k, dtype=torch.int32, device=gpu)
        w = torch.empty(T, k, dtype=torch.bfloat16, device=gpu)
        out = ops.block_forward_noalloc(xs, *W, k, logit_bias=bias, logits=logits, idx=idx, w=w)
        torch.cuda.synchronize()
        for got, want, what in zip((out, logits, idx, w), ref, ("out", "logits", "idx", "w")):
            assert torch.equal(got, want), f"{what} differs at T={T}"


def test_noalloc_refuses_shapes_beyond_scratch(gpu):
    from q38 import workloads
    from q38.hip import _lib, ops
    wl = workloads.get("c2")
    x, W, _ = _weights(wl, gpu)
    cap = int(_lib.lib.q38moe_block_noalloc_scratch_bytes())
    assert cap == 32 << 20
    T_max = max(t for t in range(2048, 2400)
                if ops.block_workspace_bytes(t, wl.hidden, wl.experts, wl.topk, wl.inter, wl.shared_inter) <= cap)
    big = torch.zeros(T_max + 1, wl.hidden, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="static scratch holds"):
        ops.block_forward_noalloc(big, *W, wl.topk)
    # the largest shape it holds runs and matches
    xs = torch.cat([x, x[: T_max - x.shape[0]]]).contiguous()
    out = ops.block_forward_noalloc(xs, *W, wl.topk)
    ref = ops.block_forward(xs, *W, wl.topk)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
