"""The block forward captured as a HIP graph (q38.hip.graph.BlockGraph): every replay equals the
eager ops.block_forward on the same input bit for bit (the graph runs the same launches; the block
has no floating-point atomics), across replays with new inputs and with eager work and
synchronisations in between, on both GEMM tilings and in fp32."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _setup(name, T, dtype=torch.bfloat16, **over):
    from q38 import workloads
    wl = workloads.get(name, **over) if over else workloads.get(name)
    x, params, bias = workloads.make(wl, tokens=4 * T, dtype=dtype)
    return wl, x, params, bias


@pytest.mark.parametrize("name,T,dtype", [("c2", 1, torch.bfloat16), ("c2", 64, torch.bfloat16),
                                          ("c3", 300, torch.bfloat16), ("c2", 4096, torch.bfloat16),
                                          ("c1", 256, torch.float32)])
def test_block_graph_replays_match_eager(gpu, name, T, dtype):
    from q38 import workloads
    from q38.hip import ops
    from q38.hip.graph import BlockGraph
    wl, x, p, bias = _setup(name, T, dtype)
    w = [p[n].to(gpu) for n in workloads.PARAM_ORDER]
    b = None if bias is None else bias.to(gpu)
    g = BlockGraph(w, wl.topk, T, logit_bias=b, return_router=True)
    xs = x.to(gpu)
    for rep in range(4):
        xin = xs[rep * T:(rep + 1) * T].contiguous()
        out = g(xin).clone()
        logits, idx, wts = g.logits.clone(), g.idx.clone(), g.w.clone()
        # eager work between replays, on the same stream
        ref, ref_logits, ref_idx, ref_w = ops.block_forward(xin, *w, wl.topk, logit_bias=b, return_router=True)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}: output differs from eager"
        assert torch.equal(logits, ref_logits) and torch.equal(idx, ref_idx) and torch.equal(wts, ref_w)
    # replaying the last input again gives the same answer
    again = g.replay().clone()
    torch.cuda.synchronize()
    assert torch.equal(again, ref)


def test_block_graph_rejects_wrong_input(gpu):
    from q38 import workloads
    from q38.hip.graph import BlockGraph
    wl, x, p, _ = _setup("c2", 8)
    w = [p[n].to(gpu) for n in workloads.PARAM_ORDER]
    g = BlockGraph(w, wl.topk, 8)
    with pytest.raises(ValueError):
        g(x[:9].to(gpu))
