"""The MoE block forward captured as one HIP graph, for callers that capture their serving loop.

Serving stacks capture whole decoder layers or models into graphs and replay them; the block must
then be capturable. It is: the library neither allocates nor clears memory inside a call (the
caller's workspace is carved, and every buffer the block reads is written first in the same call),
so a capture holds its kernel nodes only (route, permute, the two grouped GEMMs, combine, and the
shared expert's own GEMMs when its width differs), and every replay equals the eager call bit for
bit (tests/test_gpu_graph.py). Replaying the block alone is not faster than calling it: on one
MI355X at configuration 2's shapes an eager block takes 34.4 us per call at T = 1 against 37.9 us
per graph replay (bench.py --tokens 1 [--graph]), the launches being issued faster than the GPU runs
them either way.

The reference has no counterpart (its serving path runs the block eagerly, modeling:824-835); the
graph runs exactly the launches of ``ops.block_forward`` with its arguments fixed.
"""
import torch

from . import ops


class BlockGraph:
    """``ops.block_forward`` on [T, h] inputs captured into a ``torch.cuda.CUDAGraph``.

    weights: the seven block tensors in state-dict order (router, gate_up_proj, down_proj, shared
    gate, up, down, shared_expert_gate), on one GPU, all bf16 or all fp32. The input buffer ``x``,
    the output ``out`` and the workspace are allocated here and stay fixed: write the tokens into
    ``graph.x`` (or pass them to ``__call__``, which copies them in), replay, read ``graph.out``.
    With ``return_router`` the router outputs land in ``graph.logits``, ``graph.idx``, ``graph.w``
    (tensors of the graph's memory pool, rewritten by every replay).
    Replays on one BlockGraph share its buffers, so they must not overlap each other.
    """

    def __init__(self, weights, k, tokens, logit_bias=None, return_router=False, pool=None):
        w_router, w_gate_up, w_down, w_sh_gate, w_sh_up, w_sh_down, w_sh_gate_proj = weights
        self.weights = tuple(weights)
        self.k = k
        self.logit_bias = logit_bias
        dev = w_router.device
        dt = w_router.dtype
        h = w_router.shape[1]
        E = w_router.shape[0]
        I = w_gate_up.shape[1] // 2
        Is = w_sh_gate.shape[0]
        self.x = torch.zeros(tokens, h, dtype=dt, device=dev)
        self.out = torch.empty(tokens, h, dtype=dt, device=dev)
        self.workspace = torch.empty(ops.block_workspace_bytes(tokens, h, E, k, I, Is, dt), dtype=torch.uint8,
                                     device=dev)
        self.return_router = return_router
        self.logits = self.idx = self.w = None
        # One eager run (argument checks, and the library's per-device state if any) on a side
        # stream, as torch asks before a capture, then the capture itself.
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            self._launch()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=pool):
            self._launch()

    def _launch(self):
        if not self.return_router:
            ops.block_forward(self.x, *self.weights, self.k, logit_bias=self.logit_bias, workspace=self.workspace,
                              out=self.out)
            return
        # The router outputs are allocated by block_forward; allocated during the capture they come
        # from the graph's private pool and keep their addresses for every replay.
        _, self.logits, self.idx, self.w = ops.block_forward(self.x, *self.weights, self.k,
                                                             logit_bias=self.logit_bias, return_router=True,
                                                             workspace=self.workspace, out=self.out)

    def replay(self):
        self.graph.replay()
        return self.out

    def __call__(self, x=None):
        if x is not None:
            if x.shape != self.x.shape or x.dtype != self.x.dtype:
                raise ValueError(f"input must be {tuple(self.x.shape)} {self.x.dtype}, got {tuple(x.shape)} {x.dtype}")
            self.x.copy_(x)
        return self.replay()
