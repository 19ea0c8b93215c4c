"""Packed no-cache prefill of the Q38 model with the HIP MoE block in every layer (benchmark config 5).

This is the caller of the MoE hot path: the Q38 trunk (``Qwen3_8MoeTextModel.trunk`` and ``_layer``,
q38/models/qwen3_8_moe/modeling_qwen3_8_moe.py:1233-1275, plus the tied head of
``Qwen3_8MoeForCausalLM.forward``, :1398-1431) restated for inference on one GPU, with every
``layer.mlp`` a drop-in ``Qwen3_8MoeSparseMoeBlock`` running the fused HIP block. Module and
parameter names follow the reference state dict (``model.layers.{i}.linear_attn.in_proj_qkv.weight``
...), so a reference checkpoint loads with ``load_state_dict``.

Per layer (modeling:1259-1275): mHC pre-mix of the 4-way residual stream (fp32), zero-centred
RMSNorm, the token mixer (Gated DeltaNet, or QSA sparse attention on every 4th layer), mHC post-mix;
then the same around the MoE block; after layer 0 the N-gram embedding adds its gated delta. The
token mixers are torch code on the GPU (hipBLASLt GEMMs); only the MoE runs on this library's
kernels.

Numerics follow the reference op for op where a rounding point is visible (bf16 projections, fp32
mHC stream, fp32 delta-rule state, bf16 gating products). Two restatements differ in form, not in
math: the causal depthwise convolution is an explicit fp32 shift-and-add (modeling:184-205 uses
conv1d), and QSA attention gathers each query block's selected key blocks and runs dense fp32
attention on them, which equals the reference's masked attention over the full sequence
(modeling:1143-1158).
"""
import os
import zlib
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

BLK = 64  # QSA block and packing granularity (modeling:976)


@dataclass(frozen=True)
class PrefillConfig:
    """Model shape (the reference's ``presets.model_config`` fields, q38/presets.py:59-83)."""

    vocab: int = 10112
    hidden: int = 1024
    layers: int = 12
    heads: int = 38
    kv_heads: int = 2
    head_dim: int = 64
    lin_k_heads: int = 13
    lin_v_heads: int = 39
    lin_head_dim: int = 64
    conv_kernel: int = 4
    experts: int = 64
    topk: int = 5
    moe_ffn: int = 256
    shared_ffn: int = 256
    rope_theta: float = 1e7
    partial_rotary: float = 0.25
    n_branch: int = 4
    mhc_iters: int = 20
    qsa_blocks: int = 8
    indexer_heads: int = 4
    indexer_head_dim: int = 64
    ngram_rows: int = 131072
    eos_id: int = 53
    pad_id: int = 53
    rms_eps: float = 1e-6
    layer_types: tuple = ()  # empty: [lin, lin, lin, full] repeating (presets.py:55-56)

    def layer_kind(self, i):
        if self.layer_types:
            return self.layer_types[i]
        return "full_attention" if i % 4 == 3 else "linear_attention"

    @property
    def mhc_rank(self):
        return max(1, round(self.hidden / 8))


def c5_config():
    """Benchmark config 5: 12 layers at hidden 1024 with the dimension rule of
    scripts/make_q38_configs.py:81-89 (heads 2*round(1.2 h/64), 13 key / 39 value DeltaNet heads,
    expert width h/4), 64 experts top-5 + shared, vocab 10112, EOS id 53."""
    return PrefillConfig()


# ---- parameters -------------------------------------------------------------------------------

def param_specs(cfg):
    """Ordered {name: (shape, init)} of every parameter, under the reference state-dict names.

    init is ("normal", mean, std), ("uniform_log", lo, hi), ("pre_logit", slot) or
    ("res_bias",). The distributions follow the reference's initialisation (modeling:944-960,
    1036-1043, 1169-1177), except that parameters it starts at a constant that would hide a code
    path (zero-centred norm weights, the mHC B projection) get a small random spread.
    """
    c = cfg
    h, n = c.hidden, c.n_branch
    W = ("normal", 0.0, 0.02)
    NORM0 = ("normal", 0.0, 0.05)  # zero-centred RMSNorm: y = x_hat * (1 + w)
    specs = {"model.embed_tokens.weight": ((c.vocab, h), W)}
    kd, vd = c.lin_k_heads * c.lin_head_dim, c.lin_v_heads * c.lin_head_dim
    for i in range(c.layers):
        p = f"model.layers.{i}."
        specs[p + "input_layernorm.weight"] = ((h,), NORM0)
        specs[p + "post_attention_layernorm.weight"] = ((h,), NORM0)
        if c.layer_kind(i) == "linear_attention":
            a = p + "linear_attn."
            specs[a + "in_proj_qkv.weight"] = ((2 * kd + vd, h), W)
            specs[a + "in_proj_z.weight"] = ((vd, h), W)
            specs[a + "in_proj_b.weight"] = ((c.lin_v_heads, h), W)
            specs[a + "in_proj_a.weight"] = ((c.lin_v_heads, h), W)
            specs[a + "conv1d.weight"] = ((2 * kd + vd, 1, c.conv_kernel), ("normal", 0.0, 0.3))
            specs[a + "dt_bias"] = ((c.lin_v_heads,), ("normal", 1.0, 0.1))
            specs[a + "A_log"] = ((c.lin_v_heads,), ("uniform_log", 0.01, 16.0))
            specs[a + "norm.weight"] = ((c.lin_head_dim,), ("normal", 1.0, 0.05))
            specs[a + "out_proj.weight"] = ((h, vd), W)
        else:
            a = p + "self_attn."
            specs[a + "q_proj.weight"] = ((c.heads * c.head_dim * 2, h), W)
            specs[a + "k_proj.weight"] = ((c.kv_heads * c.head_dim, h), W)
            specs[a + "v_proj.weight"] = ((c.kv_heads * c.head_dim, h), W)
            specs[a + "o_proj.weight"] = ((h, c.heads * c.head_dim), W)
            specs[a + "q_norm.weight"] = ((c.head_dim,), NORM0)
            specs[a + "k_norm.weight"] = ((c.head_dim,), NORM0)
        m = p + "mlp."
        specs[m + "gate.weight"] = ((c.experts, h), W)
        specs[m + "experts.gate_up_proj"] = ((c.experts, 2 * c.moe_ffn, h), W)
        specs[m + "experts.down_proj"] = ((c.experts, h, c.moe_ffn), W)
        specs[m + "shared_expert.gate_proj.weight"] = ((c.shared_ffn, h), W)
        specs[m + "shared_expert.up_proj.weight"] = ((c.shared_ffn, h), W)
        specs[m + "shared_expert.down_proj.weight"] = ((h, c.shared_ffn), W)
        specs[m + "shared_expert_gate.weight"] = ((1, h), W)
    specs["model.norm.weight"] = ((h,), NORM0)
    for j in range(2 * c.layers):
        p = f"model.mhc.{j}."
        specs[p + "A.weight"] = ((c.mhc_rank, n * h), W)
        specs[p + "B.weight"] = ((2 * n + n * n, c.mhc_rank), W)
        specs[p + "b_pre"] = ((n,), ("pre_logit", j % n))
        specs[p + "b_post"] = ((n,), ("normal", 0.0, 0.0))
        specs[p + "b_res"] = ((n, n), ("res_bias",))
        specs[p + "alphas"] = ((3,), ("normal", 0.1, 0.0))
    for i in range(c.layers):
        if c.layer_kind(i) == "full_attention":
            p = f"model.indexers.{i}."
            specs[p + "wq.weight"] = ((c.indexer_heads * c.indexer_head_dim, h), W)
            specs[p + "wk.weight"] = ((c.indexer_head_dim, h), W)
            specs[p + "ww.weight"] = ((c.indexer_heads, h), W)
    if c.ngram_rows:
        specs["model.ngram.emb2.weight"] = ((c.ngram_rows, h), W)
        specs["model.ngram.emb3.weight"] = ((c.ngram_rows, h), W)
        specs["model.ngram.norm.weight"] = ((h,), ("normal", 0.02, 0.002))
        specs["model.ngram.gate.weight"] = ((h, h), W)
        specs["model.ngram.gate.bias"] = ((h,), ("normal", -1.0, 0.0))
    return specs


def _draw(name, shape, init, seed):
    rng = np.random.Generator(np.random.PCG64([seed, zlib.crc32(name.encode())]))
    kind = init[0]
    if kind == "normal":
        a = rng.standard_normal(shape, dtype=np.float32)
        a *= np.float32(init[2])
        a += np.float32(init[1])
    elif kind == "uniform_log":
        a = np.log(rng.uniform(init[1], init[2], shape)).astype(np.float32)
    elif kind == "pre_logit":  # H_pre starts at 0.7 on the branch this sublayer reads, 0.1 elsewhere
        pre = np.full(shape, 0.1, dtype=np.float32)
        pre[init[1]] = 0.7
        a = np.log(pre / (1 - pre)).astype(np.float32)
    elif kind == "res_bias":  # H_res near the identity after Sinkhorn: 0 on, -8 off the diagonal
        a = (np.full(shape, -8.0) + 8.0 * np.eye(shape[0])).astype(np.float32)
    else:
        raise ValueError(kind)
    return torch.from_numpy(a)


def init_params(cfg, seed=0, threads=None):
    """Seeded fp32 parameters {name: tensor} (CPU), plus ``lm_head.weight`` tied to the embedding.

    Each parameter has its own stream, numpy PCG64 seeded with (seed, crc32(name)), so any subset
    can be regenerated independently and the values do not depend on traversal order or on the
    thread pool that draws them.
    """
    specs = param_specs(cfg)
    workers = threads or min(16, os.cpu_count() or 1)
    with ThreadPoolExecutor(workers) as pool:  # numpy's generators release the GIL
        arrays = pool.map(lambda kv: _draw(kv[0], kv[1][0], kv[1][1], seed), specs.items())
        out = dict(zip(specs.keys(), arrays))
    out["lm_head.weight"] = out["model.embed_tokens.weight"]
    return out


def make_ids(batch, seq, cfg, seed=1234, eos_every=1000):
    """Packed synthetic input: ids uniform in [0, vocab) with an EOS about every ``eos_every``
    tokens (numpy RandomState(seed): uniform draws, then EOS at jittered spacing)."""
    rng = np.random.RandomState(seed)
    ids = rng.randint(0, cfg.vocab, size=(batch, seq)).astype(np.int64)
    for b in range(batch):
        pos = int(rng.randint(0, eos_every))
        while pos < seq:
            ids[b, pos] = cfg.eos_id
            pos += int(rng.randint(eos_every // 2, 3 * eos_every // 2 + 1))
    return torch.from_numpy(ids)


# ---- modules (parameter holders under the reference names) -------------------------------------

class _Norm(nn.Module):
    def __init__(self, dim, init=0.0):
        super().__init__()
        self.init_value = init  # 0 for the zero-centred norms, 1 for the gated norm
        self.weight = nn.Parameter(torch.zeros(dim))


def _linear(i, o, bias=False):
    return nn.Linear(i, o, bias=bias)


class _DeltaNet(nn.Module):
    def __init__(self, c):
        super().__init__()
        kd, vd = c.lin_k_heads * c.lin_head_dim, c.lin_v_heads * c.lin_head_dim
        conv = 2 * kd + vd
        self.in_proj_qkv = _linear(c.hidden, conv)
        self.in_proj_z = _linear(c.hidden, vd)
        self.in_proj_b = _linear(c.hidden, c.lin_v_heads)
        self.in_proj_a = _linear(c.hidden, c.lin_v_heads)
        self.conv1d = nn.Conv1d(conv, conv, c.conv_kernel, groups=conv, bias=False)
        self.dt_bias = nn.Parameter(torch.ones(c.lin_v_heads))
        self.A_log = nn.Parameter(torch.zeros(c.lin_v_heads))
        self.norm = _Norm(c.lin_head_dim, init=1.0)
        self.out_proj = _linear(vd, c.hidden)


class _Attention(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.q_proj = _linear(c.hidden, c.heads * c.head_dim * 2)
        self.k_proj = _linear(c.hidden, c.kv_heads * c.head_dim)
        self.v_proj = _linear(c.hidden, c.kv_heads * c.head_dim)
        self.o_proj = _linear(c.heads * c.head_dim, c.hidden)
        self.q_norm = _Norm(c.head_dim)
        self.k_norm = _Norm(c.head_dim)


class _Indexer(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.wq = _linear(c.hidden, c.indexer_heads * c.indexer_head_dim)
        self.wk = _linear(c.hidden, c.indexer_head_dim)
        self.ww = _linear(c.hidden, c.indexer_heads)


class _MHC(nn.Module):
    def __init__(self, c, slot=0):
        super().__init__()
        n = c.n_branch
        self.slot = slot  # the branch this sublayer mainly reads (H_pre initialisation)
        self.A = _linear(n * c.hidden, c.mhc_rank)
        self.B = _linear(c.mhc_rank, 2 * n + n * n)
        self.b_pre = nn.Parameter(torch.zeros(n))
        self.b_post = nn.Parameter(torch.zeros(n))
        self.b_res = nn.Parameter(torch.zeros(n, n))
        self.alphas = nn.Parameter(torch.zeros(3))


class _NGram(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.emb2 = nn.Embedding(c.ngram_rows, c.hidden)
        self.emb3 = nn.Embedding(c.ngram_rows, c.hidden)
        self.norm = nn.RMSNorm(c.hidden, eps=1e-6)
        self.gate = _linear(c.hidden, c.hidden, bias=True)


class _MoeConfig:
    """The fields the drop-in MoE modules read from a transformers config."""

    def __init__(self, c):
        self.hidden_size = c.hidden
        self.num_experts = c.experts
        self.num_experts_per_tok = c.topk
        self.moe_intermediate_size = c.moe_ffn
        self.shared_expert_intermediate_size = c.shared_ffn
        self.hidden_act = "silu"


class _Layer(nn.Module):
    def __init__(self, c, i):
        super().__init__()
        from .models.qwen3_8_moe.modeling_qwen3_8_moe import Qwen3_8MoeSparseMoeBlock

        self.kind = c.layer_kind(i)
        if self.kind == "linear_attention":
            self.linear_attn = _DeltaNet(c)
        else:
            self.self_attn = _Attention(c)
        self.mlp = Qwen3_8MoeSparseMoeBlock(_MoeConfig(c))
        self.input_layernorm = _Norm(c.hidden)
        self.post_attention_layernorm = _Norm(c.hidden)


class _Trunk(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.embed_tokens = nn.Embedding(c.vocab, c.hidden)
        self.layers = nn.ModuleList([_Layer(c, i) for i in range(c.layers)])
        self.norm = _Norm(c.hidden)
        self.mhc = nn.ModuleList([_MHC(c, j) for j in range(2 * c.layers)])
        self.indexers = nn.ModuleDict({str(i): _Indexer(c) for i in range(c.layers)
                                       if c.layer_kind(i) == "full_attention"})
        self.ngram = _NGram(c) if c.ngram_rows else None


# ---- the forward pass -------------------------------------------------------------------------

def _zc_norm(x, w, eps):
    """Zero-centred RMSNorm (modeling:839-853): fp32 normalise, scale by (1 + w), back to x.dtype."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (y * (1.0 + w.float())).to(x.dtype)


def _gated_norm(x, z, w, eps):
    """RMSNormGated (modeling:132-148): normalise in fp32, round to x.dtype, times w in the weight
    dtype, times silu(z) in fp32, back to x.dtype."""
    xf = x.float()
    y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    y = w * y
    return (y * F.silu(z.float())).to(x.dtype)


def rope_tables(cfg, S, dtype, device):
    """cos/sin [S, rot] of the partial rotary embedding (modeling:63-129). The three mRoPE position
    rows are equal for text, so the section recomposition leaves the table unchanged. Computed on
    the CPU in fp32 from an fp32 inverse-frequency table, then cast."""
    dim = int(cfg.head_dim * cfg.partial_rotary)
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    f = torch.arange(S, dtype=torch.float32)[:, None] * inv[None, :]
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().to(device=device, dtype=dtype), emb.sin().to(device=device, dtype=dtype)


def _rotate(x, cos, sin):
    """Rotary embedding on the first cos.shape[-1] features of x [..., S, d] (modeling:580-623)."""
    r = cos.shape[-1]
    xr, xp = x[..., :r], x[..., r:]
    half = r // 2
    turned = torch.cat([-xr[..., half:], xr[..., :half]], dim=-1)
    return torch.cat([xr * cos + turned * sin, xp], dim=-1)


def prefix_sum(g):
    """Inclusive prefix sums along the last dimension (torch.cumsum(g, -1)) in a fixed order: log-step
    doubling, elementwise adds in float64, rounded once to g's dtype. torch documents its GPU cumsum
    of floating-point tensors as non-deterministic; this has no reduction whose order can vary. The
    reference's CPU cumsum of float32 also accumulates in float64 (left to right)."""
    c = g.double()
    s = 1
    while s < c.shape[-1]:
        c = torch.cat([c[..., :s], c[..., s:] + c[..., :-s]], dim=-1)
        s *= 2
    return c.to(g.dtype)


def gated_delta_rule(q, k, v, g, beta, chunk=64):
    """Gated delta rule over a sequence (modeling:215-349 defines it; 352-413 is the token recurrence).

    q, k [B,S,H,dk], v [B,S,H,dv], g [B,S,H] fp32 log-decays (<= 0), beta [B,S,H]. Per token:
    state S <- e^{g_t} S; d_t = beta_t (v_t - S^T k_t); S <- S + k_t d_t^T; o_t = S^T q_t, with q, k
    L2-normalised and q scaled by dk^-1/2. Evaluated chunkwise: inside a chunk with cumulative decay
    c_t the updates satisfy (I + A) D = beta*V - diag(beta e^{c}) K S0, A[t,j] = beta_t e^{c_t-c_j}
    k_t.k_j (j < t), so D comes from two unit-lower-triangular solves and the chunk's outputs and
    final state from matrix products; only the chunk-to-chunk state is sequential. fp32 throughout;
    returns [B,S,H,dv] in q.dtype.
    """
    out_dtype = q.dtype
    q, k, v, beta, g = (t.transpose(1, 2).float() for t in (q, k, v, beta, g))
    q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6)
    k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    q = q * (q.shape[-1] ** -0.5)
    B, H, S, dk = k.shape
    dv = v.shape[-1]
    pad = (-S) % chunk
    if pad:
        q, k, v = (F.pad(t, (0, 0, 0, pad)) for t in (q, k, v))
        beta, g = (F.pad(t, (0, pad)) for t in (beta, g))
    n = (S + pad) // chunk
    q, k, v = (t.reshape(B, H, n, chunk, -1) for t in (q, k, v))
    beta = beta.reshape(B, H, n, chunk)
    c = prefix_sum(g.reshape(B, H, n, chunk))
    lower = torch.ones(chunk, chunk, dtype=torch.bool, device=q.device).tril()
    decay = torch.where(lower, c[..., :, None] - c[..., None, :], torch.full((), float("-inf"),
                                                                              device=q.device)).exp()
    kb = k * beta[..., None]
    system = (kb @ k.transpose(-1, -2)) * decay  # its diagonal is ignored: unit-triangular solve
    # One solve for both right-hand sides: D = d_v - d_k S0.
    rhs = torch.cat([v * beta[..., None], kb * c.exp()[..., None]], dim=-1)
    sol = torch.linalg.solve_triangular(system, rhs, upper=False, unitriangular=True)
    d_v, d_k = sol[..., :dv], sol[..., dv:]
    intra = (q @ k.transpose(-1, -2)) * decay
    q_read = q * c.exp()[..., None]
    k_write = k * (c[..., -1:] - c).exp()[..., None]
    carry = c[..., -1].exp()[..., None, None]
    state = q.new_zeros(B, H, dk, dv)
    out = q.new_empty(B, H, n, chunk, dv)
    for i in range(n):
        d = d_v[:, :, i] - d_k[:, :, i] @ state
        out[:, :, i] = q_read[:, :, i] @ state + intra[:, :, i] @ d
        state = state * carry[:, :, i] + k_write[:, :, i].transpose(-1, -2) @ d
    out = out.reshape(B, H, n * chunk, dv)[:, :, :S]
    return out.transpose(1, 2).to(out_dtype)


def _delta_net(m, x, cfg):
    """Qwen3_8MoeGatedDeltaNet.forward without cache (modeling:464-577)."""
    B, S, _ = x.shape
    nk, nv, d = cfg.lin_k_heads, cfg.lin_v_heads, cfg.lin_head_dim
    qkv = F.linear(x, m.in_proj_qkv.weight)
    # Causal depthwise convolution (kernel K, left zero padding) in fp32, then SiLU in x.dtype.
    w = m.conv1d.weight[:, 0, :].float()
    K = w.shape[1]
    xp = F.pad(qkv.transpose(1, 2).float(), (K - 1, 0))
    acc = xp[:, :, 0:S] * w[:, 0:1]
    for j in range(1, K):
        acc = acc + xp[:, :, j:j + S] * w[:, j:j + 1]
    qkv = F.silu(acc.to(x.dtype)).transpose(1, 2)
    q, k, v = torch.split(qkv, [nk * d, nk * d, nv * d], dim=-1)
    q = q.reshape(B, S, nk, d)
    k = k.reshape(B, S, nk, d)
    v = v.reshape(B, S, nv, d)
    z = F.linear(x, m.in_proj_z.weight).reshape(B, S, nv, d)
    beta = torch.sigmoid(F.linear(x, m.in_proj_b.weight))
    g = -m.A_log.float().exp() * F.softplus(F.linear(x, m.in_proj_a.weight).float() + m.dt_bias)
    if nv // nk > 1:
        q = q.repeat_interleave(nv // nk, dim=2)
        k = k.repeat_interleave(nv // nk, dim=2)
    o = gated_delta_rule(q, k, v, g, beta)
    o = _gated_norm(o.reshape(-1, d), z.reshape(-1, d), m.norm.weight, cfg.rms_eps)
    return F.linear(o.reshape(B, S, nv * d), m.out_proj.weight)


def select_blocks(lp_blk, budget):
    """Key blocks each query block attends to (modeling:1099-1114): by the indexer's block
    probabilities at the block's first query, the current block always, future blocks never.
    Returns (sel [B,nb,k] block ids, valid [nb,k]: slot j < min(qb + 1, k))."""
    B, nq, nb = lp_blk.shape
    k = min(budget, nb)
    p = lp_blk.exp()
    qb = torch.arange(nq, device=p.device)[:, None]
    kb = torch.arange(nb, device=p.device)[None, :]
    p = torch.where(kb > qb, torch.full_like(p, -1.0), p)
    p = torch.where(kb == qb, torch.full_like(p, 2.0), p)
    sel = p.topk(k, dim=-1).indices
    valid = torch.arange(k, device=p.device)[None, :] < torch.clamp(qb + 1, max=k)
    return sel, valid


def _qsa(m, ix, x, cos, sin, cfg):
    """qsa_attention for inference (modeling:1117-1165, dense=False, no KL): lightning-indexer block
    selection at block starts, then attention over the selected 64-token blocks."""
    B, S, _ = x.shape
    H, KV, hd = cfg.heads, cfg.kv_heads, cfg.head_dim
    nb = S // BLK
    qg = F.linear(x, m.q_proj.weight).view(B, S, H, 2 * hd)
    q, gate = qg[..., :hd], qg[..., hd:].reshape(B, S, H * hd)
    q = _zc_norm(q, m.q_norm.weight, cfg.rms_eps).transpose(1, 2)
    k = _zc_norm(F.linear(x, m.k_proj.weight).view(B, S, KV, hd), m.k_norm.weight, cfg.rms_eps).transpose(1, 2)
    v = F.linear(x, m.v_proj.weight).view(B, S, KV, hd).transpose(1, 2)
    q = _rotate(q, cos, sin)
    k = _rotate(k, cos, sin)

    # Indexer (modeling:1065-1081): I[t, s] = sum_j w_j(t) relu(q_j(t).k(s)) / sqrt(d) at block starts.
    nih, dih = cfg.indexer_heads, cfg.indexer_head_dim
    iq = _rotate(F.linear(x, ix.wq.weight).view(B, S, nih, dih).transpose(1, 2), cos, sin)[:, :, ::BLK]
    ik = _rotate(F.linear(x, ix.wk.weight).view(B, S, 1, dih).transpose(1, 2), cos, sin)
    iw = (F.linear(x, ix.ww.weight).float() * nih ** -0.5)[:, ::BLK]
    s = torch.matmul(iq, ik.transpose(-1, -2).contiguous())  # bf16 batched product: no transposed view
    score = (F.relu(s.float()) * dih ** -0.5 * iw.transpose(1, 2)[..., None]).sum(1)  # [B, nb, S]
    keys = torch.arange(S, device=x.device)
    starts = torch.arange(0, S, BLK, device=x.device)
    score = score.masked_fill(keys[None, :] > starts[:, None], -1e9)
    lp = torch.log_softmax(score, dim=-1)
    lp_blk = torch.logsumexp(lp.view(B, nb, nb, BLK), dim=-1)
    sel, valid = select_blocks(lp_blk, cfg.qsa_blocks)
    o = block_sparse_attention(q, k, v, sel, valid, hd ** -0.5)
    o = o.transpose(1, 2).reshape(B, S, H * hd) * torch.sigmoid(gate)
    return F.linear(o, m.o_proj.weight)


def block_sparse_attention(q, k, v, sel, valid, scale):
    """Causal attention of each 64-query block over its selected key blocks.

    q [B,H,S,d], k/v [B,KV,S,d] (query head h reads kv head h // (H/KV)), sel [B,nb,kk] key-block
    ids per query block, valid [nb,kk] which slots count. Equals attention over the full sequence
    with the mask "key block selected and key position <= query position" (modeling:1143-1158):
    each query block gathers its kk key blocks and runs dense attention on them, fp32 scores,
    softmax and accumulation. Returns [B,H,S,d] in q.dtype.
    """
    B, H, S, d = q.shape
    KV = k.shape[1]
    nb, kk = S // BLK, sel.shape[-1]

    def gather(t):
        blocks = t.reshape(B, KV, nb, BLK * d)
        idx = sel.reshape(B, 1, nb * kk, 1).expand(B, KV, nb * kk, BLK * d)
        return torch.gather(blocks, 2, idx).view(B, KV, 1, nb, kk * BLK, d).float()

    ks, vs = gather(k), gather(v)
    qf = q.reshape(B, KV, H // KV, nb, BLK, d).float()
    scores = torch.matmul(qf, ks.transpose(-1, -2)) * scale  # [B, KV, G, nb, BLK, kk*BLK]
    ar = torch.arange(BLK, device=q.device)
    key_pos = (sel[..., None] * BLK + ar).reshape(B, nb, 1, kk * BLK)
    q_pos = (torch.arange(nb, device=q.device)[:, None] * BLK + ar[None, :]).reshape(1, nb, BLK, 1)
    slot_ok = valid[:, :, None].expand(nb, kk, BLK).reshape(1, nb, 1, kk * BLK)
    allowed = slot_ok & (key_pos <= q_pos)  # [B, nb, BLK, kk*BLK]
    scores = scores.masked_fill(~allowed[:, None, None], float("-inf"))
    o = torch.matmul(torch.softmax(scores, dim=-1), vs).to(q.dtype)
    return o.reshape(B, H, S, d)


def _mhc_pre(m, X, cfg):
    """mHC coefficients and the sublayer input (modeling:994-1031): X [B,S,n,h] fp32."""
    n = cfg.n_branch
    Xf = X.flatten(2)
    Xf = Xf * torch.rsqrt(Xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    z = torch.tanh(F.linear(F.linear(Xf, m.A.weight.float()), m.B.weight.float()))
    al = m.alphas.float()
    pre = torch.sigmoid(m.b_pre.float() + al[0] * z[..., :n])
    post = 2 * torch.sigmoid(m.b_post.float() + al[1] * z[..., n:2 * n])
    logits = m.b_res.float() + al[2] * z[..., 2 * n:].reshape(*z.shape[:-1], n, n)
    P = torch.exp(logits - logits.amax(dim=(-2, -1), keepdim=True))
    for _ in range(cfg.mhc_iters):  # Sinkhorn normalisation towards a doubly stochastic H_res
        P = P / P.sum(-1, keepdim=True).clamp(min=1e-9)
        P = P / P.sum(-2, keepdim=True).clamp(min=1e-9)
    return (pre.unsqueeze(-1) * X).sum(2), (post, P)


def _mhc_post(X, y, state):
    """X' = H_res X + H_post^T y (modeling:1014-1018)."""
    post, P = state
    return torch.matmul(P, X) + post.unsqueeze(-1) * y.float().unsqueeze(2)


_P2 = (1000003, 998244353)
_P3 = (1000033, 998244353, 1000000007)
_MIX = 2654435761


def ngram_indices(ids, cfg):
    """Hashed bigram / trigram rows of each position (modeling:1182-1194): the previous tokens of
    the same document (reset after EOS; the vocab size stands for "none"), int64 wrap-around."""
    B, T = ids.shape
    V = cfg.vocab
    pos = torch.arange(T, device=ids.device).expand(B, T)
    last = torch.cummax(torch.where(ids == cfg.eos_id, pos, torch.full_like(pos, -1)), dim=1).values.clamp(min=0)

    def prev(j):
        xs = torch.cat([torch.full((B, j), V, device=ids.device, dtype=ids.dtype), ids[:, :-j]], dim=1)
        return torch.where((pos - j) >= last, xs, torch.full_like(xs, V))

    a, b, c = prev(1), ids, prev(2)
    i2 = (a * _P2[0]) ^ (b * _P2[1])
    i3 = (c * _P3[0]) ^ (a * _P3[1]) ^ (b * _P3[2])
    i2 = (i2 ^ (i2 >> 17)) * _MIX
    i3 = (i3 ^ (i3 >> 17)) * _MIX
    return i2 % cfg.ngram_rows, i3 % cfg.ngram_rows


def _ngram_delta(m, h, ids, cfg):
    """NGramEmbedding.delta (modeling:1196-1207): (h + sigmoid(gate(h)) * e) - h in h.dtype."""
    i2, i3 = ngram_indices(ids, cfg)
    e = F.rms_norm(F.embedding(i2, m.emb2.weight) + F.embedding(i3, m.emb3.weight), (cfg.hidden,),
                   m.norm.weight, 1e-6).to(h.dtype)
    g = torch.sigmoid(F.linear(h, m.gate.weight, m.gate.bias))
    return (h + g * e) - h


def _moe_default(block, x):
    return block(x)


def load_balancing_loss(router_logits, num_experts, top_k):
    """load_balancing_loss_func without an attention mask (modeling:1289-1355), the Switch
    Transformer auxiliary loss: per layer, softmax of the logits (in their dtype), the top-k set,
    per-expert assignment counts and probability sums; then E * sum_e (counts_e / rows) *
    (prob_sum_e / rows) over all layers' rows. On the GPU the top-k set comes from torch's GPU
    top-k: a tie at the k-th rank may resolve to the other expert than on the CPU."""
    dev = router_logits[0].device
    counts = torch.zeros(num_experts, dtype=torch.float32, device=dev)
    probs = torch.zeros(num_experts, dtype=torch.float32, device=dev)
    rows = 0
    for lg in router_logits:
        p = torch.softmax(lg, dim=-1)
        chosen = torch.topk(p, top_k, dim=-1).indices
        counts = counts + torch.bincount(chosen.reshape(-1), minlength=num_experts).float()
        probs = probs + p.float().sum(dim=0)
        rows += p.shape[0]
    return torch.sum((counts / rows) * (probs / rows)) * num_experts


@dataclass
class PrefillOutput:
    """The fields of MoeCausalLMOutputWithPast the packed prefill fills (modeling:1425-1433)."""

    logits: torch.Tensor
    aux_loss: Optional[torch.Tensor] = None
    router_logits: Optional[Tuple[torch.Tensor, ...]] = None


class Q38Prefill(nn.Module):
    """Qwen3_8MoeForCausalLM's packed no-cache prefill (modeling:1233-1275, 1398-1431): ids [B,S]
    -> logits [B,S,vocab] in the parameter dtype. Forward-only; the MoE blocks run the fused HIP
    block. ``moe_forward(block, x[B,S,h]) -> [B,S,h]`` replaces the MoE call (tests use it to put
    the CPU oracle in place of the kernels). With ``output_router_logits`` the forward returns a
    PrefillOutput with every layer's router logits [B*S, E] (the fused block's own) and the
    load-balancing loss over them (modeling:1410-1427)."""

    def __init__(self, cfg, moe_forward=None):
        super().__init__()
        self.cfg = cfg
        with torch.device("meta"):  # storage comes from load_params
            self.model = _Trunk(cfg)
        self.moe_forward = moe_forward or _moe_default

    def load_params(self, params):
        """Take {name: tensor} as the parameters (reference state-dict names, all present;
        ``lm_head.weight``, if given, must equal the embedding: the head is tied)."""
        params = dict(params)
        head = params.pop("lm_head.weight", None)
        if head is not None and not torch.equal(head, params["model.embed_tokens.weight"]):
            raise ValueError("lm_head.weight must equal model.embed_tokens.weight (tied head)")
        self.load_state_dict(params, strict=True, assign=True)
        self.requires_grad_(False)
        return self

    def _moe_with_router(self, block, x):
        if self.moe_forward is _moe_default:
            from .inference import hip_moe_block_forward_with_router

            return hip_moe_block_forward_with_router(block, x)
        return self.moe_forward(block, x), F.linear(x.reshape(-1, x.shape[-1]), block.gate.weight)

    @torch.no_grad()
    def forward(self, ids, output_router_logits=False):
        router = [] if output_router_logits else None
        hs = trunk_forward(self.model, self.cfg, ids, self._moe, router)
        logits = F.linear(hs, self.model.embed_tokens.weight)
        if router is None:
            return logits
        return PrefillOutput(logits, load_balancing_loss(router, self.cfg.experts, self.cfg.topk), tuple(router))

    def _moe(self, block, x, with_router):
        if not with_router:
            return self.moe_forward(block, x)
        return self._moe_with_router(block, x)


def trunk_forward(M, cfg, ids, moe, router=None):
    """Qwen3_8MoeTextModel.trunk + final norm (modeling:1233-1287) over the modules of _Trunk M:
    ids [B, S] -> normed hidden states [B, S, h] in the parameter dtype. ``moe(block, x, r)`` runs
    one MoE block, returning (y, router logits) when r is true; with a ``router`` list the logits
    of every layer are appended to it."""
    B, length = ids.shape
    if length == 0:
        raise ValueError("Q38 prefill needs at least one token")
    pad = (-length) % BLK  # right padding to whole blocks (modeling:1236-1239)
    if pad:
        ids = F.pad(ids, (0, pad), value=cfg.pad_id)
    S = ids.shape[1]
    dt = M.embed_tokens.weight.dtype
    e = F.embedding(ids, M.embed_tokens.weight)
    cos, sin = rope_tables(cfg, S, dt, ids.device)
    X = e.float().unsqueeze(2).expand(-1, -1, cfg.n_branch, -1).contiguous()
    for i, layer in enumerate(M.layers):
        xin, st = _mhc_pre(M.mhc[2 * i], X, cfg)
        x = _zc_norm(xin, layer.input_layernorm.weight, cfg.rms_eps).to(dt)
        if layer.kind == "linear_attention":
            y = _delta_net(layer.linear_attn, x, cfg)
        else:
            y = _qsa(layer.self_attn, M.indexers[str(i)], x, cos, sin, cfg)
        X = _mhc_post(X, y, st)
        xin, st = _mhc_pre(M.mhc[2 * i + 1], X, cfg)
        x = _zc_norm(xin, layer.post_attention_layernorm.weight, cfg.rms_eps).to(dt)
        if router is None:
            y = moe(layer.mlp, x, False)
        else:
            y, lg = moe(layer.mlp, x, True)
            router.append(lg)
        X = _mhc_post(X, y, st)
        if i == 0 and M.ngram is not None:
            X = X + _ngram_delta(M.ngram, X.mean(2).to(dt), ids, cfg).unsqueeze(2)
    return _zc_norm(X.sum(2)[:, :length].to(dt), M.norm.weight, cfg.rms_eps)


def build(cfg=None, seed=0, device="cuda", dtype=torch.bfloat16, moe_forward=None):
    """A seeded random-init prefill model on ``device`` in ``dtype``."""
    cfg = cfg or c5_config()
    model = Q38Prefill(cfg, moe_forward=moe_forward).load_params(init_params(cfg, seed))
    return model.to(device=device, dtype=dtype)
