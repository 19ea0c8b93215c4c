"""GPU parity of the permutation (R3-R4): counts, starts and perm bit-exact vs the CPU oracle
(stable counting sort == torch.sort(stable=True), q38/inference.py:163-171) plus tile-table
invariants."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _ops():
    from q38.hip import ops
    return ops


def _check(idx, E, gpu, shared_rows=0):
    ops = _ops()
    T, k = idx.shape
    didx = idx.to(gpu)
    hist = ops.histogram(didx, E)
    counts, starts, perm, inv, tiles, tile_count = ops.permute(didx, hist, E, shared_rows=shared_rows)
    torch.cuda.synchronize()
    rc, rs, rp = orc.permute_cpu(idx.numpy(), E)
    assert np.array_equal(counts.cpu().numpy(), rc)
    assert np.array_equal(starts.cpu().numpy(), rs)
    n = rp.size
    assert np.array_equal(perm.cpu().numpy()[:n], rp)
    # inv is the inverse permutation on the valid pairs.
    inv_np = inv.cpu().numpy()
    assert np.array_equal(inv_np[rp], np.arange(n))
    # Tile table: the BM-row blocks of every expert segment and of the shared rows, full blocks
    # first, then partial ones by falling size (the oracle's order, bit-exact).
    bm = ops.gemm_block_m()
    tl = tiles.cpu().numpy()
    used = tl[tl[:, 0] >= 0]
    assert int(tile_count.item()) == len(used)
    assert (tl[len(used):, 0] == -1).all(), "unused tiles must follow the used ones"
    expect = orc.tile_table(rc, rs, bm, shared_rows, P=T * k)
    assert [tuple(map(int, t[:3])) for t in used] == expect
    return counts, starts, perm


@pytest.mark.parametrize("T,E,k,seed", [(16384, 64, 5, 0), (2048, 64, 5, 1), (53, 8, 3, 2), (1, 64, 5, 3),
                                        (4097, 64, 8, 4), (300, 1, 1, 5)])
def test_permute_random(gpu, T, E, k, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    _check(idx, E, gpu)


def test_permute_int64_and_skew(gpu):
    """int64 indices (torch.topk's dtype) and a ~20x load skew (padding grows per expert only)."""
    rs = np.random.RandomState(3)
    p = 1.0 / np.arange(1, 65) ** 1.2
    p /= p.sum()
    rows = [rs.choice(64, size=5, replace=False, p=p) for _ in range(8192)]
    idx = torch.from_numpy(np.array(rows, dtype=np.int64))
    counts, _, _ = _check(idx, 64, gpu)
    c = counts.cpu().numpy()
    assert c.max() > 10 * max(c.min(), 1)


def test_permute_out_of_range_dropped(gpu):
    """Sentinel ids (>= E or < 0) are dropped, like transformers' grouped_mm (moe.py:405-420)."""
    g = torch.Generator().manual_seed(9)
    idx = torch.randint(-2, 10, (500, 3), generator=g).to(torch.int64)
    _check(idx, 8, gpu)


def test_permute_shared_tiles(gpu):
    """Shared-expert rows appended to the tile table (the fused grouped-GEMM launch)."""
    g = torch.Generator().manual_seed(11)
    idx = torch.randint(0, 64, (3000, 5), generator=g).to(torch.int32)
    _check(idx, 64, gpu, shared_rows=3000)


def test_permute_empty(gpu):
    ops = _ops()
    idx = torch.empty(0, 5, dtype=torch.int32, device=gpu)
    hist = ops.histogram(idx, 64)
    counts, starts, perm, inv, tiles, tile_count = ops.permute(idx, hist, 64)
    torch.cuda.synchronize()
    assert int(counts.sum()) == 0 and int(starts.abs().sum()) == 0
    assert (tiles.cpu()[:, 0] == -1).all() and int(tile_count.item()) == 0


def test_permute_deterministic(gpu):
    g = torch.Generator().manual_seed(12)
    idx = torch.randint(0, 64, (16384, 5), generator=g).to(torch.int32).to(gpu)
    ops = _ops()
    outs = []
    for _ in range(2):
        hist = ops.histogram(idx, 64)
        outs.append([t.cpu() for t in ops.permute(idx, hist, 64)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
