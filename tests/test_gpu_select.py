"""GPU parity of pool/protect/top-k/sort (select) and of the gather kernels.

Bars: selected indices bit-exact against the oracle's deterministic rule
(lowest index first among values equal to the threshold) on identical score
inputs; pooled values bit-exact; gathered K/V bit-exact against torch.gather.
"""

import pytest
import torch

from oracle import dropkv_ref as R

pytestmark = pytest.mark.gpu


def _select_case(gpu, scores, ks, window, keep):
    from dropkv_amd import ops
    idx, pooled = ops.select(scores.to(gpu), ks, window, keep, return_pooled=True)
    ref_pooled = R.pool_protect(scores.clone(), ks, window)
    ref_idx = R.topk_sorted(ref_pooled, keep)
    assert torch.equal(pooled.cpu(), ref_pooled)
    assert torch.equal(idx.cpu(), ref_idx)


@pytest.mark.parametrize("rows,Lk,keep", [(8, 32768, 3276), (2, 512, 51), (3, 100, 30), (1, 8, 8),
                                          (4, 1000, 1), (2, 70000, 7000), (1, 4096, 4096),
                                          (1, 32769, 3277), (2, 32767, 5000), (1, 40000, 1)])
def test_select_random(gpu, rows, Lk, keep):
    g = torch.Generator().manual_seed(Lk + keep)
    scores = torch.rand(1, rows, Lk, generator=g) * 1e-3
    _select_case(gpu, scores, 11, 8, keep)


@pytest.mark.parametrize("rows,Lk,ks,keep", [(2, 5000, 131, 500), (3, 3000, 1001, 300), (1, 700, 4095, 70),
                                             (2, 40000, 257, 4000), (1, 2000, 131, 2000)])
def test_select_wide_kernels(gpu, rows, Lk, ks, keep):
    """Pooling windows wider than 129 keys (block prefix / suffix maxima,
    any odd kernel size as the reference takes, dropkv_cache.py:327-328):
    pooled values and the lowest-index tie rule bit-exact, including a window
    wider than the row (every key pools to the row maximum) and wide
    plateaus tied at the threshold."""
    g = torch.Generator().manual_seed(ks + Lk)
    scores = torch.rand(1, rows, Lk, generator=g)
    _select_case(gpu, scores, ks, 8, keep)


def test_select_ties_and_plateaus(gpu):
    """Integer-valued scores: pooling makes long plateaus, so the threshold
    is tied many times over; the lowest indices must win."""
    g = torch.Generator().manual_seed(1)
    scores = torch.randint(0, 50, (1, 4, 20000), generator=g).float()
    _select_case(gpu, scores, 11, 8, 2000)
    _select_case(gpu, scores, 1, 8, 5000)
    _select_case(gpu, torch.zeros(1, 2, 3000), 11, 8, 300)


def test_select_threshold_bin_beyond_lds(gpu):
    """More than 4096 keys share the threshold's top-digit bin (here: the
    threshold's exact value), so the threshold stage resolves its digits by
    sweeping the row instead of from its LDS candidate list; the lowest
    indices among the tied keys must still win, across chunks and sweep
    rounds."""
    g = torch.Generator().manual_seed(2)
    scores = torch.randint(0, 3, (1, 3, 40000), generator=g).float()
    _select_case(gpu, scores, 1, 8, 15000)
    _select_case(gpu, scores, 11, 8, 39000)
    near = 1.0 + torch.randint(0, 2048, (1, 2, 70000), generator=g).float() * 2.0 ** -20  # one top-digit bin
    _select_case(gpu, near, 1, 8, 9000)
    _select_case(gpu, near, 11, 8, 30000)


def test_select_big_absorbed(gpu):
    """max >= 2^24: max + 1.0f == max, the protected tail ties with the maximum
    (dropkv_cache.py:465-467 semantics in fp32)."""
    scores = torch.zeros(1, 1, 512)
    scores[0, 0, 100] = 2.0 ** 25
    scores[0, 0, 300] = 2.0 ** 25
    _select_case(gpu, scores, 11, 8, 20)
    _select_case(gpu, scores, 11, 8, 8)


def test_select_window_bigger_than_keep_floor(gpu):
    g = torch.Generator().manual_seed(3)
    scores = torch.rand(1, 2, 300, generator=g)
    _select_case(gpu, scores, 3, 32, 32)
    _select_case(gpu, scores, 11, 0, 40)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_compact_bit_exact(gpu, dtype):
    from dropkv_amd import ops
    g = torch.Generator().manual_seed(0)
    B, H, L, D, keep = 2, 3, 777, 128, 100
    K = torch.randn(B, H, L, D, generator=g).to(dtype)
    V = torch.randn(B, H, L, D, generator=g).to(dtype)
    idx = torch.sort(torch.stack([torch.randperm(L, generator=g)[:keep] for _ in range(B * H)]).view(B, H, keep),
                     dim=-1).values
    ko, vo = ops.compact(K.to(gpu), V.to(gpu), idx.to(gpu))
    rk, rv = R.gather_compressed(K, V, idx)
    assert torch.equal(ko.cpu().view(torch.int16), rk.view(torch.int16))
    assert torch.equal(vo.cpu().view(torch.int16), rv.view(torch.int16))


def test_compact_strided_and_odd_dim(gpu):
    from dropkv_amd import ops
    g = torch.Generator().manual_seed(2)
    big = torch.randn(1, 4, 300, 72, generator=g).to(torch.bfloat16).to(gpu)
    K = big[:, :, 50:250, :]          # non-contiguous along L/H (strided view)
    V = (big * 2)[:, :, 50:250, :]
    idx = torch.arange(0, 200, 3).view(1, 1, -1).expand(1, 4, -1).contiguous().to(gpu)
    ko, vo = ops.compact(K, V, idx)
    rk, rv = R.gather_compressed(K.cpu(), V.cpu(), idx.cpu())
    assert torch.equal(ko.cpu(), rk) and torch.equal(vo.cpu(), rv)


def test_compact2_matches_cat_gather(gpu):
    """Two-segment gather == torch.cat then gather (dropkv_cache.py:581-607)."""
    from dropkv_amd import ops
    g = torch.Generator().manual_seed(5)
    B, H, L0, L1, D, keep = 1, 8, 409, 4096, 128, 819
    K0 = torch.randn(B, H, L0, D, generator=g).to(torch.bfloat16)
    V0 = torch.randn(B, H, L0, D, generator=g).to(torch.bfloat16)
    K1 = torch.randn(B, H, L1, D, generator=g).to(torch.bfloat16)
    V1 = torch.randn(B, H, L1, D, generator=g).to(torch.bfloat16)
    idx = torch.sort(torch.stack([torch.randperm(L0 + L1, generator=g)[:keep] for _ in range(B * H)])
                     .view(B, H, keep), dim=-1).values
    ko, vo = ops.compact2(K0.to(gpu), V0.to(gpu), K1.to(gpu), V1.to(gpu), idx.to(gpu))
    rk, rv = R.gather_compressed(torch.cat([K0, K1], 2), torch.cat([V0, V1], 2), idx)
    assert torch.equal(ko.cpu(), rk) and torch.equal(vo.cpu(), rv)


@pytest.mark.parametrize("shape", [(1, 32, 8, 128, 2048, 2048), (2, 14, 2, 64, 3000, 5000), (1, 8, 8, 128, 64, 700)])
def test_evict_fused_matches_ops(gpu, shape):
    """One dropkv_evict call (score -> select -> gather fused in the emit
    stage) equals the separate ops and torch.gather bit for bit."""
    from dropkv_amd import ops
    B, Hq, Hkv, D, Lq, Lk = shape
    g = torch.Generator().manual_seed(Lk)
    Q = torch.randn(B, Hq, Lq, D, generator=g).to(torch.bfloat16).to(gpu)
    K = torch.randn(B, Hkv, Lk, D, generator=g).to(torch.bfloat16).to(gpu)
    V = torch.randn(B, Hkv, Lk, D, generator=g).to(torch.bfloat16).to(gpu)
    keep = max(int(0.1 * Lk), 8, 1)
    plan = ops.EvictPlan(Q, K, 8, 11, keep, keep_scores=True)
    idx, ko, vo = plan(Q, K, V)
    s = ops.scores(Q, K, V, 8)
    assert torch.equal(plan.scores, s)
    ref_idx = ops.select(s, 11, 8, keep)
    assert torch.equal(idx, ref_idx)
    rk, rv = R.gather_compressed(K.cpu(), V.cpu(), idx.cpu())
    assert torch.equal(ko.cpu(), rk) and torch.equal(vo.cpu(), rv)
    # and against the oracle's selection on the same scores
    pooled = R.pool_protect(s.cpu().clone(), 11, 8)
    assert torch.equal(idx.cpu(), R.topk_sorted(pooled, keep))


@pytest.mark.parametrize("Lk,ks,window,keep,splits,vzero", [
    (1000, 11, 8, 100, 0, False),
    (777, 1, 8, 77, 0, False),        # kernel_size 1: no halo at all
    (5000, 31, 64, 4999, 0, False),   # keep ~ Lk
    (4096, 11, 8, 1, 0, False),       # keep 1: only the protected maximum competes
    (3000, 11, 8, 300, 7, False),     # uneven split ranges
    (6400, 11, 8, 640, 200, False),   # 32-key split ranges: many boundaries
    (6400, 81, 8, 640, 200, False),   # ranges shorter than the kernel: standalone selection
    (2048, 11, 600, 700, 8, False),   # protected window wider than a split range
    (3000, 11, 8, 300, 0, True),      # V = 0: every score is 0, all ties
    (32768, 11, 8, 3276, 0, False),   # the headline row length
    (40000, 11, 8, 4000, 0, False),   # 40 chunks: more than one speculative window per region
    (40000, 11, 8, 4000, 0, True),    # ... with every score tied (overflow of the speculative loads)
    (5000, 131, 8, 500, 0, False),    # windows past 129 keys: block prefix / suffix pooling kernels
    (3000, 2049, 8, 300, 0, False),   # a window two thirds of the row
    (700, 4095, 8, 70, 0, False),     # a window wider than the row
])
def test_evict_fused_selection_edges(gpu, Lk, ks, window, keep, splits, vzero):
    """dropkv_evict (selection fused into the scoring tail where the plan
    allows) against the oracle's pool / protect / rank rule on the same GPU
    scores, and a bit-exact gather."""
    from dropkv_amd import ops
    g = torch.Generator().manual_seed(Lk + ks + keep)
    B, Hq, Hkv, D = 1, 8, 2, 128
    Q = torch.randn(B, Hq, 64, D, generator=g).to(torch.bfloat16).to(gpu)
    K = torch.randn(B, Hkv, Lk, D, generator=g).to(torch.bfloat16).to(gpu)
    V = torch.randn(B, Hkv, Lk, D, generator=g).to(torch.bfloat16).to(gpu)
    if vzero:
        V.zero_()
    plan = ops.EvictPlan(Q, K, 8, ks, keep, protect_window=window, splits=splits, keep_scores=True)
    idx, ko, vo = plan(Q, K, V)
    s = ops.scores(Q, K, V, 8, splits=splits)
    assert torch.equal(plan.scores, s)
    pooled = R.pool_protect(s.cpu().clone(), ks, window)
    assert torch.equal(idx.cpu(), R.topk_sorted(pooled, keep))
    rk, rv = R.gather_compressed(K.cpu(), V.cpu(), idx.cpu())
    assert torch.equal(ko.cpu(), rk) and torch.equal(vo.cpu(), rv)
    # a second call on the same plan (workspace reused) gives the same result
    idx2, _, _ = plan(Q, K, V)
    assert torch.equal(idx2, idx)
