"""Head dimensions and input dtypes beyond the bf16/fp16 D=64/128 core: D=32
on the matrix-core kernels, any other D (up to 4096) and fp32 inputs on the
generic vector-ALU kernels, through the same C ABI entry points.

The reference's Triton scorer takes any power-of-two D >= 32 in fp16/bf16
(dropkv_triton.py:680-716); its deployed PyTorch path takes any D and dtype,
fp32 included, because ``_compute_keep_indices`` falls back to it whenever
the fast path rejects its inputs (dropkv_cache.py:392-460).

Bars: fp32 mode rtol 1e-4 with an absolute floor of 1e-6 of the row maximum
(as the core's tests); p rounded to bf16 against the float32 oracle on the
binding keys (>= 0.1x the keep threshold): every one within 2e-2, fewer than
1e-3 of them beyond 1e-3; fp32 inputs rtol 1e-4; kept sets tie-aware against
the oracle; gathers bit-exact.
"""

import pytest
import torch

from conftest import assert_binding_scores, golden_case, make_qkv
from oracle import dropkv_ref as R

pytestmark = pytest.mark.gpu


def _close_rel(got, ref, rtol):
    got, ref = got.double().cpu(), ref.double().cpu()
    atol = 1e-6 * ref.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    bad = (got - ref).abs() > atol + rtol * ref.abs()
    assert not bad.any(), (
        f"{int(bad.sum())} mismatches; worst rel err "
        f"{((got - ref).abs() / ref.abs().clamp_min(1e-30))[bad].max().item():.3e}")


def _assert_kept(idx, q, k, v, W, ks, keep, scores64):
    """Kept set equals the oracle's top-k of pooled float64 scores, up to keys
    whose pooled value is within 1e-4 of the threshold (float32 rounding of
    either evaluation can order those either way)."""
    pooled = R.pool_protect(scores64.float().clone(), ks, W).double()
    ref_idx = R.topk_sorted(pooled, keep)
    B, H, _ = pooled.shape
    for b in range(B):
        for h in range(H):
            a, r = set(idx[b, h].tolist()), set(ref_idx[b, h].tolist())
            T = pooled[b, h, ref_idx[b, h]].min().item()
            for i in a ^ r:
                assert abs(pooled[b, h, i].item() - T) <= 1e-4 * abs(T), ((b, h), i, pooled[b, h, i].item(), T)


@pytest.mark.parametrize("D", [32, 256])
def test_head_dims_fp32_mode(gpu, D):
    """fp32 mode at Lk = 4096 (reference tests:122-137 at other D)."""
    from dropkv_amd import dropkv_scores_triton
    cfg = dict(B=1, Hq=8, Hkv=2, D=D)
    Q, K, V = make_qkv(cfg, 4096, seed=D)
    ref = R.dropkv_scores_reference(Q, K, V, match_pytorch_precision=False)
    got = dropkv_scores_triton(Q.to(gpu), K.to(gpu), V.to(gpu), match_pytorch_precision=False)
    assert got.shape == ref.shape and got.dtype == torch.float32
    _close_rel(got, ref, rtol=1e-4)


@pytest.mark.parametrize("D", [32, 256])
def test_head_dims_bf16_mode_binding(gpu, D):
    """p rounded to bf16 at Lk = 4096 on the binding keys."""
    from dropkv_amd import dropkv_scores_triton
    cfg = dict(B=1, Hq=8, Hkv=2, D=D)
    W, ks, keep = 8, 11, 409
    Q, K, V = make_qkv(cfg, 4096, seed=100 + D)
    ref = R.dropkv_scores_reference(Q, K, V, W, match_pytorch_precision=True)
    got = dropkv_scores_triton(Q.to(gpu), K.to(gpu), V.to(gpu), W, match_pytorch_precision=True).cpu()
    pooled = R.pool_protect(ref.clone(), ks, W)
    n_sel, worst, n_above, _ = assert_binding_scores(got, ref, pooled, keep, Q[:, :, -W:], K, V, W, torch.bfloat16,
                                                     2e-2, 1e-3, 1e-3)
    print(f"[D={D}] binding keys {n_sel}, worst rel {worst:.2e}, beyond 1e-3: {n_above}", flush=True)


@pytest.mark.parametrize("D", [80, 96, 512, 1024, 4096])
def test_deployed_path_other_head_dims(gpu, D):
    """Head dimensions only the deployed path takes (dropkv_cache.py:401-460):
    p and y rounded to bf16 against the oracle's fallback scores."""
    from dropkv_amd import ops
    cfg = dict(B=1, Hq=4, Hkv=2, D=D)
    Q, K, V = make_qkv(cfg, 64, 1024, seed=D)
    ref = R.fallback_scores(Q, K, V, 8)
    got = ops.scores(Q.to(gpu), K.to(gpu), V.to(gpu), 8, p_round=True, y_round=True).cpu()
    torch.testing.assert_close(got, ref, rtol=2e-2, atol=1e-3)
    rel = (got.double() - ref.double()).abs() / ref.double().abs().clamp_min(1e-30)
    assert (rel > 1e-3).double().mean().item() < 1e-2


@pytest.mark.parametrize("name", ["c1"])
def test_golden_with_fp32_tensors(gpu, name):
    """The golden case with its bf16 values held in fp32 tensors: with no
    rounding of p to an fp32 input dtype the result is the exact float64
    score (golden ``exact``) to rtol 1e-4, on both the p-rounding setting
    and the deployed setting (which rounds p and y to the input dtype)."""
    from dropkv_amd import ops
    c = golden_case(name)
    B, Hq, Hkv, D, Lq, Lk, W, ks, keep = c["meta"]
    q, k, v = (c[x].float().to(gpu) for x in ("q", "k", "v"))
    assert "exact" in c and q.shape[2] >= W
    for p_round, y_round in ((False, False), (True, False), (True, True)):
        got = ops.scores(q, k, v, W, p_round=p_round, y_round=y_round)
        _close_rel(got, c["exact"], 1e-4)


def test_fp32_evict_layer_call(gpu):
    """dropkv_evict on fp32 tensors: kept set against the float64 oracle,
    the fp32 rows gathered bit for bit."""
    from dropkv_amd import ops
    cfg = dict(B=2, Hq=8, Hkv=2, D=128)
    Q, K, V = make_qkv(cfg, 64, 2048, dtype=torch.float32, seed=5)
    W, ks, keep = 8, 11, 512
    idx, ko, vo = ops.evict(Q.to(gpu), K.to(gpu), V.to(gpu), W, ks, keep, protect_window=W)
    idx = idx.cpu()
    assert idx.shape == (2, 2, keep) and torch.equal(idx, torch.sort(idx, dim=-1).values)
    s64 = R.dropkv_scores_fp64(Q, K, V, W)
    _assert_kept(idx, Q, K, V, W, ks, keep, s64)
    rk, rv = R.gather_compressed(K, V, idx)
    assert ko.dtype == torch.float32 and torch.equal(ko.cpu(), rk) and torch.equal(vo.cpu(), rv)


@pytest.mark.parametrize("use_triton", [True, False])
def test_dropkv_cache_fp32_inputs(gpu, use_triton):
    """DropKVCache on fp32 Q/K/V: the fast path rejects fp32 (its dtype
    guard, dropkv_triton.py:695-697) and the layer is scored on the deployed
    path; the stored rows are the oracle's kept set, gathered bit for bit."""
    from dropkv_amd import DropKVCache
    cfg = dict(B=1, Hq=8, Hkv=2, D=64)
    Q, K, V = make_qkv(cfg, 1024, dtype=torch.float32, seed=9)
    c = DropKVCache(keep_ratio=0.25, window_size=8, kernel_size=11, use_triton=use_triton)
    c.update(Q.to(gpu), K.to(gpu), V.to(gpu), layer_idx=0)
    keep = R.keep_length(0.25, 1024, 8)
    kc = c.key_cache[0].cpu()
    assert kc.shape == (1, 2, keep, 64) and kc.dtype == torch.float32
    # Recover the kept indices from the stored rows (random fp32 rows are distinct).
    rows = {tuple(K[0, h, j].tolist()): j for h in range(2) for j in range(1024)}
    idx = torch.tensor([[[rows[tuple(kc[0, h, i].tolist())] for i in range(keep)] for h in range(2)]])
    s64 = R.dropkv_scores_fp64(Q, K, V, 8)
    _assert_kept(idx, Q, K, V, 8, 11, keep, s64)
    rk, rv = R.gather_compressed(K, V, idx)
    assert torch.equal(kc, rk) and torch.equal(c.value_cache[0].cpu(), rv)
