"""DropKVCache / prefill eviction on the GPU, mirroring the reference's cache
and chunked-prefill tests (tests/test_dropkv_triton.py:535-1330, :1901-1960),
plus parity of the compressed cache with the CPU oracle's deployed path."""

import pytest
import torch

from conftest import LLAMA_CFG, QWEN_CFG, make_qkv
from oracle import dropkv_ref as R

pytestmark = pytest.mark.gpu


def _qkv(cfg, L, Lk=None, seed=0, dev=None):
    Q, K, V = make_qkv(cfg, L, Lk, seed=seed)
    return Q.to(dev), K.to(dev), V.to(dev)


def _cache(**kw):
    from dropkv_amd import DropKVCache
    d = dict(keep_ratio=0.3, window_size=8, kernel_size=11, use_triton=False)
    d.update(kw)
    return DropKVCache(**d)


@pytest.mark.parametrize("use_triton", [False, True])
def test_hf_4arg_with_query_states(gpu, use_triton):
    Q, K, V = _qkv(LLAMA_CFG, 128, dev=gpu)
    c = _cache(use_triton=use_triton)
    rk, rv = c.update(K, V, 0, {"query_states": Q})
    assert rk.shape[-2] == 128
    assert c.key_cache[0].shape[-2] == max(int(0.3 * 128), 8, 1)


@pytest.mark.parametrize("use_triton", [False, True])
def test_chunked_matches_single_pass_bit_exact(gpu, use_triton):
    """accumulate + evict_accumulated == single pass, bit for bit
    (reference tests:604-634)."""
    Q, K, V = _qkv(LLAMA_CFG, 256, seed=1, dev=gpu)
    single = _cache(use_triton=use_triton)
    single.update(Q, K, V, layer_idx=0)
    ch = _cache(use_triton=use_triton)
    ch._prefill_mode = "accumulate"
    ch.update(Q[:, :, :128], K[:, :, :128], V[:, :, :128], layer_idx=0)
    ch._prefill_mode = "evict_accumulated"
    ch.update(Q[:, :, 128:], K[:, :, 128:], V[:, :, 128:], layer_idx=0)
    assert torch.equal(ch.key_cache[0], single.key_cache[0])
    assert torch.equal(ch.value_cache[0], single.value_cache[0])


def test_evict_accumulated_returns_full_stores_compressed(gpu):
    Q, K, V = _qkv(LLAMA_CFG, 128, seed=2, dev=gpu)
    c = _cache()
    c._prefill_mode = "accumulate"
    c.update(Q[:, :, :64], K[:, :, :64], V[:, :, :64], layer_idx=0)
    c._prefill_mode = "evict_accumulated"
    fk, fv = c.update(Q[:, :, 64:], K[:, :, 64:], V[:, :, 64:], layer_idx=0)
    assert torch.equal(fk, K) and torch.equal(fv, V)
    assert c.key_cache[0].shape[2] == max(int(0.3 * 128), 8, 1)
    assert c._seen_tokens == 128


def test_multi_chunk_multi_layer(gpu):
    Q, K, V = _qkv(LLAMA_CFG, 192, seed=3, dev=gpu)
    c = _cache(keep_ratio=0.2)
    c._prefill_mode = "accumulate"
    for layer in range(3):
        c.update(Q[:, :, :64], K[:, :, :64], V[:, :, :64], layer_idx=layer)
    for layer in range(3):
        c.update(Q[:, :, 64:128], K[:, :, 64:128], V[:, :, 64:128], layer_idx=layer)
    c._prefill_mode = "evict_accumulated"
    for layer in range(3):
        c.update(Q[:, :, 128:], K[:, :, 128:], V[:, :, 128:], layer_idx=layer)
    for layer in range(3):
        assert c.key_cache[layer].shape[2] == max(int(0.2 * 192), 8, 1)


def test_decode_after_chunked(gpu):
    Q, K, V = _qkv(LLAMA_CFG, 129, seed=4, dev=gpu)
    c = _cache()
    c._prefill_mode = "accumulate"
    c.update(Q[:, :, :64], K[:, :, :64], V[:, :, :64], layer_idx=0)
    c._prefill_mode = "evict_accumulated"
    c.update(Q[:, :, 64:128], K[:, :, 64:128], V[:, :, 64:128], layer_idx=0)
    c._prefill_mode = "single_pass"
    n = c.key_cache[0].shape[2]
    rk, _ = c.update(Q[:, :, 128:], K[:, :, 128:], V[:, :, 128:], layer_idx=0)
    assert rk.shape[2] == n + 1 and torch.equal(rk[:, :, -1], K[:, :, 128])
    assert c.get_seq_length() == 129


def test_total_tokens_and_budget_cap(gpu):
    """reference tests:909-937, :1183-1204, :1239-1262."""
    Q, K, V = _qkv(LLAMA_CFG, 128, seed=5, dev=gpu)
    c = _cache(keep_ratio=0.3)
    assert c._compute_keep_indices(Q, K, V).shape[2] == 38
    assert c._compute_keep_indices(Q, K, V, total_tokens=512).shape[2] == 128
    assert c._compute_keep_indices(Q, K, V, total_tokens=200).shape[2] == 60
    assert _cache(keep_ratio=0.01)._compute_keep_indices(Q[:, :, :64], K[:, :, :64], V[:, :, :64],
                                                         total_tokens=10).shape[2] == 8
    Q, K, V = _qkv(LLAMA_CFG, 512, seed=6, dev=gpu)
    c = _cache(keep_ratio=0.8)
    c._evict_use_seen_tokens = True
    c._budget_max_kv_tokens = 100
    c._prefill_mode = "accumulate"
    c.update(Q[:, :, :256], K[:, :, :256], V[:, :, :256], layer_idx=0)
    c._prefill_mode = "evict_accumulated"
    c.update(Q[:, :, 256:], K[:, :, 256:], V[:, :, 256:], layer_idx=0)
    assert c.key_cache[0].shape[2] == 100


def test_every_chunk_and_budget_growth(gpu):
    Q, K, V = _qkv(LLAMA_CFG, 512, seed=7, dev=gpu)
    c = _cache(keep_ratio=0.3)
    c._evict_use_seen_tokens = True
    c._prefill_mode = "single_pass"
    c.update(Q[:, :, :64], K[:, :, :64], V[:, :, :64], layer_idx=0)
    assert c.key_cache[0].shape[2] < 64
    c._prefill_mode = "evict_accumulated"
    c.update(Q[:, :, 64:128], K[:, :, 64:128], V[:, :, 64:128], layer_idx=0)
    assert c.key_cache[0].shape[2] == max(int(0.3 * 128), 8, 1)
    c.update(Q[:, :, 128:192], K[:, :, 128:192], V[:, :, 128:192], layer_idx=0)
    assert c.key_cache[0].shape[2] == max(int(0.3 * 192), 8, 1)


def test_short_final_chunk_uses_deployed_semantics(gpu):
    """Final chunk of 6 < window 8 tokens: the fast path's guard fires and the
    deployed semantics (W = min(8, 6)) score it (reference tests:1206-1225)."""
    Q, K, V = _qkv(LLAMA_CFG, 70, seed=8, dev=gpu)
    for use_triton in (False, True):
        c = _cache(use_triton=use_triton)
        c._prefill_mode = "accumulate"
        c.update(Q[:, :, :64], K[:, :, :64], V[:, :, :64], layer_idx=0)
        c._prefill_mode = "evict_accumulated"
        c.update(Q[:, :, 64:], K[:, :, 64:], V[:, :, 64:], layer_idx=0)
        assert c.key_cache[0].shape[2] == max(int(0.3 * 70), 8, 1)


def test_fast_path_handles_mismatched_q_length(gpu):
    Q, K, V = _qkv(LLAMA_CFG, 256, seed=9, dev=gpu)
    c = _cache(use_triton=True)
    idx = c._compute_keep_indices(Q[:, :, 128:], K, V)
    assert idx.shape == (1, 8, 76)
    assert torch.equal(idx, c._compute_keep_indices(Q, K, V))


def test_fast_path_is_the_hip_op(gpu, monkeypatch):
    """With use_triton=True the cache scores with the fast path's semantics
    (reference tests:1919-1960): its prefill eviction is one fused HIP
    layer-call with y in fp32, and _compute_keep_indices calls
    dropkv_scores_triton; both keep the same rows."""
    import dropkv_amd.dropkv_triton as T
    from dropkv_amd import ops
    calls = []
    real_scores, real_evict = T.dropkv_scores_triton, ops.evict

    def spy_scores(*a, **k):
        calls.append("scores")
        return real_scores(*a, **k)

    def spy_evict(*a, **k):
        calls.append(("evict", k.get("y_round")))
        return real_evict(*a, **k)

    monkeypatch.setattr(T, "dropkv_scores_triton", spy_scores)
    monkeypatch.setattr(ops, "evict", spy_evict)
    Q, K, V = _qkv(LLAMA_CFG, 128, seed=10, dev=gpu)
    c = _cache(use_triton=True)
    c.update(Q, K, V, layer_idx=0)
    assert calls == [("evict", False)]
    idx = c._compute_keep_indices(Q, K, V)
    assert calls[-1] == "scores"
    rk, rv = ops.compact(K, V, idx)
    assert torch.equal(c.key_cache[0], rk) and torch.equal(c.value_cache[0], rv)


@pytest.mark.parametrize("cfg,L", [(LLAMA_CFG, 4096), (QWEN_CFG, 4096)])
def test_compressed_cache_vs_oracle_deployed_path(gpu, cfg, L):
    """use_triton=False: GPU scores follow the deployed path (p and y rounded
    to bf16); the kept set matches the oracle's deployed path up to exact
    threshold ties and float-rounding neighbours (overlap >= 0.99), and
    given the GPU's own indices the compressed cache is bit-exact."""
    Q, K, V = make_qkv(cfg, L, seed=11)
    c = _cache(keep_ratio=0.1)
    c.update(Q.to(gpu), K.to(gpu), V.to(gpu), layer_idx=0)
    ref_idx, pooled = R.compute_keep_indices(Q, K, V, 0.1, 8, 11)
    from dropkv_amd import ops
    gpu_scores = ops.scores(Q.to(gpu), K.to(gpu), V.to(gpu), 8, p_round=True, y_round=True)
    gpu_idx = ops.select(gpu_scores, 11, 8, ref_idx.shape[-1])
    worst, _ = R.index_overlap(gpu_idx.cpu(), ref_idx, pooled)
    assert worst >= 0.99
    rk, rv = R.gather_compressed(K, V, gpu_idx.cpu())
    assert torch.equal(c.key_cache[0].cpu(), rk) and torch.equal(c.value_cache[0].cpu(), rv)


def test_guards_on_device(gpu):
    """Guards that come after the device check (dropkv_triton.py:695-707)."""
    from dropkv_amd import dropkv_scores_triton
    Q, K, V = _qkv(LLAMA_CFG, 64, dev=gpu)
    with pytest.raises(AssertionError, match="contiguous"):
        dropkv_scores_triton(Q, K.transpose(2, 3), V)
    with pytest.raises(AssertionError, match="same dtype"):
        dropkv_scores_triton(Q, K.half(), V)
    with pytest.raises(AssertionError, match="fp16 or bf16"):
        dropkv_scores_triton(Q.float(), K.float(), V.float())
    with pytest.raises(AssertionError, match="shape mismatch"):
        dropkv_scores_triton(Q[:, :, :32], K[:, :, :32].contiguous(), V)
    Qn = Q.transpose(2, 3).contiguous().transpose(2, 3)
    assert dropkv_scores_triton(Qn, K, V).shape == (1, 8, 64)


@pytest.mark.parametrize("dtype,L0,L1,D,strided", [
    (torch.bfloat16, 6553, 4096, 128, False),   # the C3 continuation: stored rows || chunk
    (torch.float16, 0, 300, 64, False),          # nothing stored yet
    (torch.bfloat16, 1638, 1, 64, True),         # one decode row, inputs as transposed projections
    (torch.float32, 77, 5, 80, False),           # fp32 rows, D not a multiple of 16 bytes' elements
])
def test_cat_rows_equals_torch_cat(gpu, dtype, L0, L1, D, strided):
    """The continuation's append (dropkv_cache.py:573-588, :611-616) through
    the library's append kernel gives torch.cat's tensors bit for bit."""
    from dropkv_amd.dropkv_cache import cat_rows
    g = torch.Generator(device=gpu).manual_seed(L0 + L1 + D)
    B, H = 2, 3

    def draw(L):
        if strided:   # [B, L, H, D] viewed as [B, H, L, D]
            return torch.randn(B, L, H, D, device=gpu, generator=g).to(dtype).transpose(1, 2)
        return torch.randn(B, H, L, D, device=gpu, generator=g).to(dtype)

    k0, v0, k1, v1 = draw(L0), draw(L0), draw(L1), draw(L1)
    k, v = cat_rows(k0, v0, k1, v1)
    rk, rv = torch.cat([k0, k1], dim=-2), torch.cat([v0, v1], dim=-2)
    assert k.is_contiguous() and v.is_contiguous() and k.shape == rk.shape
    assert torch.equal(k, rk) and torch.equal(v, rv)
