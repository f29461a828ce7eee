"""Chunked prefill on preallocated capacity (``dropkv_append``,
``dropkv_evict_ld``, ``DropKVCache(capacity=...)``).

The bar is bit-exactness against the default mode, which follows the
reference's cat + gather semantics (dropkv_cache.py:571-622): the same kept
rows, the same stored K/V and the same K/V returned for the chunk's
attention, after every update of every schedule that ``prefill_chunked``
uses (last_chunk, every_chunk, budget), with the fast and the deployed
scoring paths.  The entry points are also checked on their own: rows
outside the ones named are neither read (NaN-filled) nor written."""

import pytest
import torch

from conftest import BATCH2_CFG, LLAMA_CFG, QWEN_CFG, make_qkv

pytestmark = pytest.mark.gpu


def test_append_matches_slice_assignment(gpu):
    from dropkv_amd import ops
    B, H, L, D, C, row0 = 2, 4, 300, 128, 512, 37
    g = torch.Generator().manual_seed(3)
    # a [B, L, H, D] projection viewed as [B, H, L, D]: strided rows
    src_k = torch.randn(B, L, H, D, generator=g).bfloat16().to(gpu).transpose(1, 2)
    src_v = torch.randn(B, L, H, D, generator=g).bfloat16().to(gpu).transpose(1, 2)
    kb = torch.full((B, H, C, D), 7.0, dtype=torch.bfloat16, device=gpu)
    vb = torch.full_like(kb, -7.0)
    ops.append(src_k, src_v, kb, vb, row0)
    torch.cuda.synchronize()
    assert torch.equal(kb[:, :, row0:row0 + L], src_k) and torch.equal(vb[:, :, row0:row0 + L], src_v)
    assert bool((kb[:, :, :row0] == 7).all()) and bool((kb[:, :, row0 + L:] == 7).all())
    assert bool((vb[:, :, :row0] == -7).all()) and bool((vb[:, :, row0 + L:] == -7).all())
    with pytest.raises(RuntimeError, match="do not fit"):
        ops.append(src_k, src_v, kb, vb, C - L + 1)


@pytest.mark.parametrize("cfg,fast,dtype", [(LLAMA_CFG, True, torch.bfloat16), (LLAMA_CFG, False, torch.bfloat16),
                                            (QWEN_CFG, True, torch.bfloat16), (BATCH2_CFG, True, torch.bfloat16),
                                            (LLAMA_CFG, True, torch.float16)])
def test_evict_ld_matches_evict(gpu, cfg, fast, dtype):
    """K/V in rows 0..Lk-1 of NaN-filled buffers, outputs into the first
    rows of sentinel-filled buffers: the same indices and rows as the
    contiguous layer-call."""
    from dropkv_amd import ops
    Lk, Lq, C, W, ks = 3000, 1024, 3100, 8, 11
    Q, K, V = make_qkv(cfg, Lq, Lk, seed=11, dtype=dtype, k_scale="lognormal")
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    keep = int(0.1 * Lk)
    plan = ops.EvictPlan(Qg, Kg, W, ks, keep, p_round=True, y_round=not fast)
    idx, kc, vc = plan(Qg, Kg, Vg)
    B, H, _, D = K.shape
    kb = torch.full((B, H, C, D), float("nan"), dtype=dtype, device=gpu)
    vb = torch.full_like(kb, float("nan"))
    kb[:, :, :Lk] = Kg
    vb[:, :, :Lk] = Vg
    ko = torch.full((B, H, keep + 40, D), 3.0, dtype=dtype, device=gpu)
    vo = torch.full_like(ko, 3.0)
    idx2 = ops.evict_ld(Qg, kb, vb, Lk, W, ks, keep, ko, vo, p_round=True, y_round=not fast)
    torch.cuda.synchronize()
    assert torch.equal(idx2, idx)
    assert torch.equal(ko[:, :, :keep], kc) and torch.equal(vo[:, :, :keep], vc)
    assert bool((ko[:, :, keep:] == 3).all()) and bool((vo[:, :, keep:] == 3).all())


def _mode(strategy, i, n_chunks, stored, chunk_len, max_kv):
    """The mode prefill_chunked sets for chunk i (dropkv_cache.py:733-771)."""
    last = i == n_chunks - 1
    if strategy == "last_chunk":
        return "evict_accumulated" if last else "accumulate"
    if strategy == "every_chunk":
        return "single_pass" if i == 0 else "evict_accumulated"
    if last:
        return "evict_accumulated"
    return "evict_accumulated" if stored + chunk_len > max_kv else "accumulate"


@pytest.mark.parametrize("strategy,use_triton,cfg", [
    ("last_chunk", True, LLAMA_CFG), ("every_chunk", True, LLAMA_CFG), ("budget", True, LLAMA_CFG),
    ("last_chunk", False, LLAMA_CFG), ("every_chunk", False, LLAMA_CFG), ("budget", False, LLAMA_CFG),
    ("every_chunk", True, QWEN_CFG), ("budget", True, BATCH2_CFG),
])
def test_capacity_cache_bit_exact_with_default(gpu, strategy, use_triton, cfg):
    """Both caches driven through update() in lock step, as a model in
    prefill_chunked drives them, compared after every layer of every chunk."""
    from dropkv_amd import DropKVCache
    L, chunk, layers, max_kv = 2304, 512, 2, 900  # the last chunk is shorter (256)
    Q, K, V = make_qkv(cfg, L, seed=5, k_scale="lognormal")
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    ref = DropKVCache(keep_ratio=0.3, use_triton=use_triton)
    cap = DropKVCache(keep_ratio=0.3, use_triton=use_triton, capacity=L)
    n_chunks = (L + chunk - 1) // chunk
    for c in (ref, cap):
        c._evict_use_seen_tokens = strategy in ("budget", "every_chunk")
        c._budget_max_kv_tokens = max_kv if strategy == "budget" else None
    for i in range(n_chunks):
        s, e = i * chunk, min((i + 1) * chunk, L)
        stored = ref.key_cache[0].shape[2] if ref.key_cache else 0
        mode = _mode(strategy, i, n_chunks, stored, e - s, max_kv)
        for layer in range(layers):
            rets = []
            for c in (ref, cap):
                c._prefill_mode = mode
                rets.append(c.update(Qg[:, :, s:e], Kg[:, :, s:e], Vg[:, :, s:e], layer_idx=layer))
            (rk, rv), (ck, cv) = rets
            assert torch.equal(ck, rk) and torch.equal(cv, rv), (i, layer, mode, "returned K/V")
            assert torch.equal(cap.key_cache[layer], ref.key_cache[layer]), (i, layer, mode, "stored K")
            assert torch.equal(cap.value_cache[layer], ref.value_cache[layer]), (i, layer, mode, "stored V")
    assert cap.get_seq_length() == ref.get_seq_length() == L
    for c in (ref, cap):
        c._prefill_mode = "single_pass"
        c._evict_use_seen_tokens = False
        c._budget_max_kv_tokens = None
    # decode steps append in place
    for t in range(3):
        kn = torch.randn(cfg["B"], cfg["Hkv"], 1, cfg["D"],
                         generator=torch.Generator().manual_seed(t)).bfloat16().to(gpu)
        a = ref.update(None, kn, kn, layer_idx=0)
        b = cap.update(None, kn, kn, layer_idx=0)
        assert torch.equal(a[0], b[0]) and torch.equal(cap.key_cache[0], ref.key_cache[0])


def test_capacity_exceeded_raises(gpu):
    from dropkv_amd import DropKVCache
    Q, K, V = make_qkv(LLAMA_CFG, 256, seed=6)
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    c = DropKVCache(keep_ratio=0.3, capacity=200)
    c._prefill_mode = "accumulate"
    c.update(Qg[:, :, :128], Kg[:, :, :128], Vg[:, :, :128], layer_idx=0)
    with pytest.raises(ValueError, match="capacity of 200 rows exceeded"):
        c.update(Qg[:, :, 128:], Kg[:, :, 128:], Vg[:, :, 128:], layer_idx=0)


TINY = dict(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=3,
            num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=8192)


@pytest.mark.parametrize("strategy", ["last_chunk", "every_chunk", "budget"])
def test_prefill_chunked_with_capacity(gpu, strategy):
    """prefill_chunked through a Transformers model: same logits, same caches."""
    from dropkv_amd import DropKVCache, prefill_chunked
    from dropkv_amd.e2e_qwen2 import build_model, make_config, random_prompt
    from dropkv_amd.hf_query import query_capture
    cfg = make_config(**TINY)
    model = build_model(cfg, gpu, dtype=torch.bfloat16, seed=0)
    ids = random_prompt(cfg.vocab_size, 1500, seed=9, device=gpu)
    outs = []
    caches = []
    for capacity in (None, 1600):
        cache = DropKVCache(keep_ratio=0.2, capacity=capacity)
        with torch.no_grad(), query_capture():
            out = prefill_chunked(model, ids, cache, chunk_size=400, evict_strategy=strategy, max_kv_tokens=700)
        outs.append(out.logits if hasattr(out, "logits") else out[0])
        caches.append(cache)
    assert torch.equal(outs[0], outs[1])
    for layer in range(cfg.num_hidden_layers):
        assert torch.equal(caches[0].key_cache[layer], caches[1].key_cache[layer])
        assert torch.equal(caches[0].value_cache[layer], caches[1].value_cache[layer])


def test_capacity_flow_makes_no_concatenation(gpu, monkeypatch):
    """The capacity mode appends in place: a full last_chunk flow (and a
    decode step) runs with torch.cat unavailable."""
    from dropkv_amd import DropKVCache
    Q, K, V = make_qkv(LLAMA_CFG, 1536, seed=8)
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    c = DropKVCache(keep_ratio=0.2, capacity=1600)

    def no_cat(*a, **k):
        raise AssertionError("torch.cat called in capacity mode")

    monkeypatch.setattr(torch, "cat", no_cat)
    for i, mode in enumerate(("accumulate", "accumulate", "evict_accumulated")):
        c._prefill_mode = mode
        s, e = 512 * i, 512 * (i + 1)
        c.update(Qg[:, :, s:e], Kg[:, :, s:e], Vg[:, :, s:e], layer_idx=0)
    c._prefill_mode = "single_pass"
    c.update(None, Kg[:, :, :1], Vg[:, :, :1], layer_idx=0)
    assert c.key_cache[0].shape[2] == max(int(0.2 * 1536), 8) + 1


def test_capacity_reorder_cache_matches_default(gpu):
    """reorder_cache (beam reordering along the batch) in capacity mode gives
    the default mode's tensors, and later appends land after them."""
    from dropkv_amd import DropKVCache
    Q, K, V = make_qkv(BATCH2_CFG, 1024, seed=12)
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    ref = DropKVCache(keep_ratio=0.2)
    cap = DropKVCache(keep_ratio=0.2, capacity=1100)
    for c in (ref, cap):
        c._prefill_mode = "accumulate"
        c.update(Qg[:, :, :512], Kg[:, :, :512], Vg[:, :, :512], layer_idx=0)
        c._prefill_mode = "evict_accumulated"
        c.update(Qg[:, :, 512:], Kg[:, :, 512:], Vg[:, :, 512:], layer_idx=0)
        c._prefill_mode = "single_pass"
        c.reorder_cache(torch.tensor([1, 0]))
    assert torch.equal(cap.key_cache[0], ref.key_cache[0]) and torch.equal(cap.value_cache[0], ref.value_cache[0])
    kn = torch.randn(2, 8, 1, 128, generator=torch.Generator().manual_seed(4)).bfloat16().to(gpu)
    for c in (ref, cap):
        c.update(None, kn, kn, layer_idx=0)
    assert torch.equal(cap.key_cache[0], ref.key_cache[0])
