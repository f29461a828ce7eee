"""Transformers 5.x integration on the GPU: a small random-init Qwen2 (bf16,
head dim 64) whose cache evicts with the HIP layer-call.

Per layer, the kept indices are compared with the CPU oracle on the very
(query, key, value) the layer received (tie-aware overlap, the north-star
bar) and the compressed K/V with a gather by those indices (bit for bit).
Decode steps on the compressed cache must equal attention over exactly the
stored rows at the logical RoPE position.  The chunked-prefill flows restate
the reference's Qwen2 integration tests (tests/test_dropkv_triton.py:757-842,
:1083-1160) on the random-init model."""

import pytest
import torch

pytest.importorskip("transformers")

from oracle import dropkv_ref as R  # noqa: E402

pytestmark = pytest.mark.gpu

TINY = dict(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=3,
            num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=8192)


@pytest.fixture(scope="module")
def tiny(gpu):
    from dropkv_amd.e2e_qwen2 import build_model, make_config
    cfg = make_config(**TINY)
    return cfg, build_model(cfg, gpu, dtype=torch.bfloat16, seed=0)


def _ids(cfg, L, seed, dev):
    from dropkv_amd.e2e_qwen2 import random_prompt
    return random_prompt(cfg.vocab_size, L, seed=seed, device=dev)


def test_layer_cache_eviction_matches_oracle_and_decodes(gpu, tiny, monkeypatch):
    from transformers import DynamicCache
    from dropkv_amd import hf_cache
    from dropkv_amd.hf_query import query_capture
    cfg, model = tiny
    L, keep_ratio = 2048, 0.1
    rec = []
    real = hf_cache._evict

    def recording(q, k, v, window, ks, keep, use_triton):
        out = real(q, k, v, window, ks, keep, use_triton)
        rec.append((q[:, :, -window:].float().cpu(), k.float().cpu(), v.float().cpu(), k.cpu(), v.cpu(),
                    [t.cpu() for t in out], window, ks, keep))
        return out
    monkeypatch.setattr(hf_cache, "_evict", recording)

    cache = hf_cache.DropKVCache(cfg, keep_ratio=keep_ratio)
    ids = _ids(cfg, L, 11, gpu)
    with torch.no_grad(), query_capture():
        out = model(ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
    assert len(rec) == cfg.num_hidden_layers
    keep = int(keep_ratio * L)
    for li, (qt, kf, vf, kb, vb, (idx, kc, vc), window, ks, kk) in enumerate(rec):
        assert kk == keep and idx.shape == (1, cfg.num_key_value_heads, keep)
        s_ref = R.dropkv_scores_reference(qt.to(torch.bfloat16), kb, vb, window, match_pytorch_precision=True)
        pooled = R.pool_protect(s_ref.clone(), ks, window)
        overlap, _ = R.index_overlap(idx, R.topk_sorted(pooled, keep), pooled)
        assert overlap >= 0.999, f"layer {li}: overlap {overlap}"
        assert torch.equal(idx, torch.sort(idx, dim=-1).values)
        rk, rv = R.gather_compressed(kb, vb, idx)
        assert torch.equal(kc, rk) and torch.equal(vc, rv)
        assert torch.equal(cache.layers[li].keys.cpu(), kc)
    assert cache.get_seq_length() == L and cache.stored_length(0) == keep

    tok = out.logits[:, -1].argmax(-1, keepdim=True)
    with torch.no_grad(), query_capture():
        for t in range(4):
            dc = DynamicCache(config=cfg)
            for i, lay in enumerate(cache.layers):
                dc.update(lay.keys.clone(), lay.values.clone(), i)
            ref = model(tok, past_key_values=dc, use_cache=True, logits_to_keep=1,
                        position_ids=torch.tensor([[L + t]], device=gpu)).logits
            got = model(tok, past_key_values=cache, use_cache=True, logits_to_keep=1).logits
            assert torch.equal(got, ref), f"decode step {t}"
            assert cache.get_seq_length() == L + t + 1 and cache.stored_length(0) == keep + t + 1
            tok = got[:, -1].argmax(-1, keepdim=True)


def _chunked(model, ids, **kw):
    from dropkv_amd import DropKVCache, prefill_chunked
    from dropkv_amd.hf_query import query_capture
    c = DropKVCache(keep_ratio=kw.pop("keep_ratio", 0.3), window_size=8)
    with query_capture():
        out = prefill_chunked(model, ids, c, **kw)
    return c, out


def test_prefill_chunked_flows(gpu, tiny):
    """Shapes and seen-token counts of the reference's Qwen2 integration tests
    (tests/test_dropkv_triton.py:757-842, :1083-1145) on the HIP kernels."""
    from dropkv_amd import DropKVCache
    from dropkv_amd.hf_query import query_capture
    cfg, model = tiny
    L = 512
    ids = _ids(cfg, L, 12, gpu)
    final = max(int(0.3 * L), 8, 1)
    c_chunk, _ = _chunked(model, ids, chunk_size=128)
    c_single = DropKVCache(keep_ratio=0.3, window_size=8)
    with torch.no_grad(), query_capture():
        model(ids, past_key_values=c_single, use_cache=True, logits_to_keep=1)
    for a, b in zip(c_chunk.key_cache, c_single.key_cache):
        assert a.shape == b.shape == (1, cfg.num_key_value_heads, final, 64)
    assert c_chunk._seen_tokens == c_single._seen_tokens == L
    c, _ = _chunked(model, _ids(cfg, 5, 13, gpu), chunk_size=4096)
    assert c.key_cache[0].shape[2] == 5
    c, _ = _chunked(model, _ids(cfg, 100, 13, gpu), keep_ratio=0.5, chunk_size=4096, evict_strategy="budget",
                    max_kv_tokens=16)
    assert c.key_cache[0].shape[2] <= 16
    for strategy, kw in (("budget", dict(max_kv_tokens=256)), ("every_chunk", {})):
        c, _ = _chunked(model, ids, chunk_size=128, evict_strategy=strategy, **kw)
        assert all(k.shape[2] == final for k in c.key_cache)
        assert c._seen_tokens == L
        assert (c._prefill_mode, c._evict_use_seen_tokens, c._budget_max_kv_tokens) == ("single_pass", False, None)


@pytest.mark.parametrize("strategy,kw", [("budget", dict(max_kv_tokens=256)), ("every_chunk", {})])
def test_chunk_after_eviction_is_causal(gpu, tiny, strategy, kw):
    """Changing the prompt's last token leaves the next-to-last position's
    logits unchanged, also when earlier chunks were evicted."""
    cfg, model = tiny
    ids = _ids(cfg, 512, 14, gpu)
    ids2 = ids.clone()
    ids2[0, -1] = (ids2[0, -1] + 1) % cfg.vocab_size
    _, o1 = _chunked(model, ids, chunk_size=128, evict_strategy=strategy, logits_to_keep=2, **kw)
    _, o2 = _chunked(model, ids2, chunk_size=128, evict_strategy=strategy, logits_to_keep=2, **kw)
    assert torch.equal(o1.logits[:, 0], o2.logits[:, 0])


def test_e2e_harness_small(gpu, capsys):
    """The end-to-end harness runs (2 layers, short prompt) and reports both
    caches; the DropKV cache holds keep + decode rows, the dynamic one all."""
    import json
    from dropkv_amd import e2e_qwen2
    e2e_qwen2.main(["--prompt", "1024", "--decode", "4", "--layers", "2", "--reps", "1", "--warmup", "0"])
    line = capsys.readouterr().out.strip().splitlines()[-1]
    r = json.loads(line)
    assert r["dropkv"]["stored_kv_rows_layer0"] == 102 + 4
    assert r["dropkv"]["logical_length"] == 1024 + 4
    assert r["dynamic"]["stored_kv_rows_layer0"] == 1024 + 4
    assert r["dropkv"]["prefill_ms"] > 0 and r["dropkv"]["decode_tok_s"] > 0
