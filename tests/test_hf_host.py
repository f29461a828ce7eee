"""Transformers 5.x integration on the CPU: query capture, logical (RoPE) vs
stored (mask) lengths, decode on the compressed cache, and ``prefill_chunked``
driving a real (tiny, random-init) Qwen2 model.

The HIP eviction cannot run without a GPU, so here the eviction step is
replaced by the CPU oracle (test infrastructure): these tests check the
plumbing around the kernels -- which query reaches them, what is stored, and
how the model attends afterwards.  The same flows run on the HIP kernels in
``test_gpu_hf.py``.  Reference behaviour: patches/dropkv_transformers.patch
(DropKVLayer / DropKVCache, query_states in cache_kwargs), dropkv_cache.py:
493-648 and the reference's Qwen2 integration tests
(tests/test_dropkv_triton.py:757-842, :1083-1160), which load a pretrained
checkpoint; a seeded random-init model of a small Qwen2 configuration stands
in for it here.
"""

import pytest
import torch

pytest.importorskip("transformers")

from transformers import DynamicCache  # noqa: E402
from transformers.models.qwen2 import modeling_qwen2  # noqa: E402

from dropkv_amd import DropKVCache, prefill_chunked  # noqa: E402
from dropkv_amd import hf_cache  # noqa: E402
from dropkv_amd.e2e_qwen2 import build_model, make_config, random_prompt  # noqa: E402
from dropkv_amd.hf_query import query_capture  # noqa: E402
from oracle import dropkv_ref as R  # noqa: E402

TINY = dict(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096)


@pytest.fixture(scope="module")
def tiny():
    cfg = make_config(**TINY)
    return cfg, build_model(cfg, "cpu", dtype=torch.float32, seed=0)


def _oracle_evict(calls=None):
    def evict(q, k, v, window, ks, keep, use_triton):
        if calls is not None:
            calls.append((q.clone(), k.clone(), v.clone()))
        idx, _ = R.compute_keep_indices(q, k, v, 1.0, window, ks, max_keep_len=keep)
        kc, vc = R.gather_compressed(k, v, idx)
        return idx, kc, vc
    return evict


def _oracle_standalone(monkeypatch):
    """The standalone cache's fused eviction (score .. gather) replaced by
    the oracle's deployed path."""
    def evict_layer(self, q, k, v, total_tokens=None, max_keep_len=None):
        idx = R.compute_keep_indices(q, k, v, self.keep_ratio, self.window_size, self.kernel_size,
                                     total_tokens, max_keep_len)[0]
        return R.gather_compressed(k, v, idx)
    monkeypatch.setattr(DropKVCache, "_evict_layer", evict_layer)


def _decode_reference(model, cfg, layers_kv, token, position):
    """One decode step through an uncompressed DynamicCache holding exactly
    the compressed K/V, with the RoPE position given explicitly."""
    dc = DynamicCache(config=cfg)
    for i, (k, v) in enumerate(layers_kv):
        dc.update(k.clone(), v.clone(), i)
    with torch.no_grad():
        out = model(token, past_key_values=dc, use_cache=True, logits_to_keep=1,
                    position_ids=torch.tensor([[position]]))
    return out.logits


def test_query_capture_records_rotated_query_and_restores(tiny, monkeypatch):
    cfg, model = tiny
    orig = modeling_qwen2.apply_rotary_pos_emb
    calls = []
    monkeypatch.setattr(hf_cache, "_evict", _oracle_evict(calls))
    ids = random_prompt(cfg.vocab_size, 64, seed=3)
    cache = hf_cache.DropKVCache(cfg, keep_ratio=0.25)
    with torch.no_grad(), query_capture():
        assert modeling_qwen2.apply_rotary_pos_emb is not orig
        model(ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
    assert modeling_qwen2.apply_rotary_pos_emb is orig
    assert len(calls) == cfg.num_hidden_layers
    # Layer 0's query, recomputed from the embedding with the library's own
    # projection and rotary functions.
    attn = model.model.layers[0].self_attn
    with torch.no_grad():
        h = model.model.layers[0].input_layernorm(model.model.embed_tokens(ids))
        q = attn.q_proj(h).view(1, 64, -1, attn.head_dim).transpose(1, 2)
        k = attn.k_proj(h).view(1, 64, -1, attn.head_dim).transpose(1, 2)
        cos, sin = model.model.rotary_emb(h, torch.arange(64)[None])
        q_rot, k_rot = orig(q, k, cos, sin)
    assert torch.equal(calls[0][0], q_rot)
    assert torch.equal(calls[0][1], k_rot)


def test_no_capture_no_eviction(tiny, monkeypatch):
    """Without a query (unpatched attention, no capture) the layer stores the
    full K/V, as the reference layer does (patch:103-109)."""
    cfg, model = tiny
    monkeypatch.setattr(hf_cache, "_evict", lambda *a: pytest.fail("evicted without a query"))
    cache = hf_cache.DropKVCache(cfg, keep_ratio=0.25)
    with torch.no_grad():
        model(random_prompt(cfg.vocab_size, 40), past_key_values=cache, use_cache=True, logits_to_keep=1)
    assert cache.stored_length(0) == 40 and cache.get_seq_length() == 40


@pytest.mark.parametrize("kind", ["layer", "standalone"])
def test_decode_on_compressed_cache(tiny, monkeypatch, kind):
    """After eviction: RoPE positions follow the logical length, the mask the
    stored length; every decode step equals attention over exactly the stored
    rows at the logical position (bit for bit)."""
    cfg, model = tiny
    L = 100
    monkeypatch.setattr(hf_cache, "_evict", _oracle_evict())
    _oracle_standalone(monkeypatch)
    cache = hf_cache.DropKVCache(cfg, keep_ratio=0.3) if kind == "layer" else DropKVCache(keep_ratio=0.3)
    ids = random_prompt(cfg.vocab_size, L, seed=5)

    def kv():
        if kind == "layer":
            return [(lay.keys, lay.values) for lay in cache.layers]
        return list(zip(cache.key_cache, cache.value_cache))

    with torch.no_grad(), query_capture():
        out = model(ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
        tok = out.logits[:, -1].argmax(-1, keepdim=True)
        assert cache.get_seq_length() == L
        assert all(k.shape[2] == 30 for k, _ in kv())
        for t in range(3):
            ref = _decode_reference(model, cfg, kv(), tok, L + t)
            out = model(tok, past_key_values=cache, use_cache=True, logits_to_keep=1)
            assert torch.equal(out.logits, ref)
            assert cache.get_seq_length() == L + t + 1
            assert all(k.shape[2] == 30 + t + 1 for k, _ in kv())
            tok = out.logits[:, -1].argmax(-1, keepdim=True)


def test_layer_crop_and_reset(tiny, monkeypatch):
    cfg, model = tiny
    monkeypatch.setattr(hf_cache, "_evict", _oracle_evict())
    cache = hf_cache.DropKVCache(cfg, keep_ratio=0.3)
    with torch.no_grad(), query_capture():
        model(random_prompt(cfg.vocab_size, 100), past_key_values=cache, use_cache=True, logits_to_keep=1)
    lay = cache.layers[0]
    assert (lay.get_seq_length(), cache.stored_length(0)) == (100, 30)
    lay.crop(-5)
    assert (lay.get_seq_length(), cache.stored_length(0)) == (25, 25)
    lay.crop(20)
    assert (lay.get_seq_length(), cache.stored_length(0)) == (20, 20)
    cache.reset()
    assert cache.stored_length(0) == 0 and lay.get_seq_length() == 0 and not lay._prefilled


def _chunked(model, ids, monkeypatch, **kw):
    _oracle_standalone(monkeypatch)
    c = DropKVCache(keep_ratio=kw.pop("keep_ratio", 0.3), window_size=8)
    with query_capture():
        out = prefill_chunked(model, ids, c, **kw)
    return c, out


def test_prefill_chunked_matches_single_pass_shapes(tiny, monkeypatch):
    """tests/test_dropkv_triton.py:757-791: chunked vs single-pass cache shapes
    and seen-token counts."""
    cfg, model = tiny
    ids = random_prompt(cfg.vocab_size, 512, seed=7)
    c_chunk, _ = _chunked(model, ids, monkeypatch, chunk_size=128)
    c_single = DropKVCache(keep_ratio=0.3, window_size=8)
    with torch.no_grad(), query_capture():
        model(ids, past_key_values=c_single, use_cache=True)
    assert len(c_chunk.key_cache) == cfg.num_hidden_layers
    for a, b in zip(c_chunk.key_cache, c_single.key_cache):
        assert a.shape == b.shape == (1, cfg.num_key_value_heads, int(0.3 * 512), 64)
    assert c_chunk._seen_tokens == c_single._seen_tokens == 512


def test_prefill_chunked_short_prompt_and_budget(tiny, monkeypatch):
    """tests/test_dropkv_triton.py:793-842: a prompt shorter than the chunk
    goes through one forward with eviction; ``budget`` enforces
    ``max_kv_tokens`` even then."""
    cfg, model = tiny
    ids = random_prompt(cfg.vocab_size, 100, seed=8)
    c, _ = _chunked(model, ids, monkeypatch, chunk_size=4096)
    assert c.key_cache[0].shape[2] == 30
    short = random_prompt(cfg.vocab_size, 5, seed=8)
    c, _ = _chunked(model, short, monkeypatch, chunk_size=4096)
    assert c.key_cache[0].shape[2] == 5          # shorter than the window: stored whole
    c, _ = _chunked(model, ids, monkeypatch, keep_ratio=0.5, chunk_size=4096, evict_strategy="budget",
                    max_kv_tokens=16)
    assert c.key_cache[0].shape[2] <= 16


@pytest.mark.parametrize("strategy,kw", [("budget", dict(max_kv_tokens=256)), ("every_chunk", {})])
def test_prefill_chunked_strategies(tiny, monkeypatch, strategy, kw):
    """tests/test_dropkv_triton.py:1083-1145: the final cache holds
    ``max(int(0.3 * L), 8, 1)`` rows per layer, all tokens were seen, and the
    mode flags are restored."""
    cfg, model = tiny
    L = 512
    ids = random_prompt(cfg.vocab_size, L, seed=9)
    c, _ = _chunked(model, ids, monkeypatch, chunk_size=128, evict_strategy=strategy, **kw)
    for k in c.key_cache:
        assert k.shape[2] == max(int(0.3 * L), 8, 1)
    assert c._seen_tokens == L
    assert (c._prefill_mode, c._evict_use_seen_tokens, c._budget_max_kv_tokens) == ("single_pass", False, None)


@pytest.mark.parametrize("strategy,kw", [("budget", dict(max_kv_tokens=256)), ("every_chunk", {}),
                                         ("last_chunk", {})])
def test_chunk_after_eviction_is_causal(tiny, monkeypatch, strategy, kw):
    """A chunk that follows an eviction attends causally in the stored frame:
    changing the prompt's last token leaves the next-to-last position's
    logits unchanged."""
    cfg, model = tiny
    ids = random_prompt(cfg.vocab_size, 512, seed=10)
    ids2 = ids.clone()
    ids2[0, -1] = (ids2[0, -1] + 1) % cfg.vocab_size
    _, out1 = _chunked(model, ids, monkeypatch, chunk_size=128, evict_strategy=strategy, logits_to_keep=2, **kw)
    _, out2 = _chunked(model, ids2, monkeypatch, chunk_size=128, evict_strategy=strategy, logits_to_keep=2, **kw)
    assert torch.equal(out1.logits[:, 0], out2.logits[:, 0])
    assert not torch.equal(out1.logits[:, 1], out2.logits[:, 1])


def test_hf5_update_forms_route_the_query(monkeypatch):
    """``update(key, value, layer_idx)`` (5.x) and ``update(key, value,
    layer_idx, cache_kwargs)`` (4.x) both reach the prefill branch with the
    query: from cache_kwargs first, else from the capture slot."""
    from dropkv_amd import hf_query
    seen = []

    def evict_layer(self, q, k, v, total_tokens=None, max_keep_len=None):
        seen.append(q)
        idx = torch.arange(k.shape[2] - 8, k.shape[2]).expand(k.shape[0], k.shape[1], 8)
        return R.gather_compressed(k, v, idx)
    monkeypatch.setattr(DropKVCache, "_evict_layer", evict_layer)
    q = torch.randn(1, 4, 32, 64)
    k = torch.randn(1, 2, 32, 64)
    c = DropKVCache(keep_ratio=0.1)
    hf_query._slot.query = q
    rk, rv = c.update(k, k, 0)
    assert seen[-1] is q and rk is k and c.key_cache[0].shape[2] == 8
    q2 = torch.randn(1, 4, 32, 64)
    hf_query._slot.query = torch.randn(1, 4, 32, 64)
    c.update(k, k, 1, {"query_states": q2})
    assert seen[-1] is q2
    assert hf_query.take_captured_query() is None    # consumed by the update
    with pytest.raises(TypeError, match="layer_idx"):
        c.update(q, k, k)
