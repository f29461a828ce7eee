"""Host-side behaviour of DropKVCache / prefill_chunked / the scoring guards
that needs no GPU compute: constructor checks, prefill modes that only store,
length bookkeeping, HF 4-argument form, prefill_chunked validation, mode
schedule and cleanup on failure (reference tests:535-1330, :1831-1899), and
the absence of any CPU fallback in the product path.  CPU only."""

import logging

import pytest
import torch

from conftest import LLAMA_CFG, make_qkv
from dropkv_amd import DropKVCache, dropkv_scores_triton, ops, prefill_chunked
from dropkv_amd.dropkv_cache import _LayerCache


def _cache(**kw):
    d = dict(keep_ratio=0.3, window_size=8, kernel_size=11, use_triton=False)
    d.update(kw)
    return DropKVCache(**d)


# --- constructor (dropkv_cache.py:321-330) ---------------------------------

@pytest.mark.parametrize("kw,msg", [
    (dict(keep_ratio=0.0), "keep_ratio"), (dict(keep_ratio=1.5), "keep_ratio"),
    (dict(window_size=0), "window_size"), (dict(kernel_size=4), "kernel_size"),
    (dict(kernel_size=0), "kernel_size"),
])
def test_constructor_rejects(kw, msg):
    with pytest.raises(ValueError, match=msg):
        DropKVCache(**kw)


def test_defaults_and_mode_attributes():
    c = DropKVCache()
    assert (c.keep_ratio, c.window_size, c.kernel_size, c.use_triton) == (0.1, 8, 11, True)
    assert c._prefill_mode == "single_pass" and c._evict_use_seen_tokens is False
    assert c._budget_max_kv_tokens is None and c._seen_tokens == 0


def test_beam_search_unsupported():
    with pytest.raises(NotImplementedError):
        _cache().batch_split(2, 1)
    with pytest.raises(NotImplementedError):
        DropKVCache.from_batch_splits([])


# --- keep length (dropkv_cache.py:470-473) ----------------------------------

def test_keep_length():
    c = _cache(keep_ratio=0.3)
    assert c._keep_length(128, None, None) == 38
    assert c._keep_length(128, 512, None) == 128
    assert c._keep_length(128, 200, None) == 60
    assert _cache(keep_ratio=0.01)._keep_length(64, 10, None) == 8
    assert _cache(keep_ratio=0.8)._keep_length(512, 512, 100) == 100


# --- store-only prefill paths -----------------------------------------------

def test_accumulate_grows_cache_and_seen_tokens():
    Q, K, V = make_qkv(LLAMA_CFG, 64)
    c = _cache()
    c._prefill_mode = "accumulate"
    rk, _ = c.update(Q[:, :, :32], K[:, :, :32], V[:, :, :32], layer_idx=0)
    assert c.key_cache[0].shape[2] == 32 and rk.shape[2] == 32
    rk, rv = c.update(Q[:, :, 32:], K[:, :, 32:], V[:, :, 32:], layer_idx=0)
    assert c.key_cache[0].shape[2] == 64 and rk.shape[2] == 64
    assert torch.equal(c.key_cache[0], K) and torch.equal(c.value_cache[0], V)
    assert c._seen_tokens == 64


def test_seen_tokens_counted_on_layer_zero_only():
    Q, K, V = make_qkv(LLAMA_CFG, 16)
    c = _cache()
    c._prefill_mode = "accumulate"
    for layer in range(3):
        c.update(Q, K, V, layer_idx=layer)
    assert c._seen_tokens == 16 and len(c) == 3


def test_short_sequence_stored_without_eviction():
    Q, K, V = make_qkv(LLAMA_CFG, 6)
    c = _cache(window_size=8)
    rk, _ = c.update(Q, K, V, layer_idx=0)
    assert c.key_cache[0].shape[2] == 6 and rk is K


def test_hf_4arg_without_query_states_stores_full(caplog):
    _, K, V = make_qkv(LLAMA_CFG, 128)
    c = _cache()
    with caplog.at_level(logging.WARNING):
        c.update(K, V, 0, {"sin": None, "cos": None})
    assert c.key_cache[0].shape[2] == 128
    assert "without query_states" in caplog.text


def test_layer_gap_rejected():
    _, K, V = make_qkv(LLAMA_CFG, 16)
    with pytest.raises(ValueError, match="DynamicCache"):
        _cache().update(None, K, V, layer_idx=2)


@pytest.mark.parametrize("L", [128, 6])
def test_invalid_prefill_mode_raises(L):
    Q, K, V = make_qkv(LLAMA_CFG, L)
    c = _cache(window_size=16)
    c._prefill_mode = "typo_mode"
    with pytest.raises(ValueError, match="Invalid _prefill_mode"):
        c.update(Q, K, V, layer_idx=0)


def test_invalid_mode_on_continuation_path_raises():
    Q, K, V = make_qkv(LLAMA_CFG, 64)
    c = _cache()
    c._prefill_mode = "accumulate"
    c.update(Q, K, V, layer_idx=0)
    c._prefill_mode = "bogus"
    with pytest.raises(ValueError, match="Invalid _prefill_mode"):
        c.update(Q[:, :, :1], K[:, :, :1], V[:, :, :1], layer_idx=0)


def test_decode_append_single_pass_mode():
    Q, K, V = make_qkv(LLAMA_CFG, 40)
    c = _cache()
    c._prefill_mode = "accumulate"
    c.update(Q[:, :, :39], K[:, :, :39], V[:, :, :39], layer_idx=0)
    c._prefill_mode = "single_pass"
    rk, _ = c.update(Q[:, :, 39:], K[:, :, 39:], V[:, :, 39:], layer_idx=0)
    assert rk.shape[2] == 40 and c.key_cache[0].shape[2] == 40


def test_lengths_for_rope_and_mask():
    """get_seq_length = tokens seen (RoPE), get_mask_sizes = stored + q_len
    (dropkv_cache.py:624-648)."""
    Q, K, V = make_qkv(LLAMA_CFG, 50)
    c = _cache()
    assert c.get_seq_length() == 0
    assert c.get_mask_sizes(torch.arange(5), 0) == (5, 0)
    c._prefill_mode = "accumulate"
    c.update(Q, K, V, layer_idx=0)
    c.key_cache[0] = c.key_cache[0][:, :, :20]      # as after an eviction
    assert c.get_seq_length() == 50
    assert c.get_mask_sizes(torch.arange(1), 0) == (21, 0)
    assert c.get_seq_length(3) == 0


def test_legacy_round_trip_stores_without_eviction():
    _, K, V = make_qkv(LLAMA_CFG, 30)
    legacy = ((K, V), (K * 2, V * 2))
    c = DropKVCache.from_legacy_cache(legacy)
    assert len(c) == 2 and c._seen_tokens == 30
    out = c.to_legacy_cache()
    assert torch.equal(out[1][0], K * 2) and torch.equal(out[0][1], V)
    assert isinstance(c, _LayerCache)


# --- no CPU fallback in the product path ------------------------------------

def test_eviction_on_cpu_tensors_fails_loudly():
    """Scoring/selection/gather run only on the HIP kernels: CPU tensors are
    rejected with RuntimeError instead of silently computing on the CPU."""
    Q, K, V = make_qkv(LLAMA_CFG, 64)
    with pytest.raises(RuntimeError):
        _cache().update(Q, K, V, layer_idx=0)
    with pytest.raises(RuntimeError):
        ops.scores(Q, K, V, 8)
    with pytest.raises(RuntimeError):
        ops.select(torch.zeros(1, 2, 64), 11, 8, 10)
    with pytest.raises(RuntimeError):
        ops.compact(K, V, torch.zeros(1, 8, 4, dtype=torch.int64))


def test_head_dim_above_the_kernel_limit_fails_early():
    """A head dimension above the kernels' 4096 is refused with ValueError
    naming the limit, before any device work (CPU tensors would otherwise
    raise RuntimeError at the device check), in both cache modes."""
    cfg = dict(B=1, Hq=2, Hkv=1, D=4104)
    Q, K, V = make_qkv(cfg, 16)
    for c in (_cache(), DropKVCache(keep_ratio=0.5, window_size=8, capacity=64)):
        with pytest.raises(ValueError, match="above 4096"):
            c.update(Q, K, V, layer_idx=0)


def test_release_workspaces_empties_the_stream_cache():
    ops._shared_ws[("probe", 0)] = object()
    ops.release_workspaces()
    assert not ops._shared_ws


# --- scoring guards reachable without a GPU (dropkv_triton.py:680-693) -------

def test_guard_window_size():
    Q, K, V = make_qkv(LLAMA_CFG, 64)
    with pytest.raises(AssertionError, match="positive int"):
        dropkv_scores_triton(Q, K, V, window_size=0)


def test_guard_lengths():
    Q, K, V = make_qkv(LLAMA_CFG, 4)
    with pytest.raises(AssertionError, match="must be >= window_size"):
        dropkv_scores_triton(Q, K, V)
    Q, K, V = make_qkv(LLAMA_CFG, 6, 64)
    with pytest.raises(AssertionError, match=r"Lq.*must be >= window_size"):
        dropkv_scores_triton(Q, K, V)
    Q, _, _ = make_qkv(LLAMA_CFG, 64)
    _, K, V = make_qkv(LLAMA_CFG, 6)
    with pytest.raises(AssertionError, match=r"Lk.*must be >= window_size"):
        dropkv_scores_triton(Q[:, :, :8], K, V)
    Q, K, V = make_qkv(LLAMA_CFG, 64, 32)
    with pytest.raises(AssertionError, match=r"Lq.*must be <= Lk"):
        dropkv_scores_triton(Q, K, V)


def test_guard_divisible_and_device():
    Q = torch.randn(1, 7, 64, 128, dtype=torch.bfloat16)
    K = torch.randn(1, 4, 64, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="divisible"):
        dropkv_scores_triton(Q, K, K)
    Q, K, V = make_qkv(LLAMA_CFG, 64)
    with pytest.raises(AssertionError, match="CUDA"):
        dropkv_scores_triton(Q, K, V)


def test_fast_path_guard_falls_back_to_deployed_semantics(monkeypatch):
    """_compute_keep_indices catches AssertionError from the fast path and
    uses the deployed-path scoring (dropkv_cache.py:389-400); a RuntimeError
    propagates (reference tests:1944-1945)."""
    import dropkv_amd.dropkv_cache as C
    calls = []

    def fast(*a, **k):
        calls.append("fast")
        raise AssertionError("guard")

    def deployed(q, k, v, w):
        calls.append(("deployed", w))
        return torch.zeros(k.shape[0], k.shape[1], k.shape[2])

    monkeypatch.setattr("dropkv_amd.dropkv_triton.dropkv_scores_triton", fast)
    monkeypatch.setattr(C, "_deployed_path_scores", deployed)
    monkeypatch.setattr(C.ops, "select", lambda s, ks, w, keep: ("select", ks, w, keep))
    Q, K, V = make_qkv(LLAMA_CFG, 64)
    c = _cache(use_triton=True)
    assert c._compute_keep_indices(Q, K, V) == ("select", 11, 8, 19)
    assert calls == ["fast", ("deployed", 8)]

    def boom(*a, **k):
        raise RuntimeError("kernel failure")

    monkeypatch.setattr("dropkv_amd.dropkv_triton.dropkv_scores_triton", boom)
    with pytest.raises(RuntimeError, match="kernel failure"):
        c._compute_keep_indices(Q, K, V)


def test_update_evicts_in_one_fused_call(monkeypatch):
    """update() runs _compute_keep_indices + _gather_compressed as one
    ops.evict call (score, pool, protect, top-k, sort, gather) with the same
    choice of scoring semantics: the fast path's (W = window, y in fp32) when
    its guards pass, else the deployed path's (W = min(window, Lq), y rounded
    to the input dtype), and the same keep length and protection."""
    import dropkv_amd.dropkv_cache as C
    import dropkv_amd.dropkv_triton as T
    calls = []

    def evict(q, k, v, W, ks, keep, protect_window=None, eps=1e-6, p_round=True, y_round=False, splits=0):
        calls.append((W, ks, keep, protect_window, p_round, y_round))
        idx = torch.arange(keep).expand(k.shape[0], k.shape[1], keep)
        return idx, k[:, :, :keep], v[:, :, :keep]

    monkeypatch.setattr(C.ops, "evict", evict)
    Q, K, V = make_qkv(LLAMA_CFG, 64)
    c = _cache(use_triton=True)          # CPU tensors fail the fast-path guard
    c.update(Q[:, :, -4:], K, V, layer_idx=0)
    assert calls[-1] == (4, 11, 19, 8, True, True)
    assert c.key_cache[0].shape[2] == 19
    monkeypatch.setattr(T, "check_scoring_inputs", lambda *a, **k: None)   # guards pass
    c.update(Q, K, V, layer_idx=1)
    assert calls[-1] == (8, 11, 19, 8, True, False)
    c2 = _cache(use_triton=False)
    c2.update(Q, K, V, layer_idx=0)
    assert calls[-1] == (8, 11, 19, 8, True, True)
    # evict_accumulated: stored || chunk, keep from the tokens seen
    c2._prefill_mode = "evict_accumulated"
    c2._evict_use_seen_tokens = True
    rk, _ = c2.update(Q[:, :, :32], K[:, :, :32], V[:, :, :32], layer_idx=0)
    assert rk.shape[2] == 19 + 32 and calls[-1] == (8, 11, int(0.3 * 96), 8, True, True)


# --- prefill_chunked (dropkv_cache.py:651-807) --------------------------------

def test_prefill_chunked_rejects_wrong_cache_type():
    with pytest.raises(TypeError, match="DropKVCache"):
        prefill_chunked(object(), torch.zeros(1, 100), object())


def test_prefill_chunked_rejects_populated_cache():
    c = _cache()
    c.key_cache.append(torch.zeros(1, 8, 10, 128))
    c.value_cache.append(torch.zeros(1, 8, 10, 128))
    with pytest.raises(ValueError, match="fresh.*empty.*cache"):
        prefill_chunked(object(), torch.zeros(1, 100), c)


@pytest.mark.parametrize("kw,msg", [
    (dict(chunk_size=4), "chunk_size.*window_size"),
    (dict(chunk_size=32, attention_mask=torch.ones(1, 100)), "sequence-shaped"),
    (dict(chunk_size=32, evict_strategy="invalid"), "evict_strategy"),
    (dict(chunk_size=32, evict_strategy="budget", max_kv_tokens=4), "window_size"),
    (dict(chunk_size=32, evict_strategy="budget", max_kv_tokens=None), "max_kv_tokens is required"),
])
def test_prefill_chunked_validation(kw, msg):
    with pytest.raises(ValueError, match=msg):
        prefill_chunked(object(), torch.zeros(1, 100), _cache(), **kw)


class BrokenModel:
    def __call__(self, *args, **kwargs):
        raise RuntimeError("simulated failure")


@pytest.mark.parametrize("kw", [dict(chunk_size=32), dict(chunk_size=32, evict_strategy="budget", max_kv_tokens=64)])
def test_prefill_chunked_cleans_up_on_error(kw):
    c = _cache()
    with pytest.raises(RuntimeError, match="simulated failure"):
        prefill_chunked(BrokenModel(), torch.zeros(1, 100), c, **kw)
    assert c._prefill_mode == "single_pass" and c._evict_use_seen_tokens is False
    assert c._budget_max_kv_tokens is None
    assert len(c.key_cache) == 0 and len(c.value_cache) == 0 and c._seen_tokens == 0


def test_cleanup_after_mid_forward_failure():
    calls = 0

    class FailAfterFirst:
        def __call__(self, chunk, past_key_values=None, **kw):
            nonlocal calls
            calls += 1
            if calls > 1:
                raise RuntimeError("OOM on chunk 2")
            Q, K, V = make_qkv(LLAMA_CFG, chunk.shape[1])
            for layer in range(2):
                past_key_values.update(Q, K, V, layer_idx=layer)
            return "out"

    c = _cache()
    with pytest.raises(RuntimeError, match="OOM on chunk 2"):
        prefill_chunked(FailAfterFirst(), torch.zeros(1, 100), c, chunk_size=32)
    assert len(c.key_cache) == 0 and c._seen_tokens == 0 and c._prefill_mode == "single_pass"


class RecordingModel:
    """Records the cache mode per chunk; stores K/V lengths like a model would
    (accumulate: append; evict modes: the keep length the cache would keep)."""

    def __init__(self):
        self.log = []

    def __call__(self, chunk, past_key_values=None, use_cache=True, **kw):
        c = past_key_values
        n = chunk.shape[1]
        self.log.append((c._prefill_mode, c._evict_use_seen_tokens, c._budget_max_kv_tokens, n))
        c._seen_tokens += n
        stored = c.key_cache[0].shape[2] if c.key_cache else 0
        if c._prefill_mode == "accumulate":
            new = stored + n
        else:
            total = stored + n
            base = c._seen_tokens if c._evict_use_seen_tokens else total
            new = c._keep_length(total, base if c._evict_use_seen_tokens else None, c._budget_max_kv_tokens)
        t = torch.zeros(1, 1, new, 1)
        if c.key_cache:
            c.key_cache[0], c.value_cache[0] = t, t
        else:
            c.key_cache.append(t)
            c.value_cache.append(t)
        return self.log[-1]


def test_prefill_chunked_schedule_last_chunk():
    m = RecordingModel()
    c = _cache()
    prefill_chunked(m, torch.zeros(1, 100, dtype=torch.long), c, chunk_size=32)
    assert [e[0] for e in m.log] == ["accumulate"] * 3 + ["evict_accumulated"]
    assert all(e[1] is False and e[2] is None for e in m.log)
    assert [e[3] for e in m.log] == [32, 32, 32, 4]
    assert c._prefill_mode == "single_pass"


def test_prefill_chunked_schedule_every_chunk():
    m = RecordingModel()
    prefill_chunked(m, torch.zeros(1, 100, dtype=torch.long), _cache(), chunk_size=32, evict_strategy="every_chunk")
    assert [e[0] for e in m.log] == ["single_pass"] + ["evict_accumulated"] * 3
    assert all(e[1] is True for e in m.log)


def test_prefill_chunked_schedule_budget():
    m = RecordingModel()
    c = _cache(keep_ratio=0.3)
    prefill_chunked(m, torch.zeros(1, 256, dtype=torch.long), c, chunk_size=64, evict_strategy="budget",
                    max_kv_tokens=128)
    modes = [e[0] for e in m.log]
    # 64 -> 128 (at budget, not over) -> 192 > 128: evict -> ... last: evict
    assert modes[:3] == ["accumulate", "accumulate", "evict_accumulated"]
    assert modes[-1] == "evict_accumulated"
    assert all(e[2] == 128 for e in m.log)
    assert c._budget_max_kv_tokens is None and c._evict_use_seen_tokens is False


def test_prefill_chunked_single_chunk_shortcut():
    m = RecordingModel()
    c = _cache()
    prefill_chunked(m, torch.zeros(1, 30, dtype=torch.long), c, chunk_size=32)
    assert [e[0] for e in m.log] == ["single_pass"]


def test_capacity_must_be_positive():
    from dropkv_amd import DropKVCache
    with pytest.raises(ValueError, match="capacity"):
        DropKVCache(capacity=0)
    assert DropKVCache(capacity=128).capacity == 128
    assert DropKVCache().capacity is None


def test_capacity_prefill_keep_above_capacity_raises():
    """A prefill eviction whose keep length exceeds the capacity raises the
    documented ValueError before anything is enqueued (also with CPU
    tensors, where no kernel could run)."""
    from dropkv_amd import DropKVCache
    Q, K, V = make_qkv(LLAMA_CFG, 256, seed=6)
    c = DropKVCache(keep_ratio=0.9, capacity=200)
    with pytest.raises(ValueError, match="capacity of 200 rows exceeded at layer 0: 230 rows needed"):
        c.update(Q, K, V, layer_idx=0)


def test_cat_rows_falls_back_to_torch_cat_off_the_gpu():
    """Off the GPU (and for shapes the append kernel does not take) the
    continuation's append is torch.cat itself, so host flows keep the
    reference's tensors."""
    from dropkv_amd.dropkv_cache import cat_rows
    g = torch.Generator().manual_seed(0)
    k0, v0 = torch.randn(1, 2, 5, 8, generator=g), torch.randn(1, 2, 5, 8, generator=g)
    k1, v1 = torch.randn(1, 2, 3, 8, generator=g), torch.randn(1, 2, 3, 8, generator=g)
    k, v = cat_rows(k0, v0, k1, v1)
    assert torch.equal(k, torch.cat([k0, k1], dim=-2)) and torch.equal(v, torch.cat([v0, v1], dim=-2))
    # inputs autograd tracks keep torch.cat's graph
    k, v = cat_rows(k0.requires_grad_(), v0, k1, v1)
    assert k.grad_fn is not None
