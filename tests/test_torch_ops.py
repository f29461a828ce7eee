"""``torch.ops.dropkv``: the scorer and the layer-call registered with the
dispatcher, with fake kernels, so that ``torch.compile`` traces callers
without a graph break.  CPU: schemas, fake shapes on meta tensors, and a
full-graph trace.  GPU: compiled callers equal the eager ctypes path."""

import pytest
import torch

import dropkv_amd  # noqa: F401  (registers the operators)
from conftest import make_qkv


def _meta_qkv(B=1, Hq=8, Hkv=2, Lq=64, Lk=512, D=128):
    q = torch.empty(B, Hq, Lq, D, device="meta", dtype=torch.bfloat16)
    k = torch.empty(B, Hkv, Lk, D, device="meta", dtype=torch.bfloat16)
    return q, k, torch.empty_like(k)


def test_schemas():
    s = str(torch.ops.dropkv.scores.default._schema)
    e = str(torch.ops.dropkv.evict.default._schema)
    assert s.startswith("dropkv::scores(Tensor q, Tensor k, Tensor v, SymInt window") and s.endswith("-> Tensor")
    assert "SymInt keep" in e and e.endswith("-> (Tensor, Tensor, Tensor)")


def test_fake_shapes_on_meta():
    q, k, v = _meta_qkv()
    s = torch.ops.dropkv.scores(q, k, v, 8)
    assert s.shape == (1, 2, 512) and s.dtype == torch.float32 and s.device.type == "meta"
    idx, ko, vo = torch.ops.dropkv.evict(q, k, v, 8, 11, 100, 8)
    assert idx.shape == (1, 2, 100) and idx.dtype == torch.int64
    assert ko.shape == vo.shape == (1, 2, 100, 128) and ko.dtype == torch.bfloat16
    sidx, pooled = torch.ops.dropkv.select(s, 11, 8, 100)
    assert sidx.shape == (1, 2, 100) and sidx.dtype == torch.int64 and pooled.shape == s.shape
    ck, cv = torch.ops.dropkv.compact(k, v, sidx)
    assert ck.shape == cv.shape == (1, 2, 100, 128)


def test_full_graph_trace_on_meta():
    """dynamo traces a caller of both operators as one graph (no break)."""
    def fn(q, k, v):
        s = torch.ops.dropkv.scores(q, k, v, 8)
        idx, ko, vo = torch.ops.dropkv.evict(q, k, v, 8, 11, 100, 8)
        return s.sum(-1), idx, ko + 1
    q, k, v = _meta_qkv()
    explanation = torch._dynamo.explain(fn)(q, k, v)
    assert explanation.graph_break_count == 0 and explanation.graph_count == 1


@pytest.mark.gpu
def test_operators_match_ops(gpu):
    """Each operator returns what the ctypes wrapper returns, bit for bit."""
    from dropkv_amd import ops
    Q, K, V = make_qkv(dict(B=1, Hq=8, Hkv=2, D=128), 128, 2048, seed=5)
    Q, K, V = Q.to(gpu), K.to(gpu), V.to(gpu)
    s = torch.ops.dropkv.scores(Q, K, V, 8)
    assert torch.equal(s, ops.scores(Q, K, V, 8))
    idx, pooled = torch.ops.dropkv.select(s, 11, 8, 204)
    ridx, rpooled = ops.select(s, 11, 8, 204, return_pooled=True)
    assert torch.equal(idx, ridx) and torch.equal(pooled, rpooled)
    ko, vo = torch.ops.dropkv.compact(K, V, idx)
    rk, rv = ops.compact(K, V, idx)
    assert torch.equal(ko, rk) and torch.equal(vo, rv)
    e = torch.ops.dropkv.evict(Q, K, V, 8, 11, 204, 8)
    r = ops.evict(Q, K, V, 8, 11, 204, protect_window=8)
    assert all(torch.equal(a, b) for a, b in zip(e, r))


@pytest.mark.gpu
def test_compiled_scorer_matches_eager(gpu):
    from dropkv_amd import dropkv_scores_triton
    Q, K, V = make_qkv(dict(B=1, Hq=8, Hkv=2, D=128), 256, 1024, seed=3)
    Q, K, V = Q.to(gpu), K.to(gpu), V.to(gpu)
    eager = dropkv_scores_triton(Q, K, V)
    compiled = torch.compile(lambda q, k, v: dropkv_scores_triton(q, k, v), backend="aot_eager", fullgraph=True)
    assert torch.equal(compiled(Q, K, V), eager)


@pytest.mark.gpu
def test_compiled_cache_layer_call_matches_eager(gpu):
    """DropKVCache's fused layer-call traced by torch.compile (full graph)
    returns the eager call's compressed K/V bit for bit."""
    from dropkv_amd import DropKVCache
    Q, K, V = make_qkv(dict(B=1, Hq=8, Hkv=2, D=64), 512, seed=4)
    Q, K, V = Q.to(gpu), K.to(gpu), V.to(gpu)
    cache = DropKVCache(keep_ratio=0.25, window_size=8, kernel_size=11)
    ek, ev = cache._evict_layer(Q, K, V)
    compiled = torch.compile(cache._evict_layer, backend="aot_eager", fullgraph=True)
    ck, cv = compiled(Q, K, V)
    assert torch.equal(ck, ek) and torch.equal(cv, ev)
