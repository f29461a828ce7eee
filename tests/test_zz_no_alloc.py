"""dropkv_evict_noalloc (the layer-call whose scratch is a static per-GPU
array, for callers that cannot allocate) against dropkv_evict with a
workspace: the same kept indices, compressed K/V and scores, bit for bit,
over consecutive calls on one GPU whose shapes shrink and grow again (the
scratch keeps the previous call's contents)."""

import ctypes

import pytest
import torch

from conftest import LLAMA_CFG, QWEN_CFG, make_qkv

pytestmark = pytest.mark.gpu


def _noalloc(lib, stream, Q, K, V, W, ks, keep, p_round=1, y_round=0):
    B, Hq, Lq, D = Q.shape
    Hkv, Lk = K.shape[1], K.shape[2]
    dev = Q.device
    scores = torch.full((B, Hkv, Lk), float("nan"), dtype=torch.float32, device=dev)
    idx = torch.full((B, Hkv, keep), -1, dtype=torch.int64, device=dev)
    ko = torch.zeros(B, Hkv, keep, D, dtype=K.dtype, device=dev)
    vo = torch.zeros_like(ko)
    rc = lib.dropkv_evict_noalloc(Q.data_ptr(), *Q.stride(), K.data_ptr(), V.data_ptr(), 1, B, Hq, Hkv, Lq, Lk,
                                  D, W, 1e-6, p_round, y_round, 0, ks, W, keep, scores.data_ptr(), idx.data_ptr(),
                                  ko.data_ptr(), vo.data_ptr(), stream)
    return rc, scores, idx, ko, vo


@pytest.mark.parametrize("order", ["shrink", "grow"])
def test_noalloc_matches_workspace_entry(gpu, order):
    from dropkv_amd import _lib, ops
    lib = _lib.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    cases = [(LLAMA_CFG, 4096, 11, 0.1, 1, 0), (QWEN_CFG, 1000, 7, 0.2, 1, 1), (LLAMA_CFG, 2048, 11, 0.1, 0, 0)]
    if order == "grow":
        cases = cases[::-1]
    for i, (cfg, L, ks, ratio, p_round, y_round) in enumerate(cases):
        W = 8
        print(f"[noalloc] call {i}: {cfg} L={L}", flush=True)
        Q, K, V = (t.to(gpu) for t in make_qkv(cfg, L, seed=40 + i))
        keep = min(L, max(int(ratio * L), W, 1))
        plan = ops.EvictPlan(Q, K, W, ks, keep, p_round=bool(p_round), y_round=bool(y_round), keep_scores=True)
        ref_idx, ref_k, ref_v = plan(Q, K, V)
        rc, s, idx, ko, vo = _noalloc(lib, stream, Q, K, V, W, ks, keep, p_round, y_round)
        _lib.check(rc, "dropkv_evict_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(idx, ref_idx), (i, "kept indices")
        assert torch.equal(ko, ref_k) and torch.equal(vo, ref_v), (i, "compressed K/V")
        assert torch.equal(s, plan.scores), (i, "scores")


def test_noalloc_scores_optional(gpu):
    """scores = NULL keeps them in the scratch; the selection is unchanged."""
    from dropkv_amd import _lib, ops
    lib = _lib.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    Q, K, V = (t.to(gpu) for t in make_qkv(LLAMA_CFG, 3000, seed=50))
    W, ks, keep = 8, 11, 300
    ref_idx, ref_k, ref_v = ops.EvictPlan(Q, K, W, ks, keep)(Q, K, V)
    idx = torch.empty(1, 8, keep, dtype=torch.int64, device=gpu)
    ko = torch.empty(1, 8, keep, 128, dtype=K.dtype, device=gpu)
    vo = torch.empty_like(ko)
    rc = lib.dropkv_evict_noalloc(Q.data_ptr(), *Q.stride(), K.data_ptr(), V.data_ptr(), 1, 1, 32, 8, 3000, 3000,
                                  128, W, 1e-6, 1, 0, 0, ks, W, keep, None, idx.data_ptr(), ko.data_ptr(),
                                  vo.data_ptr(), stream)
    _lib.check(rc, "dropkv_evict_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(idx, ref_idx) and torch.equal(ko, ref_k) and torch.equal(vo, ref_v)
