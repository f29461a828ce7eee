"""Kernel timing through the C ABI (``dropkv_timing_*``): one duration per
kernel of the most recent call, taken from the dispatches' own begin/end
time stamps, so each lies inside the call's wall time and their sum does not
exceed it; nothing is timed while timing is off."""

import ctypes

import pytest
import torch

from conftest import LLAMA_CFG, make_qkv

pytestmark = pytest.mark.gpu


def _read(lib, buf):
    n = lib.dropkv_timing_read(buf, len(buf))
    assert n >= 0, "dropkv_timing_read failed"
    return [buf[i] for i in range(n)]


def test_timing_per_kernel(gpu):
    from dropkv_amd import _lib, ops
    lib = _lib.load()
    Q, K, V = make_qkv(LLAMA_CFG, 4096, device=gpu)
    plan = ops.EvictPlan(Q, K, 8, 11, 409)
    plan(Q, K, V)
    torch.cuda.synchronize()
    buf = (ctypes.c_double * 16)()
    _lib.check(lib.dropkv_timing_enable(1), "dropkv_timing_enable")
    try:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        plan(Q, K, V)
        end.record()
        ms = _read(lib, buf)
        torch.cuda.synchronize()
        wall = start.elapsed_time(end)
        # score pass 1, merge, score pass 2 with the whole selection in its tail
        assert len(ms) == 3
        assert all(0.0 < t < wall for t in ms), (ms, wall)
        assert sum(ms) <= wall * 1.001, (ms, wall)
        # the selection as its own kernels: pass 2 (+ pooling), threshold, emit + gather
        ops.set_tail_select(False)
        try:
            plan(Q, K, V)
            ms = _read(lib, buf)
        finally:
            ops.set_tail_select(True)
        assert len(ms) == 5 and all(t > 0.0 for t in ms), ms

        # decode: partials and merge
        B, Hq, Hkv, D, C = 1, 32, 8, 128, 256
        kb = torch.randn(B, Hkv, C, D, device=gpu).bfloat16()
        vb = torch.randn_like(kb)
        q = torch.randn(B, Hq, 1, D, device=gpu).bfloat16()
        kn, vn = kb[:, :, :1].clone(), vb[:, :, :1].clone()
        n_rows = torch.tensor([100], dtype=torch.int32, device=gpu)
        out = torch.empty(B, 1, Hq, D, dtype=torch.bfloat16, device=gpu)
        ops.decode_attention(q, kn, vn, kb, vb, n_rows, D ** -0.5, out, ops.decode_workspace(B, Hq, Hkv, D, C, gpu))
        assert len(_read(lib, buf)) == 2
    finally:
        lib.dropkv_timing_enable(0)
    plan(Q, K, V)
    torch.cuda.synchronize()
    assert _read(lib, buf) == []
