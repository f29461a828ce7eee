"""Torch-tensor wrappers around the C ABI of libdropkv_amd.so.

PyTorch provides device memory (its caching allocator, also for the
workspaces) and the current HIP stream; all arithmetic runs in the HIP
kernels.  The wrappers check what the kernels assume (device, dtype, layout,
alignment) and raise ``RuntimeError`` otherwise; the reference-compatible
``AssertionError`` guards live in :mod:`dropkv_amd.dropkv_triton`.
"""

from __future__ import annotations

import threading

import torch

from . import _lib

_DTYPE_CODE = {torch.bfloat16: _lib.DROPKV_BF16, torch.float16: _lib.DROPKV_FP16, torch.float32: _lib.DROPKV_FP32}


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device) -> int:
    """The current stream of ``dev`` as a raw handle (the raw getter takes
    ~0.1 us where building a torch Stream object takes ~2 us per call)."""
    if _raw_stream is not None and dev.index is not None:
        return _raw_stream(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


def _workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def _evict_workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    """A new ``dropkv_scores`` / ``dropkv_evict`` workspace: its leading
    counters (_lib.SYNC_BYTES) start at zero, and every call leaves them zero."""
    ws = _workspace(nbytes, dev)
    ws[: _lib.SYNC_BYTES].zero_()
    return ws


# One workspace per (device, stream), grown on demand and reused by every
# ``scores`` / ``evict`` call on that stream: calls on one stream run in
# order, so they never use it at the same time.
_shared_ws: dict = {}
_shared_ws_lock = threading.Lock()


def _stream_workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    nbytes = max(int(nbytes), 1)
    if torch.cuda.is_current_stream_capturing():
        return _evict_workspace(nbytes, dev)  # a graph keeps its own (private-pool) workspace
    key = (dev.index, _stream(dev))
    with _shared_ws_lock:
        ws = _shared_ws.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = _evict_workspace(nbytes, dev)
            _shared_ws[key] = ws
    return ws


def release_workspaces() -> None:
    """Drop the per-(device, stream) workspaces kept for calls that bring
    none (they only grow, to the largest call seen on that stream, and are
    otherwise held for the life of the process).  Each goes back to
    PyTorch's caching allocator, which orders its reuse after the work
    already enqueued on its stream (``torch.cuda.empty_cache()`` can then
    return it to the device); the next call allocates a fresh workspace."""
    with _shared_ws_lock:
        _shared_ws.clear()


def _aligned(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def _kv_operand(t: torch.Tensor) -> torch.Tensor:
    """K/V must be contiguous and 16-byte aligned for the vector loads."""
    if not t.is_contiguous() or not _aligned(t):
        t = t.contiguous() if not t.is_contiguous() else t.clone()
    return t


def _check_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    if dev.type != "cuda":
        raise RuntimeError("DropKV HIP ops need tensors on a ROCm (cuda) device")
    for t in ts[1:]:
        if t.device != dev:
            raise RuntimeError("all tensors must be on the same device")
    return dev


def scores(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, window: int, eps: float = 1e-6,
           p_round: bool = True, y_round: bool = False, splits: int = 0,
           return_workspace: bool = False):
    """Per-key DropKV scores [B, Hkv, Lk] fp32 (see ``dropkv_scores`` in the C ABI)."""
    dev = _check_device(Q, K, V)
    if Q.dtype not in _DTYPE_CODE or K.dtype != Q.dtype or V.dtype != Q.dtype:
        raise RuntimeError(f"unsupported dtype combination {Q.dtype}/{K.dtype}/{V.dtype}")
    B, Hq, Lq, D = Q.shape
    Hkv, Lk = K.shape[1], K.shape[2]
    K = _kv_operand(K)
    V = _kv_operand(V)
    lib = _lib.load()
    ws_bytes = lib.dropkv_scores_workspace_bytes(B, Hq, Hkv, Lk, D, window, splits)
    ws = _evict_workspace(ws_bytes, dev) if return_workspace else _stream_workspace(ws_bytes, dev)
    out = torch.empty(B, Hkv, Lk, dtype=torch.float32, device=dev)
    rc = lib.dropkv_scores(Q.data_ptr(), *Q.stride(), K.data_ptr(), V.data_ptr(), _DTYPE_CODE[Q.dtype],
                           B, Hq, Hkv, Lq, Lk, D, window, float(eps), int(bool(p_round)), int(bool(y_round)),
                           int(splits), out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
    _lib.check(rc, "dropkv_scores")
    if return_workspace:
        return out, ws
    return out


def scores_debug_state(ws: torch.Tensor, B: int, Hq: int, Hkv: int, Lk: int, D: int, window: int,
                       splits: int = 0):
    """(lse [B,Hkv,M] natural log, y [B,Hkv,M,D] fp32) left in a scoring workspace."""
    dev = ws.device
    M = (Hq // Hkv) * window
    lse = torch.empty(B, Hkv, M, dtype=torch.float32, device=dev)
    y = torch.empty(B, Hkv, M, D, dtype=torch.float32, device=dev)
    rc = _lib.load().dropkv_scores_debug_state(ws.data_ptr(), B, Hq, Hkv, Lk, D, window, splits,
                                               lse.data_ptr(), y.data_ptr(), _stream(dev))
    _lib.check(rc, "dropkv_scores_debug_state")
    return lse, y


def select(scores_t: torch.Tensor, kernel_size: int, window: int, keep: int, return_pooled: bool = False):
    """Pool, protect, top-k and sort: int64 indices [..., keep], ascending."""
    dev = _check_device(scores_t)
    if scores_t.dtype != torch.float32:
        raise RuntimeError("select expects fp32 scores")
    s = scores_t.contiguous()
    Lk = s.shape[-1]
    rows = s.numel() // Lk
    lib = _lib.load()
    ws = _workspace(lib.dropkv_select_workspace_bytes(rows, Lk), dev)
    idx = torch.empty(*s.shape[:-1], keep, dtype=torch.int64, device=dev)
    pooled = torch.empty_like(s) if return_pooled else None
    rc = lib.dropkv_select(s.data_ptr(), rows, Lk, kernel_size, window, keep, idx.data_ptr(),
                           pooled.data_ptr() if pooled is not None else None, ws.data_ptr(), ws.numel(),
                           _stream(dev))
    _lib.check(rc, "dropkv_select")
    if return_pooled:
        return idx, pooled
    return idx


def _seg_strides(t: torch.Tensor):
    if t.stride(3) != 1:
        raise RuntimeError("the head-dim axis of K/V must be contiguous")
    return t.stride(0), t.stride(1), t.stride(2)


def compact(K: torch.Tensor, V: torch.Tensor, idx: torch.Tensor):
    """Bit-exact gather of rows ``idx`` [B,H,keep] from K/V [B,H,L,D]."""
    dev = _check_device(K, V, idx)
    if K.shape != V.shape or K.stride() != V.stride() or K.dtype != V.dtype:
        raise RuntimeError("K and V must have the same shape, strides and dtype")
    if K.stride(3) != 1:
        K, V = K.contiguous(), V.contiguous()
    idx = idx.to(torch.int64).contiguous()
    B, H, L, D = K.shape
    keep = idx.shape[-1]
    ko = torch.empty(B, H, keep, D, dtype=K.dtype, device=dev)
    vo = torch.empty_like(ko)
    rc = _lib.load().dropkv_compact(K.data_ptr(), V.data_ptr(), *_seg_strides(K), K.element_size(), B, H, L, D,
                                    idx.data_ptr(), keep, ko.data_ptr(), vo.data_ptr(), _stream(dev))
    _lib.check(rc, "dropkv_compact")
    return ko, vo


def compact2(K0: torch.Tensor, V0: torch.Tensor, K1: torch.Tensor, V1: torch.Tensor, idx: torch.Tensor):
    """Gather from the logical concatenation [K0 | K1] along the sequence axis."""
    dev = _check_device(K0, V0, K1, V1, idx)
    if K0.stride(3) != 1 or V0.stride(3) != 1:
        K0, V0 = K0.contiguous(), V0.contiguous()
    if K1.stride(3) != 1 or V1.stride(3) != 1:
        K1, V1 = K1.contiguous(), V1.contiguous()
    if K0.stride() != V0.stride() or K1.stride() != V1.stride():
        K0, V0, K1, V1 = K0.contiguous(), V0.contiguous(), K1.contiguous(), V1.contiguous()
    idx = idx.to(torch.int64).contiguous()
    B, H, L0, D = K0.shape
    L1 = K1.shape[2]
    keep = idx.shape[-1]
    ko = torch.empty(B, H, keep, D, dtype=K0.dtype, device=dev)
    vo = torch.empty_like(ko)
    rc = _lib.load().dropkv_compact2(K0.data_ptr(), V0.data_ptr(), *_seg_strides(K0), L0,
                                     K1.data_ptr(), V1.data_ptr(), *_seg_strides(K1), L1,
                                     K0.element_size(), B, H, D, idx.data_ptr(), keep, ko.data_ptr(),
                                     vo.data_ptr(), _stream(dev))
    _lib.check(rc, "dropkv_compact2")
    return ko, vo


def _check_buffer(buf: torch.Tensor, name: str):
    if buf.dim() != 4 or not buf.is_contiguous() or not _aligned(buf):
        raise RuntimeError(f"{name} must be a contiguous, 16-byte aligned [B, H, capacity, D] buffer")


def append(K: torch.Tensor, V: torch.Tensor, k_buf: torch.Tensor, v_buf: torch.Tensor, row0: int):
    """Copy K/V [B, H, L, D] (any strides, head dim contiguous) bit for bit
    to rows ``row0 .. row0+L-1`` of the [B, H, capacity, D] buffers
    (``dropkv_append``)."""
    dev = _check_device(K, V, k_buf, v_buf)
    _check_buffer(k_buf, "k_buf")
    _check_buffer(v_buf, "v_buf")
    if K.shape != V.shape or K.dtype != V.dtype or k_buf.shape != v_buf.shape:
        raise RuntimeError("K/V and the buffers must match in shape and dtype")
    if K.dtype != k_buf.dtype or K.shape[:2] != k_buf.shape[:2] or K.shape[3] != k_buf.shape[3]:
        raise RuntimeError("K/V do not fit the buffers")
    if K.stride(3) != 1 or V.stride(3) != 1 or K.stride() != V.stride():
        K, V = K.contiguous(), V.contiguous()
    B, H, L, D = K.shape
    rc = _lib.load().dropkv_append(K.data_ptr(), V.data_ptr(), *_seg_strides(K), K.element_size(), B, H, L, D,
                                   k_buf.data_ptr(), v_buf.data_ptr(), k_buf.shape[2], int(row0), _stream(dev))
    _lib.check(rc, "dropkv_append")


def evict_ld(Q: torch.Tensor, k_buf: torch.Tensor, v_buf: torch.Tensor, Lk: int, window: int, kernel_size: int,
             keep: int, k_out: torch.Tensor, v_out: torch.Tensor, protect_window: int | None = None,
             eps: float = 1e-6, p_round: bool = True, y_round: bool = False) -> torch.Tensor:
    """One layer-call (``dropkv_evict_ld``) on K/V held in rows 0 .. Lk-1 of
    [B, Hkv, capacity, D] buffers, writing the compressed rows to rows
    0 .. keep-1 of the ``k_out`` / ``v_out`` buffers.  Returns the kept
    indices [B, Hkv, keep] (ascending)."""
    dev = _check_device(Q, k_buf, v_buf, k_out, v_out)
    for t, n in ((k_buf, "k_buf"), (v_buf, "v_buf"), (k_out, "k_out"), (v_out, "v_out")):
        _check_buffer(t, n)
    if Q.dtype not in _DTYPE_CODE or k_buf.dtype != Q.dtype or v_buf.dtype != Q.dtype or k_out.dtype != Q.dtype:
        raise RuntimeError("Q, the K/V buffers and the outputs must share a bf16/fp16 dtype")
    if k_buf.shape != v_buf.shape or k_out.shape != v_out.shape:
        raise RuntimeError("K and V buffers must have the same shape")
    B, Hq, Lq, D = Q.shape
    Hkv = k_buf.shape[1]
    lib = _lib.load()
    ws = _stream_workspace(lib.dropkv_evict_workspace_bytes(B, Hq, Hkv, Lk, D, window, 0), dev)
    idx = torch.empty(B, Hkv, keep, dtype=torch.int64, device=dev)
    pw = window if protect_window is None else protect_window
    rc = lib.dropkv_evict_ld(Q.data_ptr(), *Q.stride(), k_buf.data_ptr(), v_buf.data_ptr(), k_buf.shape[2],
                             _DTYPE_CODE[Q.dtype], B, Hq, Hkv, Lq, int(Lk), D, int(window), float(eps),
                             int(bool(p_round)), int(bool(y_round)), 0, int(kernel_size), int(pw), int(keep), None,
                             idx.data_ptr(), k_out.data_ptr(), v_out.data_ptr(), k_out.shape[2], ws.data_ptr(),
                             ws.numel(), _stream(dev))
    _lib.check(rc, "dropkv_evict_ld")
    return idx


def evict(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, window: int, kernel_size: int, keep: int,
          protect_window: int | None = None, eps: float = 1e-6, p_round: bool = True, y_round: bool = False,
          splits: int = 0):
    """One layer-call (``dropkv_evict``): score, pool, protect, top-k, sort and
    gather in one call.  Returns fresh ``(keep_idx [B,Hkv,keep] int64,
    k_out, v_out [B,Hkv,keep,D])``, like the reference's
    ``_compute_keep_indices`` + ``_gather_compressed``; the workspace is the
    current stream's shared one."""
    dev = _check_device(Q, K, V)
    if Q.dtype not in _DTYPE_CODE or K.dtype != Q.dtype or V.dtype != Q.dtype:
        raise RuntimeError(f"unsupported dtype combination {Q.dtype}/{K.dtype}/{V.dtype}")
    if K.shape != V.shape:
        raise RuntimeError("K and V must have the same shape")
    B, Hq, Lq, D = Q.shape
    Hkv, Lk = K.shape[1], K.shape[2]
    K = _kv_operand(K)
    V = _kv_operand(V)
    lib = _lib.load()
    ws = _stream_workspace(lib.dropkv_evict_workspace_bytes(B, Hq, Hkv, Lk, D, window, splits), dev)
    idx = torch.empty(B, Hkv, keep, dtype=torch.int64, device=dev)
    ko = torch.empty(B, Hkv, keep, D, dtype=K.dtype, device=dev)
    vo = torch.empty_like(ko)
    pw = window if protect_window is None else protect_window
    rc = lib.dropkv_evict(Q.data_ptr(), *Q.stride(), K.data_ptr(), V.data_ptr(), _DTYPE_CODE[Q.dtype],
                          B, Hq, Hkv, Lq, Lk, D, int(window), float(eps), int(bool(p_round)), int(bool(y_round)),
                          int(splits), int(kernel_size), int(pw), int(keep), None, idx.data_ptr(), ko.data_ptr(),
                          vo.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev))
    _lib.check(rc, "dropkv_evict")
    return idx, ko, vo


def set_tail_select(enabled: bool = True, spin_polls: int = -1, spin_polls_b: int = -1) -> None:
    """``dropkv_set_tail_select``: whether layer-calls finish their selection
    (threshold, ordered emit, K/V gather) in the scoring kernel's tail when
    the call allows it (on by default) or always in two further kernels; the
    polls a workgroup waits at the tail's first barrier before it leaves its
    row to the last one to arrive (``spin_polls``), and at the second barrier
    before it finishes the row alone (``spin_polls_b``); < 0 leaves a limit
    unchanged, 0 forces that path.  Same results every way."""
    _lib.check(_lib.load().dropkv_set_tail_select(int(bool(enabled)), int(spin_polls), int(spin_polls_b)),
               "dropkv_set_tail_select")


class EvictPlan:
    """Pre-sized workspace and outputs for repeated layer-calls of one shape
    (``dropkv_evict``); avoids per-call allocation in tight loops."""

    def __init__(self, Q: torch.Tensor, K: torch.Tensor, window: int, kernel_size: int, keep: int,
                 protect_window: int | None = None, eps: float = 1e-6, p_round: bool = True,
                 y_round: bool = False, splits: int = 0, keep_scores: bool = False):
        dev = _check_device(Q, K)
        B, Hq, Lq, D = Q.shape
        Hkv, Lk = K.shape[1], K.shape[2]
        self.shape = (B, Hq, Hkv, Lq, Lk, D)
        self.dtype = Q.dtype
        self.window, self.kernel_size, self.keep = int(window), int(kernel_size), int(keep)
        self.protect_window = int(window if protect_window is None else protect_window)
        self.eps, self.p_round, self.y_round, self.splits = float(eps), int(p_round), int(y_round), int(splits)
        lib = _lib.load()
        self.ws = _evict_workspace(lib.dropkv_evict_workspace_bytes(B, Hq, Hkv, Lk, D, window, splits), dev)
        self.scores = torch.empty(B, Hkv, Lk, dtype=torch.float32, device=dev) if keep_scores else None
        self.keep_idx = torch.empty(B, Hkv, keep, dtype=torch.int64, device=dev)
        self.k_out = torch.empty(B, Hkv, keep, D, dtype=Q.dtype, device=dev)
        self.v_out = torch.empty_like(self.k_out)
        self.dev = dev

    def __call__(self, Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor):
        B, Hq, Hkv, Lq, Lk, D = self.shape
        if tuple(Q.shape) != (B, Hq, Lq, D) or tuple(K.shape) != (B, Hkv, Lk, D) or K.shape != V.shape:
            raise RuntimeError("input shapes differ from the plan")
        if Q.dtype != self.dtype or K.dtype != self.dtype or V.dtype != self.dtype:
            raise RuntimeError("input dtype differs from the plan")
        K = _kv_operand(K)
        V = _kv_operand(V)
        rc = _lib.load().dropkv_evict(
            Q.data_ptr(), *Q.stride(), K.data_ptr(), V.data_ptr(), _DTYPE_CODE[self.dtype],
            B, Hq, Hkv, Lq, Lk, D, self.window, self.eps, self.p_round, self.y_round, self.splits,
            self.kernel_size, self.protect_window, self.keep,
            self.scores.data_ptr() if self.scores is not None else None, self.keep_idx.data_ptr(),
            self.k_out.data_ptr(), self.v_out.data_ptr(), self.ws.data_ptr(), self.ws.numel(),
            _stream(self.dev))
        _lib.check(rc, "dropkv_evict")
        return self.keep_idx, self.k_out, self.v_out


def decode_workspace(B: int, Hq: int, Hkv: int, D: int, capacity: int, device) -> torch.Tensor:
    """Workspace of ``decode_attention`` for one cache geometry (reusable
    across steps and layers of that geometry)."""
    nbytes = _lib.load().dropkv_decode_workspace_bytes(B, Hq, Hkv, D, capacity)
    if nbytes == 0:
        raise RuntimeError("unsupported decode geometry")
    return _workspace(nbytes, torch.device(device))


def decode_attention(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                     v_cache: torch.Tensor, n_rows: torch.Tensor, scale: float, out: torch.Tensor,
                     workspace: torch.Tensor) -> torch.Tensor:
    """One decode step on preallocated cache buffers (``dropkv_decode_attention``):
    stores k_new / v_new at row ``n_rows`` and writes the attention of q over
    rows 0 .. n_rows into ``out`` [B, 1, Hq, D].  ``n_rows`` (int32, device)
    is not advanced.  Launches only kernels: capturable in a HIP graph."""
    dev = _check_device(q, k_new, v_new, k_cache, v_cache, n_rows, out, workspace)
    if q.dtype not in _DTYPE_CODE or {k_new.dtype, v_new.dtype, k_cache.dtype, v_cache.dtype, out.dtype} != {q.dtype}:
        raise RuntimeError("decode_attention: all tensors must share a bf16/fp16 dtype")
    if n_rows.dtype != torch.int32:
        raise RuntimeError("decode_attention: n_rows must be int32")
    B, Hq, Lq, D = q.shape
    _, Hkv, C, Dk = k_cache.shape
    if Lq != 1 or Dk != D or tuple(k_new.shape) != (B, Hkv, 1, D) or v_new.shape != k_new.shape:
        raise RuntimeError("decode_attention: shape mismatch")
    if k_cache.shape != v_cache.shape or not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise RuntimeError("decode_attention: cache buffers must be contiguous and alike")
    if k_new.stride() != v_new.stride():
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    if tuple(out.shape) != (B, 1, Hq, D):
        raise RuntimeError("decode_attention: out must be [B, 1, Hq, D]")
    rc = _lib.load().dropkv_decode_attention(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(3), k_new.data_ptr(), v_new.data_ptr(),
        k_new.stride(0), k_new.stride(1), k_new.stride(3), k_cache.data_ptr(), v_cache.data_ptr(),
        n_rows.data_ptr(), _DTYPE_CODE[q.dtype], B, Hq, Hkv, D, C, float(scale), out.data_ptr(),
        out.stride(0), out.stride(2), out.stride(3), workspace.data_ptr(), workspace.numel(), _stream(dev))
    _lib.check(rc, "dropkv_decode_attention")
    return out


def mfma_selftest(device="cuda") -> torch.Tensor:
    out = torch.empty(16, 16, dtype=torch.float32, device=device)
    rc = _lib.load().dropkv_selftest_mfma(out.data_ptr(), _stream(out.device))
    _lib.check(rc, "dropkv_selftest_mfma")
    return out
