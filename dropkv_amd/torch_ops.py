"""The scorer and the layer-call as PyTorch operators (``torch.ops.dropkv``).

Registered with ``torch.library.custom_op`` together with fake (shape-only)
implementations, so that ``torch.compile`` traces code that calls them into
one graph, with the operator as an opaque node that runs the HIP library,
instead of breaking the graph at the ctypes call:

* ``torch.ops.dropkv.scores(q, k, v, window, eps, p_round, y_round, splits)``
  -> scores ``[B, Hkv, Lk]`` float32 (``dropkv_scores`` in the C ABI; the
  scoring of ``dropkv_scores_triton``, dropkv_triton.py:643-828);
* ``torch.ops.dropkv.select(scores, kernel_size, window, keep)`` ->
  ``(keep_idx [..., keep] int64 ascending, pooled)`` (``dropkv_select``: pool,
  protect, top-k, sort, dropkv_cache.py:464-475);
* ``torch.ops.dropkv.compact(k, v, keep_idx)`` -> ``(k_out, v_out)``
  (``dropkv_compact``: ``_gather_compressed``, dropkv_cache.py:479-491);
* ``torch.ops.dropkv.evict(q, k, v, window, kernel_size, keep, protect_window,
  eps, p_round, y_round, splits)`` -> ``(keep_idx [B, Hkv, keep] int64,
  k_out, v_out [B, Hkv, keep, D])`` (``dropkv_evict``: ``_compute_keep_indices``
  then ``_gather_compressed``, dropkv_cache.py:355-491, in one call).

All return fresh tensors.  ``dropkv_scores_triton`` and ``DropKVCache`` call
them while ``torch.compile`` traces, and the ctypes wrappers of
:mod:`dropkv_amd.ops` otherwise (no dispatcher overhead in eager code).
"""

from typing import Tuple

import torch

from . import ops


@torch.library.custom_op("dropkv::scores", mutates_args=())
def scores(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int, eps: float = 1e-6,
           p_round: bool = True, y_round: bool = False, splits: int = 0) -> torch.Tensor:
    return ops.scores(q, k, v, window, eps=eps, p_round=p_round, y_round=y_round, splits=splits)


@scores.register_fake
def _scores_fake(q, k, v, window, eps=1e-6, p_round=True, y_round=False, splits=0):
    torch._check(k.dim() == 4 and v.shape == k.shape and q.dim() == 4)
    return q.new_empty((k.shape[0], k.shape[1], k.shape[2]), dtype=torch.float32)


@torch.library.custom_op("dropkv::evict", mutates_args=())
def evict(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int, kernel_size: int, keep: int,
          protect_window: int, eps: float = 1e-6, p_round: bool = True, y_round: bool = False,
          splits: int = 0) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return ops.evict(q, k, v, window, kernel_size, keep, protect_window=protect_window, eps=eps, p_round=p_round,
                     y_round=y_round, splits=splits)


@evict.register_fake
def _evict_fake(q, k, v, window, kernel_size, keep, protect_window, eps=1e-6, p_round=True, y_round=False,
                splits=0):
    torch._check(k.dim() == 4 and v.shape == k.shape and q.dim() == 4)
    B, Hkv, _, D = k.shape
    idx = q.new_empty((B, Hkv, keep), dtype=torch.int64)
    return idx, k.new_empty((B, Hkv, keep, D)), v.new_empty((B, Hkv, keep, D))


@torch.library.custom_op("dropkv::select", mutates_args=())
def select(scores: torch.Tensor, kernel_size: int, window: int, keep: int) -> Tuple[torch.Tensor, torch.Tensor]:
    idx, pooled = ops.select(scores, kernel_size, window, keep, return_pooled=True)
    return idx, pooled


@select.register_fake
def _select_fake(scores, kernel_size, window, keep):
    torch._check(scores.dtype == torch.float32)
    return scores.new_empty((*scores.shape[:-1], keep), dtype=torch.int64), torch.empty_like(scores)


@torch.library.custom_op("dropkv::compact", mutates_args=())
def compact(k: torch.Tensor, v: torch.Tensor, keep_idx: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    return ops.compact(k, v, keep_idx)


@compact.register_fake
def _compact_fake(k, v, keep_idx):
    torch._check(k.dim() == 4 and v.shape == k.shape and keep_idx.dim() == 3)
    B, H, _, D = k.shape
    keep = keep_idx.shape[-1]
    return k.new_empty((B, H, keep, D)), v.new_empty((B, H, keep, D))


def compiling() -> bool:
    """Whether ``torch.compile`` is tracing the caller."""
    return torch.compiler.is_compiling()
