"""MI355X (gfx950) implementation of DropKV's prefill-time KV eviction.

Public API (same names and semantics as the reference modules
``dropkv_triton`` / ``dropkv_cache``):

* :func:`dropkv_scores_triton` -- per-key eviction scores;
* :class:`DropKVCache`, :func:`prefill_chunked` -- the evicting cache;
* :mod:`dropkv_amd.ops` -- lower-level ops (scores, select, compact,
  compact2, EvictPlan for one-call layer eviction).
"""

from .dropkv_cache import DropKVCache, prefill_chunked
from .dropkv_triton import dropkv_scores_triton

__all__ = ["dropkv_scores_triton", "DropKVCache", "prefill_chunked"]
