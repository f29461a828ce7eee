"""Drop-in for the reference's cache module (dropkv_cache.py), on gfx950.

``DropKVCache`` and ``prefill_chunked`` keep the reference API, prefill modes,
length bookkeeping and error types (dropkv_cache.py:310-807).  Scoring,
pooling, top-k, sorting and gathering run in the HIP kernels of
libdropkv_amd.so:

* fast path (``use_triton=True`` and the scoring guards pass):
  :func:`dropkv_amd.dropkv_triton.dropkv_scores_triton`;
* otherwise the reference's deployed scoring semantics
  (dropkv_cache.py:401-460: ``W = min(window, Lq)``, softmax rounded to the
  input dtype, ``y = p @ V`` in the input dtype) run on the same kernels with
  ``y`` rounded to the input dtype;
* selection (dropkv_cache.py:464-475) and gather (:479-491) always run on the
  HIP select / compact kernels.

fp32 inputs and head dimensions outside the matrix-core set run on the
library's generic HIP kernels with the same semantics.  There is no CPU
fallback: CPU tensors raise ``RuntimeError``.
"""

from __future__ import annotations

import logging
from typing import Any, Iterable, Optional

import torch

from . import _lib, ops, torch_ops
from .hf_query import take_captured_query

logger = logging.getLogger(__name__)


def cat_rows(k0: torch.Tensor, v0: torch.Tensor, k1: torch.Tensor, v1: torch.Tensor):
    """``torch.cat([k0, k1], dim=-2)`` and the same for v, the reference's
    cache append (dropkv_cache.py:573-578, :583-588, :611-616): a new
    contiguous [B, H, L0 + L1, D] tensor each, filled by two launches of the
    library's append kernel, whose non-temporal stores do not leave the copy
    waiting at its end for dirty cache lines.  The same values as torch.cat;
    torch.cat itself where the kernel does not apply (tensors off the GPU,
    mismatched shapes or dtypes, while torch.compile traces, or where autograd
    would record the op)."""
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in (k0, v0, k1, v1))
    ok = (not grad and not torch_ops.compiling() and k0.is_cuda and k0.dim() == 4 and k1.dim() == 4
          and k0.dtype == v0.dtype == k1.dtype == v1.dtype and k0.shape == v0.shape and k1.shape == v1.shape
          and k0.shape[:2] == k1.shape[:2] and k0.shape[3] == k1.shape[3]
          and len({k0.device, v0.device, k1.device, v1.device}) == 1)
    if not ok:
        return torch.cat([k0, k1], dim=-2), torch.cat([v0, v1], dim=-2)
    B, H, L0, D = k0.shape
    k = torch.empty(B, H, L0 + k1.shape[2], D, dtype=k0.dtype, device=k0.device)
    v = torch.empty_like(k)
    ops.append(k0, v0, k, v, 0)
    ops.append(k1, v1, k, v, L0)
    return k, v


class _LayerCache:
    """Per-layer K/V lists with the legacy HF container protocol that the
    reference's ``DropKVCache`` inherits (dropkv_cache.py:104-307): only the
    parts the eviction path relies on (layout of ``key_cache`` /
    ``value_cache``, ``_seen_tokens``, indexing, legacy conversion)."""

    is_compileable = False

    def __init__(self, _distributed_cache_data: Optional[Iterable] = None) -> None:
        self._seen_tokens = 0
        self.key_cache: list[torch.Tensor] = []
        self.value_cache: list[torch.Tensor] = []
        if _distributed_cache_data is not None:
            for k, v in _distributed_cache_data:
                self.key_cache.append(k)
                self.value_cache.append(v)

    def __getitem__(self, layer_idx: int):
        if layer_idx < len(self):
            return self.key_cache[layer_idx], self.value_cache[layer_idx]
        raise KeyError(f"Cache only has {len(self)} layers, attempted to access layer with index {layer_idx}")

    def __iter__(self):
        for i in range(len(self)):
            yield self.key_cache[i], self.value_cache[i]

    def __len__(self):
        return len(self.key_cache)

    def get_max_cache_shape(self) -> Optional[int]:
        return None

    def to_legacy_cache(self):
        return tuple((self.key_cache[i], self.value_cache[i]) for i in range(len(self)))

    @classmethod
    def from_legacy_cache(cls, past_key_values=None):
        cache = cls()
        if past_key_values is not None:
            for i, (k, v) in enumerate(past_key_values):
                cache.update(None, k, v, i)
        return cache

    def reorder_cache(self, beam_idx: torch.LongTensor):
        for i in range(len(self.key_cache)):
            if self.key_cache[i].numel():
                dev = self.key_cache[i].device
                self.key_cache[i] = self.key_cache[i].index_select(0, beam_idx.to(dev))
            if self.value_cache[i].numel():
                dev = self.value_cache[i].device
                self.value_cache[i] = self.value_cache[i].index_select(0, beam_idx.to(dev))


def _deployed_path_scores(query_states, key_states, value_states, window_size: int) -> torch.Tensor:
    """Scores with the deployed PyTorch path's precision (dropkv_cache.py:401-460)
    on the HIP kernels: ``W = min(window, Lq)``, p and y rounded to the input
    dtype."""
    Hq, Hkv = query_states.shape[1], key_states.shape[1]
    if Hq % Hkv != 0:
        raise ValueError(f"Query heads {Hq} must be divisible by KV heads {Hkv}")
    W = min(window_size, query_states.shape[2])
    if torch_ops.compiling():
        return torch.ops.dropkv.scores(query_states, key_states, value_states, W, 1e-6, True, True, 0)
    return ops.scores(query_states, key_states, value_states, W, eps=1e-6, p_round=True, y_round=True)


def _check_head_dim(head_dim: int) -> None:
    """The HIP scoring kernels take head dimensions up to
    ``_lib.MAX_HEAD_DIM``; larger ones are refused here, before any device
    work (the reference's PyTorch path scores any D)."""
    if head_dim > _lib.MAX_HEAD_DIM:
        raise ValueError(f"head dimension {head_dim} is above {_lib.MAX_HEAD_DIM}, the largest the DropKV HIP "
                         "kernels score")


class DropKVCache(_LayerCache):
    """KV cache that evicts at prefill by the DropKV score
    (dropkv_cache.py:310-648).

    ``capacity`` (not in the reference): keep each layer's K/V in two
    preallocated buffer pairs of ``capacity`` rows per head instead of
    concatenating and gathering into new tensors.  A chunk is appended in
    place after the stored rows, the model attends over that buffer's first
    rows (a view), and an eviction gathers from it straight into the other
    pair's first rows (``dropkv_evict_ld``).  The stored and returned K/V are
    bit for bit those of the default mode; ``capacity`` must cover the
    largest stored-plus-chunk length, decode steps included, or ``update``
    raises ``ValueError``.  The stored tensors are views of the buffers."""

    def __init__(self, keep_ratio: float = 0.1, window_size: int = 8, kernel_size: int = 11,
                 use_triton: bool = True, capacity: Optional[int] = None) -> None:
        super().__init__()
        if not 0 < keep_ratio <= 1.0:
            raise ValueError(f"keep_ratio must be in (0, 1], got {keep_ratio}")
        self.keep_ratio = keep_ratio
        if window_size <= 0:
            raise ValueError(f"window_size must be positive, got {window_size}")
        self.window_size = window_size
        if kernel_size < 1 or kernel_size % 2 == 0:
            raise ValueError(f"kernel_size must be a positive odd integer, got {kernel_size}")
        self.kernel_size = kernel_size
        self.use_triton = use_triton
        # "single_pass" | "accumulate" | "evict_accumulated" (dropkv_cache.py:332-340)
        self._prefill_mode = "single_pass"
        self._evict_use_seen_tokens = False
        self._budget_max_kv_tokens: Optional[int] = None
        if capacity is not None and int(capacity) < 1:
            raise ValueError(f"capacity must be a positive number of rows, got {capacity}")
        self.capacity = None if capacity is None else int(capacity)
        self._buf: list = []  # capacity mode, per layer: [k0, v0, k1, v1]
        self._cur: list = []  # capacity mode, per layer: the pair holding the stored rows

    def batch_split(self, full_batch_size: int, split_size: int):
        raise NotImplementedError(
            "DropKVCache does not support batch_split (beam search). "
            "Use DynamicCache for beam search or implement DropKV-aware splitting.")

    @classmethod
    def from_batch_splits(cls, splits, **kwargs):
        raise NotImplementedError(
            "DropKVCache does not support from_batch_splits (beam search). "
            "Use DynamicCache for beam search or implement DropKV-aware merging.")

    # -- keep length (dropkv_cache.py:470-473) ---------------------------------
    def _keep_length(self, seq_len: int, total_tokens: Optional[int], max_keep_len: Optional[int]) -> int:
        base = total_tokens if total_tokens is not None else seq_len
        keep = min(seq_len, max(int(self.keep_ratio * base), self.window_size, 1))
        if max_keep_len is not None:
            keep = min(keep, max_keep_len)
        return keep

    def _compute_keep_indices(self, query_states: torch.Tensor, key_states: torch.Tensor,
                              value_states: torch.Tensor, total_tokens: Optional[int] = None,
                              max_keep_len: Optional[int] = None) -> torch.Tensor:
        """Sorted indices [B, Hkv, keep] of the keys to retain
        (dropkv_cache.py:355-477)."""
        bsz, num_kv_heads, seq_len, head_dim = key_states.shape
        num_query_heads = query_states.shape[1]
        if num_query_heads % num_kv_heads != 0:
            raise ValueError(f"Query heads {num_query_heads} must be divisible by KV heads {num_kv_heads}")
        _check_head_dim(head_dim)

        scores = None
        if self.use_triton:
            try:
                from . import dropkv_triton as _scoring
                scores = _scoring.dropkv_scores_triton(
                    query_states, key_states.contiguous(), value_states.contiguous(),
                    window_size=self.window_size)
            except (ImportError, AssertionError):
                scores = None
        if scores is None:
            scores = _deployed_path_scores(query_states, key_states, value_states, self.window_size)

        keep_len = self._keep_length(seq_len, total_tokens, max_keep_len)
        protect = min(self.window_size, seq_len)
        if torch_ops.compiling():
            return torch.ops.dropkv.select(scores, self.kernel_size, protect, keep_len)[0]
        return ops.select(scores, self.kernel_size, protect, keep_len)

    def _fast_path_ok(self, query_states, key_states, value_states) -> bool:
        """Whether ``dropkv_scores_triton`` accepts these inputs (its
        ``AssertionError`` guards, dropkv_triton.py:680-716); K/V count as
        contiguous because the fused call makes them so, as
        ``_compute_keep_indices`` passes ``.contiguous()`` copies
        (dropkv_cache.py:392-398)."""
        if not self.use_triton:
            return False
        try:
            from .dropkv_triton import check_scoring_inputs
            check_scoring_inputs(query_states, key_states, value_states, self.window_size,
                                 require_contiguous=False)
            return True
        except (ImportError, AssertionError):
            return False

    def _evict_layer(self, query_states: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
                     total_tokens: Optional[int] = None, max_keep_len: Optional[int] = None):
        """``_compute_keep_indices`` followed by ``_gather_compressed``
        (dropkv_cache.py:355-491) as one fused layer-call (``dropkv_evict``:
        score, pool, protect, top-k, sort, gather), with the same scoring
        choice, keep length and protection.  Returns the compressed K/V."""
        bsz, num_kv_heads, seq_len, head_dim = key_states.shape
        num_query_heads = query_states.shape[1]
        if num_query_heads % num_kv_heads != 0:
            raise ValueError(f"Query heads {num_query_heads} must be divisible by KV heads {num_kv_heads}")
        _check_head_dim(head_dim)
        fast = self._fast_path_ok(query_states, key_states, value_states)
        W = self.window_size if fast else min(self.window_size, query_states.shape[2])
        keep = self._keep_length(seq_len, total_tokens, max_keep_len)
        protect = min(self.window_size, seq_len)
        if torch_ops.compiling():
            _, key_c, value_c = torch.ops.dropkv.evict(query_states, key_states, value_states, W, self.kernel_size,
                                                       keep, protect, 1e-6, True, not fast, 0)
        else:
            _, key_c, value_c = ops.evict(query_states, key_states, value_states, W, self.kernel_size, keep,
                                          protect_window=protect, eps=1e-6, p_round=True, y_round=not fast)
        return key_c, value_c

    @staticmethod
    def _gather_compressed(key_states: torch.Tensor, value_states: torch.Tensor,
                           keep_idx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Gather the retained rows (dropkv_cache.py:479-491), bit-exact."""
        if torch_ops.compiling():
            return torch.ops.dropkv.compact(key_states, value_states, keep_idx)
        return ops.compact(key_states, value_states, keep_idx)

    def update(self, query_states: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
               layer_idx: Optional[int] = None, cache_kwargs: Optional[dict[str, Any]] = None):
        """Same control flow as dropkv_cache.py:493-622.

        Besides the native ``update(query, key, value, layer_idx)`` form, the
        calls a Transformers model makes are recognised:
        ``update(key, value, layer_idx, cache_kwargs)`` (4.x, the reference's
        detection, dropkv_cache.py:505-516) and ``update(key, value,
        layer_idx)`` (5.x).  In both the query comes from
        ``cache_kwargs["query_states"]`` or, failing that, from the rotary
        call recorded by :func:`dropkv_amd.hf_query.query_capture`."""
        hf_call = isinstance(value_states, int) and (layer_idx is None or isinstance(layer_idx, dict))
        if hf_call:
            cache_kwargs = layer_idx if isinstance(layer_idx, dict) else cache_kwargs
            layer_idx = value_states
            value_states = key_states
            key_states = query_states
            query_states = cache_kwargs.get("query_states") if cache_kwargs else None
            captured = take_captured_query()
            if query_states is None:
                query_states = captured
            if query_states is None:
                logger.warning(
                    "DropKVCache.update() called without query_states — eviction disabled for this layer. "
                    "Patch your transformers to pass query_states in cache_kwargs, or run the model inside "
                    "dropkv_amd.hf_query.query_capture().")
        elif layer_idx is None:
            raise TypeError("update() missing required argument: 'layer_idx'")

        if layer_idx == 0:
            self._seen_tokens += key_states.shape[-2]

        if len(self.key_cache) < layer_idx:
            raise ValueError("Use DynamicCache.")
        if self.capacity is not None:
            return self._update_capacity(query_states, key_states, value_states, layer_idx)
        if len(self.key_cache) == layer_idx:
            # --- prefill ---
            if query_states is None:
                if self._prefill_mode != "single_pass":
                    logger.warning("query_states is None at layer %d — storing full KV without eviction.",
                                   layer_idx)
                self.key_cache.append(key_states)
                self.value_cache.append(value_states)
                return key_states, value_states

            seq_len = key_states.shape[2]
            if self._prefill_mode not in ("single_pass", "accumulate", "evict_accumulated"):
                raise ValueError(f"Invalid _prefill_mode: {self._prefill_mode!r}")
            if self._prefill_mode == "accumulate" or seq_len < self.window_size:
                self.key_cache.append(key_states)
                self.value_cache.append(value_states)
                return key_states, value_states

            total_tok = self._seen_tokens if self._evict_use_seen_tokens else None
            key_c, value_c = self._evict_layer(query_states, key_states, value_states, total_tokens=total_tok,
                                               max_keep_len=self._budget_max_kv_tokens)
            self.key_cache.append(key_c)
            self.value_cache.append(value_c)
            return key_states, value_states

        # --- decode / chunked-prefill continuation ---
        if self._prefill_mode == "accumulate":
            self.key_cache[layer_idx], self.value_cache[layer_idx] = cat_rows(
                self.key_cache[layer_idx], self.value_cache[layer_idx], key_states, value_states)
            return self.key_cache[layer_idx], self.value_cache[layer_idx]
        if self._prefill_mode == "evict_accumulated":
            full_key, full_value = cat_rows(self.key_cache[layer_idx], self.value_cache[layer_idx], key_states,
                                            value_states)
            if query_states is not None and full_key.shape[2] >= self.window_size:
                total_tok = self._seen_tokens if self._evict_use_seen_tokens else None
                key_c, value_c = self._evict_layer(query_states, full_key, full_value, total_tokens=total_tok,
                                                   max_keep_len=self._budget_max_kv_tokens)
                self.key_cache[layer_idx] = key_c
                self.value_cache[layer_idx] = value_c
            else:
                self.key_cache[layer_idx] = full_key
                self.value_cache[layer_idx] = full_value
            return full_key, full_value
        if self._prefill_mode == "single_pass":
            self.key_cache[layer_idx], self.value_cache[layer_idx] = cat_rows(
                self.key_cache[layer_idx], self.value_cache[layer_idx], key_states, value_states)
            return self.key_cache[layer_idx], self.value_cache[layer_idx]
        raise ValueError(f"Invalid _prefill_mode {self._prefill_mode!r} in decode path")

    # -- capacity mode ---------------------------------------------------------
    def _alloc(self, layer_idx: int, like: torch.Tensor) -> None:
        B, H, _, D = like.shape
        shape = (B, H, self.capacity, D)
        if layer_idx < len(self._buf):
            b = self._buf[layer_idx][0]
            if b.shape == shape and b.dtype == like.dtype and b.device == like.device:
                self._cur[layer_idx] = 0
                return
        bufs = [torch.empty(shape, dtype=like.dtype, device=like.device) for _ in range(4)]
        if layer_idx < len(self._buf):
            self._buf[layer_idx], self._cur[layer_idx] = bufs, 0
        else:
            self._buf.append(bufs)
            self._cur.append(0)

    def _pair(self, layer_idx: int, which: Optional[int] = None):
        i = self._cur[layer_idx] if which is None else which
        b = self._buf[layer_idx]
        return b[2 * i], b[2 * i + 1]

    def _set_stored(self, layer_idx: int, n: int) -> None:
        k, v = self._pair(layer_idx)
        kv, vv = k[:, :, :n], v[:, :, :n]
        if len(self.key_cache) == layer_idx:
            self.key_cache.append(kv)
            self.value_cache.append(vv)
        else:
            self.key_cache[layer_idx] = kv
            self.value_cache[layer_idx] = vv

    def _fits(self, layer_idx: int, rows: int) -> None:
        if rows > self.capacity:
            raise ValueError(f"DropKVCache capacity of {self.capacity} rows exceeded at layer {layer_idx}: "
                             f"{rows} rows needed")

    def _evict_into(self, layer_idx: int, query_states, k_src, v_src, Lk: int, k_out, v_out) -> int:
        """Eviction of rows 0 .. Lk-1 of k_src / v_src ([B, Hkv, ld, D]) into
        the first rows of k_out / v_out; the same scoring choice, keep length
        and protection as _compute_keep_indices.  Returns the keep length;
        raises ``ValueError`` when the kept rows exceed the capacity."""
        if query_states.shape[1] % k_src.shape[1] != 0:
            raise ValueError(f"Query heads {query_states.shape[1]} must be divisible by KV heads {k_src.shape[1]}")
        _check_head_dim(k_src.shape[3])
        fast = self._fast_path_ok(query_states, k_src[:, :, :Lk], v_src[:, :, :Lk])
        W = self.window_size if fast else min(self.window_size, query_states.shape[2])
        total_tok = self._seen_tokens if self._evict_use_seen_tokens else None
        keep = self._keep_length(Lk, total_tok, self._budget_max_kv_tokens)
        self._fits(layer_idx, keep)
        ops.evict_ld(query_states, k_src, v_src, Lk, W, self.kernel_size, keep, k_out, v_out,
                     protect_window=min(self.window_size, Lk), p_round=True, y_round=not fast)
        return keep

    def _update_capacity(self, query_states, key_states, value_states, layer_idx: int):
        """update() in capacity mode: the control flow of the default mode,
        with appends into and gathers between the layer's buffers."""
        L = key_states.shape[2]
        if len(self.key_cache) == layer_idx:
            # --- prefill ---
            self._alloc(layer_idx, key_states)
            store_all = query_states is None
            if store_all:
                if self._prefill_mode != "single_pass":
                    logger.warning("query_states is None at layer %d — storing full KV without eviction.",
                                   layer_idx)
            else:
                if self._prefill_mode not in ("single_pass", "accumulate", "evict_accumulated"):
                    raise ValueError(f"Invalid _prefill_mode: {self._prefill_mode!r}")
                store_all = self._prefill_mode == "accumulate" or L < self.window_size
            if store_all:
                self._fits(layer_idx, L)
                k, v = self._pair(layer_idx)
                ops.append(key_states, value_states, k, v, 0)
                self._set_stored(layer_idx, L)
                return key_states, value_states
            src_k, src_v = key_states.contiguous(), value_states.contiguous()
            if src_k.data_ptr() % 16 or src_v.data_ptr() % 16:
                src_k, src_v = src_k.clone(), src_v.clone()
            k, v = self._pair(layer_idx)
            keep = self._evict_into(layer_idx, query_states, src_k, src_v, L, k, v)
            self._set_stored(layer_idx, keep)
            return key_states, value_states

        # --- decode / chunked-prefill continuation ---
        if self._prefill_mode not in ("single_pass", "accumulate", "evict_accumulated"):
            raise ValueError(f"Invalid _prefill_mode {self._prefill_mode!r} in decode path")
        n = self.key_cache[layer_idx].shape[2]
        self._fits(layer_idx, n + L)
        k, v = self._pair(layer_idx)
        ops.append(key_states, value_states, k, v, n)
        full_k, full_v = k[:, :, :n + L], v[:, :, :n + L]
        if (self._prefill_mode == "evict_accumulated" and query_states is not None
                and n + L >= self.window_size):
            other = 1 - self._cur[layer_idx]
            ko, vo = self._pair(layer_idx, other)
            keep = self._evict_into(layer_idx, query_states, k, v, n + L, ko, vo)
            self._cur[layer_idx] = other
            self._set_stored(layer_idx, keep)
        else:
            self._set_stored(layer_idx, n + L)
        return full_k, full_v

    def reorder_cache(self, beam_idx: torch.LongTensor):
        if self.capacity is None:
            return super().reorder_cache(beam_idx)
        for i in range(len(self.key_cache)):
            n = self.key_cache[i].shape[2]
            k, v = self._pair(i)
            other = 1 - self._cur[i]
            ko, vo = self._pair(i, other)
            sel = beam_idx.to(k.device)
            ko[:, :, :n].copy_(k[:, :, :n].index_select(0, sel))
            vo[:, :, :n].copy_(v[:, :, :n].index_select(0, sel))
            self._cur[i] = other
            self._set_stored(i, n)

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        """Logical length (tokens seen) for RoPE positions (dropkv_cache.py:624-633)."""
        if len(self.key_cache) <= layer_idx:
            return 0
        return self._seen_tokens

    def _stored_length(self, layer_idx: int) -> int:
        empty = (len(self.key_cache) == 0 or len(self.key_cache) <= layer_idx
                 or not self.key_cache[layer_idx].numel())
        return 0 if empty else self.key_cache[layer_idx].shape[-2]

    def get_mask_sizes(self, cache_position, layer_idx: int = 0) -> tuple[int, int]:
        """(stored length + query length, 0) for the attention mask
        (dropkv_cache.py:635-648).  The query length comes from a
        ``cache_position`` tensor (Transformers 4.x, the reference's
        convention) or as an int (5.x)."""
        query_length = cache_position.shape[0] if isinstance(cache_position, torch.Tensor) else int(cache_position)
        return self._stored_length(layer_idx) + query_length, 0

    def get_query_offset(self, layer_idx: int = 0) -> int:
        """Index of the step's first query in the stored-K/V frame of the mask
        (Transformers 5.x asks for it separately from the RoPE length).

        It is the stored length: the mask pairs query ``i`` with key column
        ``kv`` iff ``kv <= offset + i``, so with the logical length (what the
        reference's pinned Transformers used, through ``cache_position``) a
        chunk that follows an eviction (``budget``, ``every_chunk``) would let
        query ``i`` see up to ``_seen_tokens - stored`` later keys of its own
        chunk."""
        return self._stored_length(layer_idx)


def prefill_chunked(model, input_ids, cache, chunk_size=4096, evict_strategy="last_chunk",
                    max_kv_tokens=32768, **forward_kwargs):
    """Chunked prefill with eviction strategies ``last_chunk`` / ``budget`` /
    ``every_chunk`` (dropkv_cache.py:651-807).  Same validation errors, mode
    schedule and cleanup on failure as the reference."""
    if not isinstance(cache, DropKVCache):
        raise TypeError(f"cache must be DropKVCache, got {type(cache).__name__}")
    if len(cache.key_cache) > 0:
        raise ValueError("prefill_chunked() requires a fresh (empty) cache. Create a new DropKVCache instance.")
    if chunk_size < cache.window_size:
        raise ValueError(f"chunk_size ({chunk_size}) must be >= window_size ({cache.window_size})")
    bad = {"attention_mask", "position_ids", "cache_position"} & forward_kwargs.keys()
    if bad:
        raise ValueError(
            f"prefill_chunked() does not support sequence-shaped kwargs {bad} — the model computes these "
            f"internally per chunk. Remove them from forward_kwargs.")
    strategies = ("last_chunk", "budget", "every_chunk")
    if evict_strategy not in strategies:
        raise ValueError(f"evict_strategy must be one of {strategies}, got {evict_strategy!r}")
    if evict_strategy == "budget":
        if max_kv_tokens is None:
            raise ValueError("max_kv_tokens is required when evict_strategy='budget'")
        if max_kv_tokens < cache.window_size:
            raise ValueError(f"max_kv_tokens ({max_kv_tokens}) must be >= window_size ({cache.window_size}) "
                             f"to preserve protected tail tokens")

    B, L = input_ids.shape
    if L <= chunk_size and evict_strategy == "last_chunk":
        with torch.no_grad():
            return model(input_ids, past_key_values=cache, use_cache=True, **forward_kwargs)

    starts = list(range(0, L, chunk_size))
    try:
        cache._evict_use_seen_tokens = evict_strategy in ("budget", "every_chunk")
        if evict_strategy == "budget":
            cache._budget_max_kv_tokens = max_kv_tokens
        with torch.no_grad():
            output = None
            for i, start in enumerate(starts):
                end = min(start + chunk_size, L)
                is_last = i == len(starts) - 1
                if evict_strategy == "last_chunk":
                    cache._prefill_mode = "evict_accumulated" if is_last else "accumulate"
                elif evict_strategy == "every_chunk":
                    cache._prefill_mode = "single_pass" if i == 0 else "evict_accumulated"
                else:
                    if is_last:
                        cache._prefill_mode = "evict_accumulated"
                    else:
                        stored = cache.key_cache[0].shape[2] if cache.key_cache else 0
                        cache._prefill_mode = ("evict_accumulated" if stored + (end - start) > max_kv_tokens
                                               else "accumulate")
                output = model(input_ids[:, start:end], past_key_values=cache, use_cache=True, **forward_kwargs)
            return output
    except BaseException:
        cache.key_cache.clear()
        cache.value_cache.clear()
        cache._seen_tokens = 0
        raise
    finally:
        cache._prefill_mode = "single_pass"
        cache._evict_use_seen_tokens = False
        cache._budget_max_kv_tokens = None
