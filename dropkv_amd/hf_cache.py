"""DropKV eviction behind the layer-based Cache API of HF Transformers 5.x.

The reference ships its Transformers integration as a patch to a pinned
Transformers commit (patches/dropkv_transformers.patch): a ``DropKVLayer``
(a ``DynamicLayer`` that evicts once, at prefill; patch:48-234), a
``DropKVCache(config, ...)`` holding one such layer per decoder layer
(patch:237-264), and a one-line change to ``Qwen2Attention`` /
``LlamaAttention`` that passes the post-RoPE ``query_states`` in
``cache_kwargs`` (patch:330, :343).

The installed Transformers (5.15) is unpatched: its attention calls
``past_key_values.update(key_states, value_states, layer_idx)`` with no
``cache_kwargs``.  :func:`query_capture` supplies the query instead: while it
is active, the modeling modules' ``apply_rotary_pos_emb`` also records the
rotated query, and the next ``DropKVLayer.update`` on the same thread takes
it.  A ``query_states`` entry in ``cache_kwargs`` (a patched Transformers)
wins over the captured one.

Eviction runs in one call of the fused HIP layer-call (``dropkv_evict``:
score, pool, protect, top-k, sort, gather); there is no CPU fallback.
"""

from __future__ import annotations

import logging
from typing import Any, Optional

import torch
from transformers.cache_utils import Cache, DynamicLayer

from . import ops, torch_ops
from .dropkv_cache import cat_rows
from .dropkv_triton import check_scoring_inputs
from .hf_query import query_capture, take_captured_query

logger = logging.getLogger(__name__)

__all__ = ["DropKVCache", "DropKVLayer", "query_capture"]


def _evict(query_states: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
           window_size: int, kernel_size: int, keep: int, use_triton: bool):
    """Sorted kept indices and the compressed K/V of one prefill layer-call.

    With ``use_triton`` and inputs the fast scoring path accepts, the scores
    follow ``dropkv_scores_triton`` (patch:125-137); otherwise the patch's
    PyTorch scoring precision (patch:138-179: softmax rounded to the input
    dtype, ``y = p @ V`` in the input dtype).  Pooling over ``kernel_size``,
    protection of the last ``window_size`` keys at ``max + 1``, top-``keep``
    and the ascending sort follow patch:181-192; the gather patch:194-202.
    One fused layer-call; the outputs are new tensors and the workspace is
    the current stream's shared one, so consecutive layers allocate no
    workspace.
    """
    key_states = key_states.contiguous()
    value_states = value_states.contiguous()
    fast = False
    if use_triton:
        try:
            check_scoring_inputs(query_states, key_states, value_states, window_size)
            fast = True
        except AssertionError:
            fast = False
    W = window_size if fast else min(window_size, query_states.shape[2])
    if torch_ops.compiling():
        return torch.ops.dropkv.evict(query_states, key_states, value_states, W, kernel_size, keep, window_size,
                                      1e-6, True, not fast, 0)
    return ops.evict(query_states, key_states, value_states, W, kernel_size, keep, protect_window=window_size,
                     p_round=True, y_round=not fast)


class DropKVLayer(DynamicLayer):
    """One decoder layer's cache: evicts at prefill, appends at decode
    (patch:48-234)."""

    def __init__(self, keep_ratio: float = 0.1, window_size: int = 8, kernel_size: int = 11,
                 use_triton: bool = True):
        super().__init__()
        if not 0 < keep_ratio <= 1.0:
            raise ValueError(f"keep_ratio must be in (0, 1], got {keep_ratio}")
        if window_size <= 0:
            raise ValueError(f"window_size must be positive, got {window_size}")
        if kernel_size < 1 or kernel_size % 2 == 0:
            raise ValueError(f"kernel_size must be a positive odd integer, got {kernel_size}")
        self.keep_ratio = keep_ratio
        self.window_size = window_size
        self.kernel_size = kernel_size
        self.use_triton = use_triton
        self._prefilled = False
        self.cumulative_length = 0
        self._warned_no_query = False
        self.last_keep_idx: Optional[torch.Tensor] = None

    def reset(self) -> None:
        """Forget the stored K/V and the prefill state (patch:71-79)."""
        super().reset()
        self._prefilled = False
        self._warned_no_query = False
        self.last_keep_idx = None
        if self.is_initialized:
            self.keys = torch.tensor([], dtype=self.dtype, device=self.device)
            self.values = torch.tensor([], dtype=self.dtype, device=self.device)

    def _stored_length(self) -> int:
        return 0 if (not self.is_initialized or self.keys.numel() == 0) else self.keys.shape[-2]

    def crop(self, tokens_to_remove: int) -> None:
        """Crop the stored K/V and set the logical length to the stored one
        (patch:81-86).  A negative argument removes that many tokens, a
        positive one is the length to keep (the Transformers convention)."""
        stored = self._stored_length()
        if tokens_to_remove > 0:
            remove = stored - tokens_to_remove if tokens_to_remove < stored else 0
        else:
            remove = min(-tokens_to_remove, stored)
        if remove:
            self.keys = self.keys[..., : stored - remove, :]
            self.values = self.values[..., : stored - remove, :]
        self.cumulative_length = self._stored_length()

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor,
               cache_kwargs: Optional[dict[str, Any]] = None, *args, **kwargs):
        """Prefill: score, keep the top fraction, store it compressed and
        return the full K/V for this step's attention.  Decode: append and
        return the stored K/V (patch:88-213)."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self.cumulative_length += key_states.shape[-2]

        query_states = cache_kwargs.get("query_states") if cache_kwargs is not None else None
        captured = take_captured_query()
        if query_states is None:
            query_states = captured
        if query_states is None and not self._prefilled and not self._warned_no_query:
            self._warned_no_query = True
            logger.warning(
                "DropKVLayer received no query_states. Eviction will not occur. Run the model inside "
                "dropkv_amd.hf_query.query_capture() or pass query_states in cache_kwargs.")

        if not self._prefilled and query_states is not None:
            self._prefilled = True
            bsz, num_kv_heads, seq_len, head_dim = key_states.shape
            if seq_len < self.window_size:
                self.keys = key_states
                self.values = value_states
                return key_states, value_states
            if query_states.shape[1] % num_kv_heads != 0:
                raise ValueError(
                    f"Query heads {query_states.shape[1]} must be divisible by KV heads {num_kv_heads}")
            keep = max(int(self.keep_ratio * seq_len), self.window_size, 1)
            keep_idx, k_c, v_c = _evict(query_states, key_states, value_states, self.window_size,
                                        self.kernel_size, keep, self.use_triton)
            self.last_keep_idx = keep_idx
            self.keys = k_c
            self.values = v_c
            return key_states, value_states

        self._prefilled = True
        self.keys, self.values = cat_rows(self.keys, self.values, key_states, value_states)
        return self.keys, self.values

    def get_seq_length(self) -> int:
        """Logical length (tokens seen), which RoPE positions follow
        (patch:215-222)."""
        return self.cumulative_length if self.is_initialized else 0

    def get_mask_sizes(self, query_length) -> tuple[int, int]:
        """(stored length + query length, 0): the mask matches the stored
        tensors, not the logical length (patch:224-234).  Transformers 5.x
        passes the query length as an int; a ``cache_position`` tensor (the
        patched commit's convention) is accepted too."""
        if isinstance(query_length, torch.Tensor):
            query_length = query_length.shape[0]
        return self._stored_length() + int(query_length), 0


class DropKVCache(Cache):
    """One :class:`DropKVLayer` per decoder layer of ``config``
    (patch:237-264)."""

    def __init__(self, config, keep_ratio: float = 0.1, window_size: int = 8, kernel_size: int = 11,
                 use_triton: bool = True):
        text = config.get_text_config(decoder=True)
        layers = [DropKVLayer(keep_ratio=keep_ratio, window_size=window_size, kernel_size=kernel_size,
                              use_triton=use_triton)
                  for _ in range(text.num_hidden_layers)]
        super().__init__(layers=layers)

    def stored_length(self, layer_idx: int = 0) -> int:
        """Number of K/V rows held for ``layer_idx`` (after eviction)."""
        if layer_idx >= len(self.layers):
            return 0
        return self.layers[layer_idx]._stored_length()

    def get_query_offset(self, layer_idx: int = 0) -> int:
        """Index of the step's first query in the stored-K/V frame of the
        attention mask: the stored length, not the logical one.

        The mask pairs query ``i`` with key column ``kv`` iff
        ``kv <= offset + i`` over ``stored + q_len`` columns.  With the logical
        length as offset (what the pinned Transformers commit of the reference
        did through ``cache_position``) a multi-token step after an eviction
        would let query ``i`` see up to ``logical - stored`` later keys of its
        own step.  RoPE positions still follow :meth:`get_seq_length`."""
        return self.stored_length(layer_idx)
