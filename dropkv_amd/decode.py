"""Decode on the compressed cache: preallocated K/V buffers, a HIP attention
kernel that appends and attends in one launch, and a HIP graph per step.

The reference decodes eagerly: every step appends the new row with
``torch.cat`` (dropkv_cache.py:609-617, patches/dropkv_transformers.patch:
206-213) and the model's SDPA attends over the concatenation.  Here, after
the prefill has evicted, each layer's kept rows are copied once into a
buffer with room for ``max_new_tokens`` more rows; the model (the installed
Transformers' own forward) runs with an attention function that calls
``dropkv_decode_attention`` on those buffers, whose row count lives on the
device.  Nothing in a step depends on the host, so the whole forward is
captured once as a HIP graph and replayed per token.
"""

from __future__ import annotations

import contextlib
import threading
from typing import Optional

import torch

from . import ops

ATTN_NAME = "dropkv_decode"
_active = threading.local()


def _decode_attention(module, query, key, value, attention_mask=None, scaling=None, dropout=0.0, **kwargs):
    """Attention function for the Transformers attention interface: one
    decode step of layer ``module.layer_idx`` on the active decoder's buffers.
    Returns ([B, 1, Hq, D], None)."""
    dec = getattr(_active, "decoder", None)
    if dec is None:
        raise RuntimeError("dropkv_decode attention used outside CompressedDecoder")
    if query.shape[2] != 1:
        raise RuntimeError("dropkv_decode attention takes one query position per step")
    i = module.layer_idx
    B, Hq, _, D = query.shape
    out = torch.empty(B, 1, Hq, D, dtype=query.dtype, device=query.device)
    scale = scaling if scaling is not None else D ** -0.5
    ops.decode_attention(query, key, value, dec.k_buf[i], dec.v_buf[i], dec.n_rows[i:i + 1], scale, out, dec.ws)
    return out, None


def _register():
    from transformers import AttentionInterface
    if ATTN_NAME not in AttentionInterface._global_mapping:
        AttentionInterface.register(ATTN_NAME, _decode_attention)


class _StepCache:
    """The ``past_key_values`` of a decode step: K/V already live in the
    decoder's buffers, so ``update`` hands the new rows straight to the
    attention, which stores them."""

    is_compileable = False

    def __init__(self, logical: int):
        self.logical = logical

    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        return key_states, value_states

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.logical


def _stored_kv(cache):
    if hasattr(cache, "layers"):
        return [(lay.keys, lay.values) for lay in cache.layers]
    return list(zip(cache.key_cache, cache.value_cache))


class CompressedDecoder:
    """Greedy-decode driver on a cache that a prefill filled (and evicted).

    ``cache`` is a :class:`dropkv_amd.hf_cache.DropKVCache` or a
    :class:`dropkv_amd.DropKVCache` after the prefill; its rows are copied
    into buffers of ``stored + max_new_tokens`` rows (rounded up to 64).
    RoPE positions continue from the cache's logical length.  With
    ``use_graph`` the forward is captured once and replayed per step.
    """

    def __init__(self, model, cache, max_new_tokens: int, use_graph: bool = True):
        _register()
        self.model = model
        kv = _stored_kv(cache)
        if not kv:
            raise ValueError("the cache holds no layers: run the prefill first")
        k0 = kv[0][0]
        self.device = k0.device
        B, Hkv, _, D = k0.shape
        stored = [k.shape[2] for k, _ in kv]
        self.capacity = (max(stored) + max_new_tokens + 63) // 64 * 64
        self.max_new_tokens = max_new_tokens
        self.k_buf, self.v_buf = [], []
        for k, v in kv:
            kb = torch.empty(B, Hkv, self.capacity, D, dtype=k.dtype, device=self.device)
            vb = torch.empty_like(kb)
            kb[:, :, :k.shape[2]].copy_(k)
            vb[:, :, :v.shape[2]].copy_(v)
            self.k_buf.append(kb)
            self.v_buf.append(vb)
        self.n_rows = torch.tensor(stored, dtype=torch.int32, device=self.device)
        Hq = model.config.num_attention_heads
        self.ws = ops.decode_workspace(B, Hq, Hkv, D, self.capacity, self.device)
        self.logical = cache.get_seq_length()
        self.pos = torch.full((B, 1), self.logical, dtype=torch.int64, device=self.device)
        self.tok = torch.zeros(B, 1, dtype=torch.int64, device=self.device)
        self.steps = 0
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.logits: Optional[torch.Tensor] = None
        if use_graph:
            self._capture()

    @contextlib.contextmanager
    def _active(self):
        cfg = self.model.config
        prev_impl, prev_dec = cfg._attn_implementation, getattr(_active, "decoder", None)
        cfg._attn_implementation = ATTN_NAME
        _active.decoder = self
        try:
            yield
        finally:
            cfg._attn_implementation = prev_impl
            _active.decoder = prev_dec

    @torch.no_grad()
    def _forward(self) -> torch.Tensor:
        with self._active():
            out = self.model(self.tok, position_ids=self.pos, past_key_values=_StepCache(self.logical),
                             use_cache=True, logits_to_keep=1)
        return out.logits

    @torch.no_grad()
    def _capture(self):
        # One eager run on a side stream first (library workspaces, lazy
        # initialisation); it stores a row at n that the first replay rewrites.
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._forward()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self._forward()
            self.n_rows.add_(1)
            self.pos.add_(1)

    @torch.no_grad()
    def step(self, token: torch.Tensor) -> torch.Tensor:
        """Logits [B, 1, vocab] of the next position after ``token`` [B, 1]."""
        if self.steps >= self.max_new_tokens:
            raise RuntimeError(f"decode capacity of {self.max_new_tokens} new tokens reached")
        self.tok.copy_(token)
        self.steps += 1
        if self.graph is not None:
            self.graph.replay()
            return self.logits
        logits = self._forward()
        self.n_rows.add_(1)
        self.pos.add_(1)
        return logits

    @torch.no_grad()
    def generate(self, token: torch.Tensor, steps: int) -> torch.Tensor:
        """``steps`` greedy tokens [B, steps] after ``token``; stays on the device."""
        toks = []
        for _ in range(steps):
            logits = self.step(token)
            token = logits[:, -1].argmax(-1, keepdim=True)
            toks.append(token)
        return torch.cat(toks, dim=1)
