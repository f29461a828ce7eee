"""Post-RoPE query capture for unpatched HF Transformers 5.x attention.

The reference's eviction needs the attention's rotated ``query_states`` at
cache-update time; its Transformers patch adds them to ``cache_kwargs`` in
``Qwen2Attention`` and ``LlamaAttention`` (patches/dropkv_transformers.patch:330,
:343).  The installed Transformers calls ``past_key_values.update(key, value,
layer_idx)`` right after ``apply_rotary_pos_emb``, so recording that
function's rotated query gives the cache the same tensor without patching
the library.
"""

from __future__ import annotations

import contextlib
import importlib
import threading
from typing import Optional

import torch

# Modeling modules whose attention the reference patch changes (patch:330, :343).
DEFAULT_MODELING_MODULES = (
    "transformers.models.qwen2.modeling_qwen2",
    "transformers.models.llama.modeling_llama",
)

_slot = threading.local()


def take_captured_query() -> Optional[torch.Tensor]:
    """The query recorded by the last rotary call on this thread (or None),
    cleared so that it is used by one cache update only."""
    q = getattr(_slot, "query", None)
    _slot.query = None
    return q


@contextlib.contextmanager
def query_capture(*modules):
    """Record the post-RoPE query of every attention call made inside the
    block, for the ``DropKVLayer.update`` that follows it on the same thread.

    ``modules`` are modeling modules (or their dotted names) whose
    ``apply_rotary_pos_emb`` the attention looks up at call time; the default
    covers Qwen2 and Llama, the two models the reference patch changes.
    The original functions are restored on exit, also on error.
    """
    mods = [importlib.import_module(m) if isinstance(m, str) else m for m in (modules or DEFAULT_MODELING_MODULES)]
    saved = []
    for mod in mods:
        orig = mod.apply_rotary_pos_emb

        def recording(q, k, *args, _orig=orig, **kwargs):
            q_rot, k_rot = _orig(q, k, *args, **kwargs)
            _slot.query = q_rot
            return q_rot, k_rot

        recording.__wrapped__ = orig
        saved.append((mod, orig))
        mod.apply_rotary_pos_emb = recording
    try:
        yield
    finally:
        for mod, orig in reversed(saved):
            mod.apply_rotary_pos_emb = orig
        _slot.query = None
