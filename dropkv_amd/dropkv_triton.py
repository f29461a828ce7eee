"""Drop-in for the reference's scoring module (dropkv_triton.py), on gfx950.

``dropkv_scores_triton`` keeps the reference signature, argument meaning and
``AssertionError`` guards (dropkv_triton.py:643-716); the work runs in the HIP
kernels of libdropkv_amd.so (split-K flash partials, cross-split merge,
per-key score).  The module name is kept so callers only change the import
root.  The reference's pure-PyTorch oracle ``dropkv_scores_reference`` is not
part of this package: the CPU restatement used for checking lives under
``oracle/`` in the repository.
"""

from __future__ import annotations

import math

import torch

from . import ops, torch_ops


def _next_power_of_2(n: int) -> int:
    """Round up to a power of two, at least 16 (dropkv_triton.py:618-621)."""
    n = max(n, 16)
    return 1 << (n - 1).bit_length()


def _compute_num_splits(B: int, Hkv: int, L: int, BLOCK_N: int, device) -> int:
    """Split-K depth heuristic of the reference (dropkv_triton.py:624-640):
    aim for two programs per compute unit, at least 4 tiles of ``BLOCK_N``
    keys per split, at most 64 splits.  Kept for API compatibility; the HIP
    path sizes its own grids (see ``dropkv_scores`` ``splits=0``)."""
    num_cus = torch.cuda.get_device_properties(device).multi_processor_count
    total_tiles = (L + BLOCK_N - 1) // BLOCK_N
    target = 2 * num_cus
    base = B * Hkv
    if base >= target:
        return 1
    wanted = math.ceil(target / base)
    return max(1, min(wanted, max(1, total_tiles // 4), 64))


def check_scoring_inputs(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, window_size: int,
                         require_contiguous: bool = True) -> None:
    """The input contract of the fast scoring path, message for message as
    dropkv_triton.py:680-716; raises ``AssertionError``.  Callers whose K/V
    are rows of a row-capacity buffer (the kernels take its row stride) pass
    ``require_contiguous=False``."""
    B, Hq, Lq, D = Q.shape
    Hkv = K.shape[1]
    Lk = K.shape[2]

    assert isinstance(window_size, int) and window_size > 0, (
        f"window_size must be a positive int, got {window_size}"
    )
    assert Lq >= window_size, f"Lq ({Lq}) must be >= window_size ({window_size})"
    assert Lk >= window_size, f"Lk ({Lk}) must be >= window_size ({window_size})"
    assert Lq <= Lk, f"Lq ({Lq}) must be <= Lk ({Lk}) (Q must be tail-aligned suffix)"
    assert Hq % Hkv == 0, f"Hq ({Hq}) must be divisible by Hkv ({Hkv})"
    assert Q.is_cuda, "Inputs must be on CUDA"
    assert Q.device == K.device == V.device, "All inputs must be on same device"
    assert not require_contiguous or (K.is_contiguous() and V.is_contiguous()), (
        "K and V must be contiguous (Q is sliced internally)"
    )
    assert Q.dtype == K.dtype == V.dtype, "All inputs must have same dtype"
    assert Q.dtype in (torch.float16, torch.bfloat16), (
        f"Input dtype must be fp16 or bf16, got {Q.dtype}"
    )
    assert K.shape == V.shape, f"K and V shape mismatch: K={K.shape}, V={V.shape}"
    assert K.shape[0] == B and K.shape[3] == D, (
        f"K batch/head_dim mismatch: expected B={B}, D={D}, got K={K.shape}"
    )
    assert D >= 32, f"D ({D}) must be >= BLOCK_K (32)"
    assert D & (D - 1) == 0, f"D ({D}) must be a power of 2"


def dropkv_scores_triton(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    window_size: int = 8,
    eps: float = 1e-6,
    allow_tf32: bool = True,
    match_pytorch_precision: bool = True,
) -> torch.Tensor:
    """DropKV eviction scores [B, Hkv, Lk] fp32 computed by the HIP kernels.

    Q [B,Hq,Lq,D] (bf16/fp16, any strides; only the last ``window_size`` rows
    are read), K/V [B,Hkv,Lk,D] contiguous, Lq <= Lk, the query being the
    tail-aligned suffix of the keys.

    ``match_pytorch_precision=True`` rounds the softmax probabilities to the
    input dtype before ``w = (p/(1-p+eps))^2`` (dropkv_triton.py:584-587).
    Head dimensions 32, 64 and 128 run on the matrix-core kernels, other
    powers of two (up to 4096) on the library's generic fp32 kernels.

    ``allow_tf32`` is accepted for compatibility and has no effect: gfx950 has
    no TF32 matrix path; P.V and Y.V^T run as bf16/fp16 MFMAs with the fp32
    operand split into two bf16/fp16 terms, which is at least as accurate.
    """
    check_scoring_inputs(Q, K, V, window_size)
    if torch_ops.compiling():
        return torch.ops.dropkv.scores(Q, K, V, window_size, eps, match_pytorch_precision, False, 0)
    return ops.scores(Q, K, V, window_size, eps=eps, p_round=match_pytorch_precision, y_round=False)
