"""CPU oracle for the DropKV prefill KV-eviction path.  TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product package (``dropkv_amd``) never imports it and fails
loudly when its HIP library is missing.

Every function restates one piece of the reference algorithm on the CPU with
PyTorch ops, and cites the reference file:line it follows (paths relative to
the reference checkout, ``AozhongZhang/DropKV``).

Pinning (how each function is checked independently of this file; the checks
live in ``tests/test_oracle.py``, the fixtures in ``tests/golden/``):

* ``dropkv_scores_reference`` -- float64 brute force with the *direct*
  ``||v_j - y_m||^2`` distance (not termA-termB+termC) on small shapes,
  including Lq < Lk, g = 1 and B = 2; golden fixtures written by
  ``tests/golden/make_golden.py`` (an independent NumPy float64 brute force);
  closed forms V = 0 -> 0, Q = 0 -> uniform softmax with y = causal prefix
  mean, a two-key logit gap; invariants: duplicated query heads leave the
  score unchanged (the 1/g average), contiguous head grouping, only the Q
  tail is read, scores >= 0.  ``eps`` is pinned only by presence: the Lk == W
  case (p = 1) stays finite; its value is below the float32 resolution of the
  reference's own expansion wherever that expansion is accurate.
* ``dropkv_scores_fp64`` (float64 arbiter of selections) -- the per-(b, hkv,
  gi, w) float64 brute force of ``tests/test_oracle.py``, with and without
  the bf16 rounding of p, to float64 rounding.
* ``fallback_scores`` (deployed ``use_triton=False`` path) -- float64 brute
  force with round-to-nearest-even of p and y to bf16; golden fixtures
  (including a final chunk shorter than the window); the reference tests'
  own bound against ``dropkv_scores_reference(match_pytorch_precision=True)``.
* ``pool_protect`` -- brute-force sliding max; the protected tail is
  ``max + 1`` in float32, absorbed at max >= 2^24.
* ``keep_length`` -- the keep-length table of the BASELINE configs and the
  reference tests' arithmetic (tests/test_dropkv_triton.py:909-937, :1183-1262).
* ``topk_sorted`` -- a rank rule on rows full of ties (i is kept iff
  #greater + #equal-with-lower-index < keep) and the tie-aware comparison
  against ``torch.topk``.
* ``gather_compressed`` -- bit equality with per-row fancy indexing.
* ``index_overlap`` -- planted mistakes (a non-tied swap is counted, a swap
  among threshold ties is excused).

No golden vectors were written by the reference itself: the reference's tests
hold none (they compare implementations on unseeded random inputs), and every
function here is pinned by the checks above, so the reference module was not
imported.

Tie rule: among keys whose pooled score equals the k-th largest value, the
lowest indices are kept.  The reference uses ``torch.topk``, whose choice among
exact ties is implementation-defined; the north-star metric excuses exactly
those positions (``index_overlap``).
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# a9: dropkv_scores_reference  (dropkv_triton.py:29-109)
# ---------------------------------------------------------------------------

def dropkv_scores_reference(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    window_size: int = 8,
    eps: float = 1e-6,
    match_pytorch_precision: bool = False,
) -> torch.Tensor:
    """Per-key residual-output perturbation score, fp32, shape [B, Hkv, Lk].

    Follows dropkv_triton.py:29-109: loop over (hkv, gi); logits of the last W
    query rows of head ``hkv*g+gi`` against all keys, scaled by 1/sqrt(D)
    (:79), causal ``triu`` mask with diagonal ``Lk-W+1`` (:81-85), fp32
    softmax (:87), optional round of p to the input dtype (:88-92), y = p@V
    in fp32 (:93), w = (p/(1-p+eps))^2 (:94), termA - termB + termC summed
    over the window rows (:96-106), divided by g (:108).

    Only the last W rows of Q are touched, so callers may pass just the tail.
    """
    B, Hq, Lq, D = Q.shape
    Hkv = K.shape[1]
    Lk = K.shape[2]
    g = Hq // Hkv
    W = window_size
    assert Lq >= W, f"Lq ({Lq}) must be >= window_size ({W})"
    assert Lk >= W, f"Lk ({Lk}) must be >= window_size ({W})"
    assert Lq <= Lk, f"Lq ({Lq}) must be <= Lk ({Lk}) (Q must be tail-aligned suffix)"

    Qt = Q[:, :, -W:, :].float()  # slice first: only the tail is read (:73)
    K_f = K.float()
    V_f = V.float()
    scores = torch.zeros(B, Hkv, Lk, dtype=torch.float32)
    mask = torch.triu(torch.full((W, Lk), float("-inf"), dtype=torch.float32), diagonal=Lk - W + 1)
    for hkv in range(Hkv):
        K_h = K_f[:, hkv:hkv + 1]
        V_h = V_f[:, hkv:hkv + 1]
        v_norm2 = (V_h ** 2).sum(dim=-1)
        for gi in range(g):
            Q_w = Qt[:, hkv * g + gi:hkv * g + gi + 1]
            logits = (Q_w @ K_h.transpose(-1, -2)) / math.sqrt(D) + mask
            p = F.softmax(logits, dim=-1, dtype=torch.float32)
            if match_pytorch_precision:
                p = p.to(Q.dtype).float()
            y = p @ V_h
            Wm = (p / (1.0 - p + eps)) ** 2
            termA = Wm.sum(dim=-2) * v_norm2
            termB = 2.0 * (V_h * (Wm.transpose(-1, -2) @ y)).sum(dim=-1)
            termC = (Wm.transpose(-1, -2) @ (y ** 2).sum(dim=-1).unsqueeze(-1)).squeeze(-1)
            scores[:, hkv:hkv + 1] += termA - termB + termC
    scores /= g
    return scores


def dropkv_scores_fp64(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    window_size: int = 8,
    eps: float = 1e-6,
    p_round: Optional[torch.dtype] = None,
    p_scale: float = 1.0,
    keys: Optional[torch.Tensor] = None,
    return_bound: bool = False,
):
    """The score of ``dropkv_scores_reference`` evaluated in float64 with the
    direct distance ``||v_j - y_m||^2`` instead of the float32 expansion
    termA - termB + termC (dropkv_triton.py:96-106); ``p_round`` rounds p to
    that dtype before the weight and before y (the
    ``match_pytorch_precision`` semantics, :88-93).  Returns float64
    [B, Hkv, Lk], or [B, Hkv, len(keys)] for the key indices ``keys`` only.

    Used as the arbiter of selections where the float32 reference is not
    decisive: with p rounded to bf16, a last-bit difference in a logit can
    move p to the neighbouring bf16 value (w changes by about 2^-7, and by far
    more where p is close to 1), so two float32 evaluations of the same
    formula can rank keys near the keep threshold differently.  The float64
    evaluation rounds p from a p that is exact to float32 precision.
    ``p_scale`` multiplies p before that rounding: a probe of how far a score
    moves when p is off by a few float32 ulps.

    ``return_bound`` also returns, per key, the scale of the rounding error
    of any float32 evaluation through the expansion:
    ``sum_m w * (|v|^2 + 2|<v,y>| + |y|^2) * 2^-24 / g``.  Where one key takes
    almost all of a row's attention, w reaches 1e12 and this bound exceeds
    the score itself: no float32 expansion determines such a score."""
    B, Hq, Lq, D = Q.shape
    Hkv, Lk = K.shape[1], K.shape[2]
    g = Hq // Hkv
    W = window_size
    Qt = Q[:, :, -W:, :].double()
    Kd, Vd = K.double(), V.double()
    sel = torch.arange(Lk) if keys is None else keys.to(torch.int64)
    out = torch.zeros(B, Hkv, sel.numel(), dtype=torch.float64)
    bound = torch.zeros_like(out)
    mask = torch.triu(torch.full((W, Lk), float("-inf"), dtype=torch.float64), diagonal=Lk - W + 1)
    for hkv in range(Hkv):
        Kh, Vh = Kd[:, hkv], Vd[:, hkv]                      # [B, Lk, D]
        Vs = Vh[:, sel]                                      # [B, n, D]
        vn2 = (Vs ** 2).sum(-1)                              # [B, n]
        for gi in range(g):
            q = Qt[:, hkv * g + gi]                          # [B, W, D]
            p = torch.softmax(q @ Kh.transpose(-1, -2) / math.sqrt(D) + mask, dim=-1)   # [B, W, Lk]
            if p_scale != 1.0:
                p = p * p_scale
            if p_round is not None:
                p = p.to(p_round).double()
            y = p @ Vh                                       # [B, W, D]
            ps = p[:, :, sel]
            wt = (ps / (1.0 - ps + eps)) ** 2
            for w in range(W):
                d2 = ((Vs - y[:, w:w + 1]) ** 2).sum(-1)     # [B, n]
                out[:, hkv] += wt[:, w] * d2
                if return_bound:
                    yw = y[:, w]                             # [B, D]
                    mag = vn2 + 2.0 * (Vs @ yw.unsqueeze(-1)).squeeze(-1).abs() + (yw ** 2).sum(-1, keepdim=True)
                    bound[:, hkv] += wt[:, w] * mag
    if return_bound:
        return out / g, bound * 2.0 ** -24 / g
    return out / g


# ---------------------------------------------------------------------------
# a10: deployed PyTorch scoring path of _compute_keep_indices
#      (dropkv_cache.py:401-460)
# ---------------------------------------------------------------------------

def fallback_scores(
    query_states: torch.Tensor,
    key_states: torch.Tensor,
    value_states: torch.Tensor,
    window_size: int,
    eps: float = 1e-6,
) -> torch.Tensor:
    """GQA-batched scoring used when ``use_triton=False`` or the fast path
    rejects its inputs.  dropkv_cache.py:401-460.

    Differences from ``dropkv_scores_reference`` that matter numerically:
    W = min(window, Lq) (:407); p = softmax(fp32).to(input dtype) (:431);
    y = p @ V in the *input dtype* (:434); ||y||^2 and <v, y> from that
    rounded y (:448-455).
    """
    bsz, Hkv, L, D = key_states.shape
    Hq = query_states.shape[1]
    if Hq % Hkv != 0:
        raise ValueError(f"Query heads {Hq} must be divisible by KV heads {Hkv}")
    g = Hq // Hkv
    W = min(window_size, query_states.shape[2])
    M = g * W
    Q_w = query_states[..., -W:, :].reshape(bsz, Hkv, M, D)
    K_f = key_states.float()
    V_f = value_states.float()
    logits = torch.matmul(Q_w.float(), K_f.transpose(-1, -2)) / math.sqrt(D)
    offs_m = torch.arange(M)
    bounds = L - W + (offs_m % W)
    col = torch.arange(L)
    logits.masked_fill_(col[None, None, None, :] > bounds[None, None, :, None], float("-inf"))
    p = F.softmax(logits, dim=-1, dtype=torch.float32).to(query_states.dtype)
    y = torch.matmul(p, value_states)
    p_f = p.float()
    Wm = (p_f / (1.0 - p_f + eps)) ** 2
    termA = Wm.sum(dim=-2) * (V_f ** 2).sum(dim=-1)
    termB = 2.0 * (Wm.transpose(-1, -2) * torch.matmul(V_f, y.float().transpose(-1, -2))).sum(dim=-1)
    termC = torch.matmul(Wm.transpose(-1, -2), (y.float() ** 2).sum(dim=-1).unsqueeze(-1)).squeeze(-1)
    return (termA - termB + termC) / g


# ---------------------------------------------------------------------------
# a11: max-pool + protect the observation window  (dropkv_cache.py:464-467)
# ---------------------------------------------------------------------------

def pool_protect(scores: torch.Tensor, kernel_size: int, window_size: int) -> torch.Tensor:
    """Sliding max with -inf padding (:464), then the last ``window_size``
    positions become ``amax + 1.0`` computed in fp32 (:465-467)."""
    pooled = F.max_pool1d(scores, kernel_size=kernel_size, padding=kernel_size // 2, stride=1)
    big = pooled.amax(dim=-1, keepdim=True) + 1.0
    if window_size > 0:
        pooled[:, :, -window_size:] = big
    return pooled


# ---------------------------------------------------------------------------
# a12: keep length, top-k, ascending sort  (dropkv_cache.py:470-475)
# ---------------------------------------------------------------------------

def keep_length(keep_ratio: float, seq_len: int, window_size: int,
                total_tokens: Optional[int] = None, max_keep_len: Optional[int] = None) -> int:
    """``min(seq_len, max(int(keep_ratio * base), window_size, 1))`` with
    ``base = total_tokens or seq_len``, then capped by ``max_keep_len``
    (dropkv_cache.py:470-473)."""
    base = total_tokens if total_tokens is not None else seq_len
    keep = min(seq_len, max(int(keep_ratio * base), window_size, 1))
    if max_keep_len is not None:
        keep = min(keep, max_keep_len)
    return keep


def topk_sorted(pooled: torch.Tensor, keep: int) -> torch.Tensor:
    """Indices of the ``keep`` largest values per row, ascending
    (dropkv_cache.py:474-475), with the deterministic rule "lowest index first
    among equal values".  A stable descending sort gives exactly that order.
    Returns int64 [..., keep]."""
    order = torch.sort(pooled, dim=-1, descending=True, stable=True).indices
    return torch.sort(order[..., :keep], dim=-1).values


# ---------------------------------------------------------------------------
# a13: gather into the compressed cache  (dropkv_cache.py:479-491)
# ---------------------------------------------------------------------------

def gather_compressed(key_states: torch.Tensor, value_states: torch.Tensor,
                      keep_idx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``torch.gather(dim=2)`` of K and V with the index broadcast over D."""
    D = key_states.shape[-1]
    idx = keep_idx.unsqueeze(-1).expand(-1, -1, -1, D)
    return torch.gather(key_states, 2, idx), torch.gather(value_states, 2, idx)


# ---------------------------------------------------------------------------
# a10-a13 composed: _compute_keep_indices (dropkv_cache.py:355-477)
# ---------------------------------------------------------------------------

def compute_keep_indices(q, k, v, keep_ratio, window_size, kernel_size,
                         total_tokens=None, max_keep_len=None, scores=None):
    """Deployed CPU path: fallback scores -> pool/protect -> keep -> top-k ->
    sort.  ``scores`` may be supplied to run only the selection part."""
    Lk = k.shape[2]
    if scores is None:
        scores = fallback_scores(q, k, v, window_size)
    pooled = pool_protect(scores.clone(), kernel_size, window_size)
    keep = keep_length(keep_ratio, Lk, window_size, total_tokens, max_keep_len)
    return topk_sorted(pooled, keep), pooled


# ---------------------------------------------------------------------------
# Parity metric: tie-aware index overlap
# ---------------------------------------------------------------------------

def index_overlap(new_idx: torch.Tensor, ref_idx: torch.Tensor, pooled_ref: torch.Tensor):
    """Per-row tie-aware overlap between two kept-index sets.

    Let T be the reference's k-th largest pooled value for the row.  An index
    in the symmetric difference is excused iff ``pooled_ref[index] == T``
    exactly.  Returns (min overlap over rows, total unexcused differences),
    where overlap = 1 - unexcused / keep."""
    rows_new = new_idx.reshape(-1, new_idx.shape[-1])
    rows_ref = ref_idx.reshape(-1, ref_idx.shape[-1])
    pr = pooled_ref.reshape(-1, pooled_ref.shape[-1])
    keep = rows_ref.shape[-1]
    worst, total = 1.0, 0
    for r in range(rows_ref.shape[0]):
        a = set(rows_new[r].tolist())
        b = set(rows_ref[r].tolist())
        T = pr[r][rows_ref[r]].min().item()
        unexcused = sum(1 for i in (a ^ b) if pr[r, i].item() != T)
        total += unexcused
        worst = min(worst, 1.0 - unexcused / keep)
    return worst, total
