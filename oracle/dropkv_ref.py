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


def _fp64_terms(Q, K, V, window_size, eps, p_round, keys, p_scale=1.0, bracket=False):
    """Shared float64 evaluation of the reference score (dropkv_triton.py:29-109)
    for every (b, hkv, gi): the softmax in float64, p scaled by ``p_scale``
    and rounded to ``p_round`` for the weight w = (p/(1-p+eps))^2, y = p @ V
    from the unscaled rounded p, and the distance ||v - y||^2 taken as
    |v|^2 - 2<v,y> + |y|^2 in float64 (clamped at 0; its float64 rounding,
    below 2^-50 of the magnitudes, is far under any float32 evaluation's).

    Returns a dict of float64 [B, Hkv, n] sums over the window rows, divided
    by g: ``s`` the score; ``emag`` the magnitude sum_m w (|v|^2 +
    2 sum_d |v_d y_d| + |y|^2) over which a float32 expansion
    termA - termB + termC (:96-106) rounds.  With ``bracket`` also:
    ``lo`` / ``hi``, the scores with every p at the low / high end of the
    float32 error model ``_p_err32`` before the rounding (w grows with p and
    the rounding is monotone, so these are the least and the largest
    weights any such p rounds to); ``ymag``, per key sum_m w_hi sum_d
    (|v_d| + |y_md|) E_md with E_md = 32 * 2^-24 * sum_j p_mj |v_jd| +
    sum_j (p_hi - p_lo)_mj |v_jd|, a bound on how far a float32 y (a sum over
    up to 131072 keys that cancels: measured off by at most ~21 * 2^-24 of
    sum_j p |v|) and a y from p values at other ends of the model move the
    distance (|d2' - d2| <= 2 sum_d |v_d - y_d| |dy_d|)."""
    B, Hq, Lq, D = Q.shape
    Hkv, Lk = K.shape[1], K.shape[2]
    g = Hq // Hkv
    W = window_size
    Qt = Q[:, :, -W:, :].double()
    Kd, Vd = K.double(), V.double()
    sel = torch.arange(Lk) if keys is None else keys.to(torch.int64)
    n = sel.numel()
    names = ("s", "emag") + (("lo", "hi", "ymag") if bracket else ())
    acc = {k: torch.zeros(B, Hkv, n, dtype=torch.float64) for k in names}
    mask = torch.triu(torch.full((W, Lk), float("-inf"), dtype=torch.float64), diagonal=Lk - W + 1)

    def rnd(x):
        return x.to(p_round).double() if p_round is not None else x

    def weight(x):
        return (x / (1.0 - x + eps)) ** 2

    for hkv in range(Hkv):
        Kh, Vh = Kd[:, hkv], Vd[:, hkv]                      # [B, Lk, D]
        Vs = Vh[:, sel]                                      # [B, n, D]
        vn2 = (Vs ** 2).sum(-1)                              # [B, n]
        for gi in range(g):
            q = Qt[:, hkv * g + gi]                          # [B, W, D]
            logits = q @ Kh.transpose(-1, -2) / math.sqrt(D) + mask     # [B, W, Lk]
            p = torch.softmax(logits, dim=-1)
            p0 = rnd(p)
            y = p0 @ Vh                                      # [B, W, D]
            G = Vs @ y.transpose(-1, -2)                     # [B, n, W]
            yn2 = (y ** 2).sum(-1)                           # [B, W]
            d2 = (vn2[..., None] - 2.0 * G + yn2[:, None, :]).clamp_min(0.0)
            ps = p[:, :, sel].transpose(-1, -2)              # [B, n, W]
            w0 = weight(rnd(ps * p_scale) if p_scale != 1.0 else p0[:, :, sel].transpose(-1, -2))
            acc["s"][:, hkv] += (w0 * d2).sum(-1)
            A = Vs.abs() @ y.abs().transpose(-1, -2)          # sum_d |v_d y_d|, [B, n, W]
            mag = vn2[..., None] + 2.0 * A + yn2[:, None, :]
            if not bracket:
                acc["emag"][:, hkv] += (w0 * mag).sum(-1)
                continue
            err = _p_err32(q, Kh, logits)                    # [B, W, Lk]
            p_lo, p_hi = rnd(p * (1.0 - err)), rnd(p * (1.0 + err))
            w_lo = torch.minimum(weight(p_lo[:, :, sel].transpose(-1, -2)), w0)
            w_hi = torch.maximum(weight(p_hi[:, :, sel].transpose(-1, -2)), w0)
            acc["lo"][:, hkv] += (w_lo * d2).sum(-1)
            acc["hi"][:, hkv] += (w_hi * d2).sum(-1)
            acc["emag"][:, hkv] += (w_hi * mag).sum(-1)
            E = 32.0 * 2.0 ** -24 * (p0 @ Vh.abs()) + (p_hi - p_lo) @ Vh.abs()   # [B, W, D]
            Ey = Vs.abs() @ E.transpose(-1, -2) + (y.abs() * E).sum(-1)[:, None, :]
            acc["ymag"][:, hkv] += (w_hi * Ey).sum(-1)
    return {k: v / g for k, v in acc.items()}


def _p_err32(q, Kh, logits):
    """Relative error of a float32 softmax entry p_mj = exp(l_mj - lse_m):
    the logit is a float32 dot product, off by up to a few 2^-24 of
    a_mj = sum_d |q_d k_d| / sqrt(D) (measured: at most ~5x, 99.9% under
    1.6x at the stress shape); it and the log-sum-exp are held in float32,
    each off by about 2^-24 of its size; and the softmax's denominator, a
    float32 sum over the row's Lk keys, is off by about sqrt(Lk) 2^-24
    (torch's CPU softmax: 3.2e-5 relative measured at Lk = 131072, which
    flips a bf16 rounding).  So
        err_mj = 2^-24 (4 (a_mj + a_m* + |l_mj| + |lse_m| + sqrt(Lk)) + 8),
    m* the row's largest logit."""
    D, Lk = q.shape[-1], Kh.shape[-2]
    a = q.abs() @ Kh.abs().transpose(-1, -2) / math.sqrt(D)             # [B, W, Lk]
    l = torch.nan_to_num(logits, neginf=0.0)
    a_top = torch.gather(a, -1, logits.argmax(-1, keepdim=True))
    lse = torch.logsumexp(logits, -1, keepdim=True)
    return (4.0 * (a + a_top + l.abs() + lse.abs() + math.sqrt(Lk)) + 8.0) * 2.0 ** -24


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
    """The score of ``dropkv_scores_reference`` evaluated in float64
    (the terms of ``_fp64_terms``) instead of the float32 expansion
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
    ``p_scale`` multiplies p before that rounding (the weight only; y keeps
    the unscaled p): a probe of how far a score moves when p is off by a few
    float32 ulps.

    ``return_bound`` also returns, per key, the scale of the rounding error
    of any float32 evaluation through the expansion:
    ``sum_m w * (|v|^2 + 2|<v,y>| + |y|^2) * 2^-24 / g``.  Where one key takes
    almost all of a row's attention, w reaches 1e12 and this bound exceeds
    the score itself: no float32 expansion determines such a score."""
    t = _fp64_terms(Q, K, V, window_size, eps, p_round, keys, p_scale=p_scale)
    if return_bound:
        return t["s"], t["emag"] * 2.0 ** -24
    return t["s"]


def dropkv_score_bracket(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    window_size: int = 8,
    eps: float = 1e-6,
    p_round: Optional[torch.dtype] = None,
    bound_factor: float = 16.0,
    keys: Optional[torch.Tensor] = None,
):
    """Per key, float64 ``(score, lo, hi)``: the float64 score of
    ``dropkv_scores_fp64`` and an interval that holds the value a float32
    evaluation of the reference formula (dropkv_triton.py:29-109) returns for
    it, as far as its rounding is modelled (``_fp64_terms``):
    * p off by the float32 softmax error ``_p_err32`` before the bf16
      rounding (flips to the neighbouring bf16 value): the weights from the
      low and high ends of p;
    * y off by its float32 summation error and by those p flips: the
      distance moved by at most 2 ``ymag``;
    * the expansion |v|^2 - 2<v,y> + |y|^2 rounding away up to
      ``bound_factor`` * 2^-24 of the magnitudes it cancels, which at an
      attention sink (p ~ 1, w ~ 1e12) exceeds the score itself.
    The float32 reference (and any float32 implementation of the formula)
    stays inside; ``tests/test_oracle.py`` checks it on the configurations'
    row shapes."""
    t = _fp64_terms(Q, K, V, window_size, eps, p_round, keys, bracket=True)
    slack = bound_factor * 2.0 ** -24 * t["emag"] + 2.0 * t["ymag"]
    return t["s"], t["lo"] - slack, t["hi"] + slack


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

def selection_band(lo: torch.Tensor, hi: torch.Tensor, kernel_size: int, protect: int, keep: int) -> torch.Tensor:
    """Indices whose selection the reference formula does not decide, given
    per-key score brackets ``lo <= score <= hi`` (``dropkv_score_bracket``):
    bool [..., Lk].

    Max-pooling is monotone, so pooled values lie in [pool(lo), pool(hi)];
    the keep-th largest pooled value T of the unprotected keys then lies in
    [T_lo, T_hi], the same order statistic of pool(lo) and of pool(hi).  An
    index with pool(lo) > T_hi is above every possible T (kept by every
    evaluation inside the brackets), one with pool(hi) < T_lo below every
    possible T (never kept); the protected tail is always kept
    (dropkv_cache.py:464-475).  Every other index is undecided: its pooled
    bracket meets the threshold band."""
    Lk = lo.shape[-1]
    ks = kernel_size
    plo = F.max_pool1d(lo.double(), ks, padding=ks // 2, stride=1)
    phi = F.max_pool1d(hi.double(), ks, padding=ks // 2, stride=1)
    n = max(Lk - protect, 0)
    kf = keep - (Lk - n)
    und = torch.zeros(lo.shape, dtype=torch.bool)
    if n > 0 and kf > 0:
        t_lo = torch.topk(plo[..., :n], kf, dim=-1).values[..., -1:]
        t_hi = torch.topk(phi[..., :n], kf, dim=-1).values[..., -1:]
        und[..., :n] = ~((plo[..., :n] > t_hi) | (phi[..., :n] < t_lo))
    return und


def index_overlap(new_idx: torch.Tensor, ref_idx: torch.Tensor, pooled_ref: torch.Tensor,
                  undecided: Optional[torch.Tensor] = None, return_counts: bool = False):
    """Per-row overlap between two kept-index sets, with every index of the
    symmetric difference either excused for a named reason or counted.

    Let T be the reference's k-th largest pooled value for the row.  An index
    in the symmetric difference is excused
      (tie)  if ``pooled_ref[index] == T`` exactly: torch.topk's choice among
             equal values is open; or
      (band) if ``undecided[index]`` (``selection_band``): the reference
             formula does not decide that index at float32 precision (its
             pooled bracket meets the threshold band; at an attention sink
             the bracket spans the whole pooling window, and the keys it
             displaces across the threshold lie inside the band too).
    Every other index counts.  Returns (min overlap over rows, total counted
    differences), overlap = 1 - counted / keep; with ``return_counts`` also
    the totals excused as ties and as band indices."""
    rows_new = new_idx.reshape(-1, new_idx.shape[-1])
    rows_ref = ref_idx.reshape(-1, ref_idx.shape[-1])
    pr = pooled_ref.reshape(-1, pooled_ref.shape[-1])
    und = undecided.reshape(-1, undecided.shape[-1]) if undecided is not None else None
    keep = rows_ref.shape[-1]
    worst, total, n_tie, n_band = 1.0, 0, 0, 0
    for r in range(rows_ref.shape[0]):
        a = set(rows_new[r].tolist())
        b = set(rows_ref[r].tolist())
        T = pr[r][rows_ref[r]].min().item()
        unexcused = 0
        for i in a ^ b:
            if pr[r, i].item() == T:
                n_tie += 1
            elif und is not None and bool(und[r, i]):
                n_band += 1
            else:
                unexcused += 1
        total += unexcused
        worst = min(worst, 1.0 - unexcused / keep)
    if return_counts:
        return worst, total, n_tie, n_band
    return worst, total
