"""Pins the CPU oracle (oracle/dropkv_ref.py) independently of its own code.

Each oracle function is checked against something that does not share its
formula: a float64 brute force with the direct ||v - y||^2 distance, closed
forms, invariants and the golden fixtures (written by
tests/golden/make_golden.py from the mathematics).  A plausible mistake --
a dropped 1/g, a causal bound off by one, the wrong head grouping, eps
missing, the protect value, the tie rule -- fails at least one of these.
CPU only.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import golden_case, golden_names, make_qkv
from oracle import dropkv_ref as R

EPS = 1e-6


def brute_fp64(Q, K, V, W, p_round=None, y_round=None):
    """float64 brute force over (b, hkv, gi, w) with the direct distance
    ||v_j - y_m||^2 (dropkv_triton.py:29-109 semantics; rounding optional)."""
    Q, K, V = Q.double(), K.double(), V.double()
    B, Hq, Lq, D = Q.shape
    Hkv, Lk = K.shape[1], K.shape[2]
    g = Hq // Hkv
    out = torch.zeros(B, Hkv, Lk, dtype=torch.float64)
    for b in range(B):
        for h in range(Hkv):
            for gi in range(g):
                for w in range(W):
                    q = Q[b, h * g + gi, Lq - W + w]
                    bound = Lk - W + w
                    logit = K[b, h, :bound + 1] @ q / math.sqrt(D)
                    p = torch.softmax(logit, 0)
                    if p_round is not None:
                        p = p.float().to(p_round).double()
                    y = p @ V[b, h, :bound + 1]
                    if y_round is not None:
                        y = y.float().to(y_round).double()
                    wt = (p / (1.0 - p + EPS)) ** 2
                    d2 = ((V[b, h, :bound + 1] - y) ** 2).sum(-1)
                    out[b, h, :bound + 1] += wt * d2
            out[b, h] /= g
    return out


def assert_rel(got, ref, rtol):
    """|got-ref| <= rtol*|ref| + 1e-6*rowmax (scores span orders of magnitude)."""
    got, ref = got.double(), ref.double()
    atol = 1e-6 * ref.abs().amax(dim=-1, keepdim=True)
    bad = (got - ref).abs() > rtol * ref.abs() + atol
    assert not bad.any(), f"{int(bad.sum())} keys outside rtol {rtol}"


SHAPES = [
    # (B, Hq, Hkv, D, Lq, Lk, W)
    (1, 4, 2, 32, 40, 40, 8),
    (2, 6, 3, 16, 12, 50, 4),      # Lq < Lk, B=2, g=2
    (1, 3, 3, 32, 20, 33, 8),      # MHA (g=1)
    (1, 8, 2, 32, 12, 12, 9),      # Lk close to W: the first row sees 4 keys
]


def test_reference_l_equals_w_finite():
    """Lk == W: row 0 sees one key, p = 1 and w = 1/eps^2; the fp32
    expansion termA - termB + termC then cancels catastrophically at that key
    (the reference's tests check only finiteness there, tests:385-396)."""
    Q, K, V = make_qkv(dict(B=1, Hq=8, Hkv=2, D=32), 9, 9, dtype=torch.float32, seed=13)
    s = R.dropkv_scores_reference(Q, K, V, 9)
    assert torch.isfinite(s).all()
    assert_rel(s[..., 1:], brute_fp64(Q, K, V, 9)[..., 1:], 1e-3)


@pytest.mark.parametrize("shape", SHAPES)
def test_reference_fp32_vs_bruteforce(shape):
    B, Hq, Hkv, D, Lq, Lk, W = shape
    cfg = dict(B=B, Hq=Hq, Hkv=Hkv, D=D)
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=torch.float32, seed=sum(shape))
    got = R.dropkv_scores_reference(Q, K, V, W, match_pytorch_precision=False)
    assert got.dtype == torch.float32 and got.shape == (B, Hkv, Lk)
    assert_rel(got, brute_fp64(Q, K, V, W), 1e-4)


@pytest.mark.parametrize("shape", SHAPES[:3])
def test_reference_bf16_mode_vs_bruteforce(shape):
    """p rounded to bf16 before the weight (dropkv_triton.py:88-92)."""
    B, Hq, Hkv, D, Lq, Lk, W = shape
    cfg = dict(B=B, Hq=Hq, Hkv=Hkv, D=D)
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=torch.bfloat16, seed=1 + sum(shape))
    got = R.dropkv_scores_reference(Q, K, V, W, match_pytorch_precision=True)
    ref = brute_fp64(Q, K, V, W, p_round=torch.bfloat16)
    # p computed in float32 vs float64 can round to different bf16 neighbours
    # when it sits next to a rounding boundary: w then moves by ~2^-7.
    rel = (got.double() - ref).abs() / ref.abs().clamp_min(1e-30)
    assert rel.max() < 2e-2
    assert (rel > 1e-4).double().mean() < 0.03


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("p_round", [None, torch.bfloat16])
def test_fp64_arbiter_vs_bruteforce(shape, p_round):
    """The vectorised float64 evaluation equals the per-(b, hkv, gi, w)
    brute force to float64 rounding."""
    B, Hq, Hkv, D, Lq, Lk, W = shape
    cfg = dict(B=B, Hq=Hq, Hkv=Hkv, D=D)
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=torch.bfloat16, seed=7 + sum(shape))
    got = R.dropkv_scores_fp64(Q, K, V, W, p_round=p_round)
    ref = brute_fp64(Q, K, V, W, p_round=p_round)
    assert got.dtype == torch.float64
    assert_rel(got, ref, 1e-12)
    keys = torch.tensor([0, Lk // 2, Lk - 1])
    assert_rel(R.dropkv_scores_fp64(Q, K, V, W, p_round=p_round, keys=keys), got[..., keys], 1e-13)


def test_fp64_arbiter_rounding_bound():
    """The float32-expansion rounding bound is negligible for diffuse
    attention and exceeds the score at an attention sink (p rounds to 1)."""
    cfg = dict(B=1, Hq=2, Hkv=1, D=32)
    Q, K, V = make_qkv(cfg, 64, 64, dtype=torch.bfloat16, seed=3)
    s, bnd = R.dropkv_scores_fp64(Q, K, V, 8, p_round=torch.bfloat16, return_bound=True)
    assert (bnd >= 0).all() and (bnd / s).max() < 1e-4
    K = K.clone()
    K[0, 0, 20] = (Q[0, 0, -1].float() * 4).to(torch.bfloat16)   # key 20 takes the last row's attention
    s, bnd = R.dropkv_scores_fp64(Q, K, V, 8, p_round=torch.bfloat16, return_bound=True)
    assert bnd[0, 0, 20] > s[0, 0, 20]


@pytest.mark.parametrize("shape", SHAPES[:3] + [(1, 4, 2, 32, 3, 40, 8)])
def test_fallback_vs_bruteforce(shape):
    """Deployed path: W = min(window, Lq), p and y rounded to the input dtype
    (dropkv_cache.py:407, :431, :434)."""
    B, Hq, Hkv, D, Lq, Lk, W = shape
    cfg = dict(B=B, Hq=Hq, Hkv=Hkv, D=D)
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=torch.bfloat16, seed=2 + sum(shape))
    got = R.fallback_scores(Q, K, V, W)
    ref = brute_fp64(Q, K, V, min(W, Lq), p_round=torch.bfloat16, y_round=torch.bfloat16)
    # y rounding from a float32 vs float64 accumulation can land on either
    # side of a bf16 boundary; that moves a key's distance by ~2^-8 relative.
    rel = (got.double() - ref).abs() / ref.abs().clamp_min(1e-30)
    assert rel.max() < 2e-2
    assert (rel > 1e-4).double().mean() < 0.02


def test_fallback_close_to_reference_bf16_mode():
    """The reference's own relation between its oracle (match=True) and the
    deployed path (tests/test_dropkv_triton.py:105-115: rtol 5e-2, atol 5e-3)."""
    Q, K, V = make_qkv(dict(B=1, Hq=8, Hkv=2, D=64), 256, dtype=torch.bfloat16, seed=3)
    a = R.dropkv_scores_reference(Q, K, V, 8, match_pytorch_precision=True)
    b = R.fallback_scores(Q, K, V, 8)
    torch.testing.assert_close(a, b, rtol=5e-2, atol=5e-3)


def test_v_zero_scores_zero():
    Q, K, V = make_qkv(dict(B=1, Hq=4, Hkv=2, D=32), 30, dtype=torch.float32, seed=4)
    s = R.dropkv_scores_reference(Q, K, torch.zeros_like(V), 8)
    assert torch.count_nonzero(s) == 0


def test_q_zero_uniform_closed_form():
    """Q = 0: row w attends uniformly to keys 0..Lk-W+w, y_w = prefix mean;
    score_j = (1/g) sum_w [j <= b_w] (p_w/(1-p_w+eps))^2 ||v_j - mean_w||^2
    with p_w = 1/(b_w+1).  g copies of the same rows average to one copy."""
    cfg = dict(B=1, Hq=2, Hkv=1, D=16)
    _, K, V = make_qkv(cfg, 20, 20, dtype=torch.float32, seed=5)
    Q = torch.zeros(1, 2, 20, 16)
    W, Lk = 4, 20
    got = R.dropkv_scores_reference(Q, K, V, W).double()
    Vd = V[0, 0].double()
    ref = torch.zeros(Lk, dtype=torch.float64)
    for w in range(W):
        bnd = Lk - W + w
        p = 1.0 / (bnd + 1)
        mean = Vd[:bnd + 1].mean(0)
        ref[:bnd + 1] += (p / (1 - p + EPS)) ** 2 * ((Vd[:bnd + 1] - mean) ** 2).sum(-1)
    torch.testing.assert_close(got[0, 0], ref, rtol=1e-5, atol=1e-9)


def test_two_key_logit_gap_closed_form():
    """Row 0 of a Lk = W+1 head sees keys 0 and 1.  With a logit gap of 4,
    p0 = 1/(1+e^-4), y = p0 v0 + p1 v1, so row 0 gives key 0
    (p0/(p1+eps))^2 * p1^2 ||v0-v1||^2 -- pins the weight (p/(1-p+eps))^2
    (a weight of p^2, or of p/(1-p) unsquared, misses by orders of magnitude).
    eps itself is below the float32 resolution of the reference's expansion
    here; its presence is pinned by the p = 1 case of
    test_reference_l_equals_w_finite (without it the weight is infinite)."""
    D, W = 16, 4
    Lk = W + 1
    q = torch.zeros(1, 1, Lk, D)
    q[0, 0, Lk - W, 0] = 4.0 * math.sqrt(D)    # row 0 (position Lk-W): logit gap 4
    K = torch.zeros(1, 1, Lk, D)
    K[0, 0, 0, 0] = 1.0                          # key 0: logit 4, key 1: logit 0
    g = torch.Generator().manual_seed(6)
    V = torch.randn(1, 1, Lk, D, generator=g)
    got = R.dropkv_scores_reference(q, K, V, W).double()[0, 0, 0]
    p0 = 1.0 / (1.0 + math.exp(-4.0))
    p1 = 1.0 - p0
    d01 = float(((V[0, 0, 0] - V[0, 0, 1]).double() ** 2).sum())
    # rows w >= 1 have zero queries: uniform over keys 0..w+1
    others = 0.0
    for w in range(1, W):
        n = Lk - W + w + 1
        p = 1.0 / n
        mean = V[0, 0, :n].double().mean(0)
        others += (p / (1 - p + EPS)) ** 2 * float(((V[0, 0, 0].double() - mean) ** 2).sum())
    ref = (p0 / (p1 + EPS)) ** 2 * p1 ** 2 * d01 + others
    assert abs(got - ref) / ref < 1e-3


def test_gqa_grouping_and_average():
    """Query heads hkv*g .. hkv*g+g-1 belong to KV head hkv (contiguous
    grouping, dropkv_triton.py:73); duplicating every query head g times
    leaves the score unchanged (the 1/g average), and permuting heads inside
    a group does not matter while moving one across groups does."""
    cfg = dict(B=1, Hq=3, Hkv=3, D=32)
    Q1, K, V = make_qkv(cfg, 24, 24, dtype=torch.float32, seed=7)
    s1 = R.dropkv_scores_reference(Q1, K, V, 8)
    Q2 = Q1.repeat_interleave(2, dim=1)        # heads 2h, 2h+1 = head h
    s2 = R.dropkv_scores_reference(Q2, K, V, 8)
    torch.testing.assert_close(s2, s1, rtol=1e-5, atol=1e-9)
    Q4 = torch.cat([Q1, Q1.flip(1)], dim=1).reshape(1, 2, 3, 24, 32).transpose(1, 2).reshape(1, 6, 24, 32)
    s4 = R.dropkv_scores_reference(Q4, K, V, 8)
    Q5 = Q4[:, [1, 0, 2, 3, 4, 5]]             # swap inside group 0
    torch.testing.assert_close(R.dropkv_scores_reference(Q5, K, V, 8), s4, rtol=1e-5, atol=1e-9)
    Q6 = Q4[:, [2, 1, 0, 3, 4, 5]]             # move a head across groups
    assert not torch.allclose(R.dropkv_scores_reference(Q6, K, V, 8), s4, rtol=1e-3)


def test_only_query_tail_is_read():
    """scores(Q) == scores(Q[..., -W:, :]) bit for bit; rows before the tail
    can hold anything."""
    cfg = dict(B=1, Hq=4, Hkv=2, D=32)
    Q, K, V = make_qkv(cfg, 40, 64, dtype=torch.float32, seed=8)
    a = R.dropkv_scores_reference(Q, K, V, 8)
    Qn = Q.clone()
    Qn[:, :, :-8] = float("nan")
    b = R.dropkv_scores_reference(Qn[:, :, -8:], K, V, 8)
    c = R.dropkv_scores_reference(Qn, K, V, 8)
    assert torch.equal(a, b) and torch.equal(a, c)


def test_causal_bound_tail_aligned():
    """Key Lk-W+w+1 .. is invisible to window row w: changing the last key
    only changes the score of that key through the last row."""
    cfg = dict(B=1, Hq=2, Hkv=1, D=16)
    Q, K, V = make_qkv(cfg, 16, 16, dtype=torch.float64, seed=9)
    W = 4
    ref = brute_fp64(Q, K, V, W)
    K2 = K.clone()
    K2[0, 0, -1] *= 3.0
    ref2 = brute_fp64(Q, K2, V, W)
    # rows 0..W-2 never see key Lk-1; only the last row does -> every key's
    # score changes (through that row's softmax) but the contribution of rows
    # 0..W-2 to key Lk-2 is unchanged: check via the brute force per row
    got = R.dropkv_scores_reference(Q.float(), K.float(), V.float(), W).double()
    got2 = R.dropkv_scores_reference(Q.float(), K2.float(), V.float(), W).double()
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-9)
    torch.testing.assert_close(got2, ref2, rtol=1e-5, atol=1e-9)


def test_scores_nonnegative_up_to_rounding():
    Q, K, V = make_qkv(dict(B=1, Hq=8, Hkv=2, D=64), 128, dtype=torch.bfloat16, seed=10)
    s = R.dropkv_scores_reference(Q, K, V, 8, match_pytorch_precision=True)
    assert (s >= -1e-6 * s.abs().max()).all()


# ---------------------------------------------------------------------------
# pool / protect / keep length / top-k / gather
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("ks,window", [(11, 8), (1, 8), (3, 0), (7, 32)])
def test_pool_protect_bruteforce(ks, window):
    g = torch.Generator().manual_seed(ks * 10 + window)
    s = torch.randn(2, 3, 100, generator=g)
    got = R.pool_protect(s.clone(), ks, window)
    h = ks // 2
    ref = torch.empty_like(s)
    for j in range(100):
        ref[..., j] = s[..., max(0, j - h):min(100, j + h + 1)].amax(-1)
    big = ref.amax(-1, keepdim=True) + 1.0
    if window > 0:
        ref[..., 100 - window:] = big
    assert torch.equal(got, ref)


def test_protect_big_absorbed_in_float32():
    """max >= 2^24: max + 1.0f == max (dropkv_cache.py:465 in fp32)."""
    s = torch.zeros(1, 1, 50)
    s[0, 0, 10] = 2.0 ** 25
    got = R.pool_protect(s.clone(), 3, 4)
    assert (got[0, 0, -4:] == 2.0 ** 25).all()


@pytest.mark.parametrize("ratio,L,expect", [
    (0.1, 512, 51), (0.1, 32768, 3276), (0.1, 16384, 1638), (0.1, 65536, 6553),
    (0.05, 131072, 6553), (0.3, 128, 38), (0.01, 64, 8), (1.0, 100, 100),
])
def test_keep_length_table(ratio, L, expect):
    assert R.keep_length(ratio, L, 8) == expect


def test_keep_length_total_tokens_and_cap():
    """Reference tests:909-937, :1183-1204."""
    assert R.keep_length(0.3, 128, 8, total_tokens=512) == 128     # capped at seq_len
    assert R.keep_length(0.3, 128, 8, total_tokens=200) == 60
    assert R.keep_length(0.01, 64, 8, total_tokens=10) == 8         # window floor
    assert R.keep_length(0.8, 512, 8, total_tokens=512, max_keep_len=100) == 100
    assert R.keep_length(0.5, 4, 8) == 4                            # never above seq_len


def _rank_rule(x, keep):
    n = x.numel()
    return [i for i in range(n)
            if int((x > x[i]).sum()) + int((x[:i] == x[i]).sum()) < keep]


@pytest.mark.parametrize("seed", range(6))
def test_topk_sorted_rank_rule(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randint(0, 6, (4, 40), generator=g).float()
    keep = 1 + seed * 5
    got = R.topk_sorted(x.view(1, 4, 40), keep)[0]
    for r in range(4):
        assert got[r].tolist() == _rank_rule(x[r], keep)


def test_topk_sorted_vs_torch_topk_tie_aware():
    g = torch.Generator().manual_seed(11)
    x = torch.randint(0, 30, (1, 3, 500), generator=g).float()
    pooled = R.pool_protect(x.clone(), 11, 8)
    keep = 77
    mine = R.topk_sorted(pooled, keep)
    theirs = torch.sort(torch.topk(pooled, keep, dim=-1).indices, dim=-1).values
    worst, unexcused = R.index_overlap(mine, theirs, pooled)
    assert unexcused == 0 and worst == 1.0
    for r in range(3):   # equal multisets of kept values
        assert torch.equal(torch.sort(pooled[0, r, mine[0, r]]).values,
                           torch.sort(pooled[0, r, theirs[0, r]]).values)


def test_index_overlap_catches_planted_mistake():
    pooled = torch.arange(20, dtype=torch.float32).view(1, 1, 20).clone()
    pooled[0, 0, 10] = pooled[0, 0, 11] = 100.0          # a tie pair, above everything
    ref = R.topk_sorted(pooled, 5)                        # 10, 11, 17, 18, 19
    assert ref[0, 0].tolist() == [10, 11, 17, 18, 19]
    wrong = ref.clone()
    wrong[0, 0, 3] = 3                                    # 18 -> 3: neither is a tie
    worst, unexcused = R.index_overlap(torch.sort(wrong, -1).values, ref, pooled)
    assert unexcused == 2 and worst == pytest.approx(1 - 2 / 5)
    wrong = ref.clone()
    wrong[0, 0, 2] = 3                                    # 17 (the threshold) -> 3
    worst, unexcused = R.index_overlap(torch.sort(wrong, -1).values, ref, pooled)
    assert unexcused == 1                                 # only 3 is unexcused
    pooled2 = pooled.clone()
    pooled2[0, 0, 16] = pooled2[0, 0, 17]                 # 16 ties the threshold 17
    ref2 = R.topk_sorted(pooled2, 5)
    assert ref2[0, 0].tolist() == [10, 11, 16, 18, 19]   # lowest index wins the tie
    swapped = ref2.clone()
    swapped[0, 0, 2] = 17
    worst, unexcused = R.index_overlap(torch.sort(swapped, -1).values, ref2, pooled2)
    assert unexcused == 0


# ---------------------------------------------------------------------------
# score brackets and the selection band (the excuse rule of index_overlap)
# ---------------------------------------------------------------------------

def _t3_case(seed, L=16384, g=8, W=32, D=128):
    """One KV head of the stress configuration's statistics (Student-t(3)
    keys, N(0,1) queries and values, GQA 8, window 32) at a CPU-sized Lk."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(1, g, W, D, generator=gen).to(torch.bfloat16)
    z = torch.randn(1, 1, L, D, generator=gen)
    chi2 = sum(torch.randn(1, 1, L, D, generator=gen) ** 2 for _ in range(3))
    k = (z / torch.sqrt(chi2 / 3)).to(torch.bfloat16)
    v = torch.randn(1, 1, L, D, generator=gen).to(torch.bfloat16)
    return q, k, v


def _permuted_reference(q, k, v, W, seed):
    """The float32 reference on the same keys in another order (the prefix
    every window row sees is permuted; the causal tail stays in place):
    the same mathematics, other float32 summation orders in the softmax
    denominator, y = p @ V and the expansion."""
    L = k.shape[2]
    perm = torch.cat([torch.randperm(L - W, generator=torch.Generator().manual_seed(seed)), torch.arange(L - W, L)])
    s = R.dropkv_scores_reference(q, k[:, :, perm], v[:, :, perm], W, match_pytorch_precision=True)
    out = torch.empty_like(s)
    out[..., perm] = s
    return out


@pytest.mark.parametrize("case", ["t3-0", "t3-9", "lognormal", "gauss"])
def test_bracket_holds_float32_evaluations(case):
    """Every key's float32 reference score, and that of a float32 evaluation
    in another summation order, lies in the key's bracket; off the heavy
    tails the brackets are narrow (median relative width under 1e-3)."""
    if case.startswith("t3"):
        q, k, v = _t3_case(int(case[3:]))
        W = 32
    else:
        cfg = dict(B=1, Hq=16, Hkv=4, D=128)
        Q, k, v = make_qkv(cfg, 4096, seed=21, k_scale="lognormal" if case == "lognormal" else None)
        W = 8
        q = Q[:, :, -W:].contiguous()
    s, lo, hi = R.dropkv_score_bracket(q, k, v, W, p_round=torch.bfloat16)
    assert (lo <= s).all() and (s <= hi).all()
    for r32 in (R.dropkv_scores_reference(q, k, v, W, match_pytorch_precision=True), _permuted_reference(q, k, v, W, 5)):
        r = r32.double()
        out = (r < lo) | (r > hi)
        assert not out.any(), (case, int(out.sum()), torch.nonzero(out.flatten())[:5].flatten().tolist())
    if not case.startswith("t3"):
        width = (hi - lo) / s.abs().clamp_min(1e-300)
        assert width.median() < 1e-3


def test_bracket_catches_a_dropped_term():
    """Without the y term the bracket misses float32 values at the stress
    statistics, and without the p-error model it misses p values that round
    to the other bf16 neighbour: both are needed, neither is padding."""
    q, k, v = _t3_case(9)
    W = 32
    r = R.dropkv_scores_reference(q, k, v, W, match_pytorch_precision=True).double()
    t = R._fp64_terms(q, k, v, W, 1e-6, torch.bfloat16, None, bracket=True)
    u = 2.0 ** -24
    no_y = ((r < t["lo"] - 16 * u * t["emag"]) | (r > t["hi"] + 16 * u * t["emag"])).sum()
    no_p = ((r < t["s"] - 16 * u * t["emag"] - 2 * t["ymag"]) | (r > t["s"] + 16 * u * t["emag"] + 2 * t["ymag"])).sum()
    assert int(no_y) > 0 and int(no_p) > 0, (int(no_y), int(no_p))


def test_band_excuses_undecided_indices_and_counts_the_rest():
    """Heavy-tailed keys: the float32 reference's selection differs from the
    float64 evaluation's in tens of indices (attention sinks whose score no
    float32 expansion determines move whole pooling windows across the
    threshold, and displace the keys at the threshold).  The band excuses
    every one of them; a planted swap of a kept key far above the band with
    a dropped key far below it is counted, as is a planted swap inside the
    decided region next to a band index."""
    q, k, v = _t3_case(9)
    W, ks, ratio = 32, 11, 0.05
    L = k.shape[2]
    keep = R.keep_length(ratio, L, W)
    r32 = R.dropkv_scores_reference(q, k, v, W, match_pytorch_precision=True)
    s, lo, hi = R.dropkv_score_bracket(q, k, v, W, p_round=torch.bfloat16)
    i32, p32 = R.compute_keep_indices(q, k, v, ratio, W, ks, scores=r32)
    i64, _ = R.compute_keep_indices(q, k, v, ratio, W, ks, scores=s)
    und = R.selection_band(lo, hi, ks, W, keep)
    _, ties_only = R.index_overlap(i64, i32, p32)
    assert ties_only >= 10                                    # the rule is needed here
    worst, counted, n_tie, n_band = R.index_overlap(i64, i32, p32, undecided=und, return_counts=True)
    assert counted == 0 and n_band >= 10 and worst == 1.0
    assert int(und.sum()) < 0.5 * keep                        # most of the selection is decided
    # planted: the most certain kept key out, the most certain dropped key in
    plo = F.max_pool1d(lo.double(), ks, padding=ks // 2, stride=1)[0, 0]
    phi = F.max_pool1d(hi.double(), ks, padding=ks // 2, stride=1)[0, 0]
    kept = set(i64[0, 0].tolist())
    free = [j for j in range(L - W) if not und[0, 0, j]]
    best_in = max((j for j in free if j in kept), key=lambda j: float(plo[j]))
    best_out = min((j for j in free if j not in kept), key=lambda j: float(phi[j]))
    wrong = torch.tensor(sorted((kept - {best_in}) | {best_out})).view(1, 1, -1)
    _, counted = R.index_overlap(wrong, i32, p32, undecided=und)
    assert counted == 2


def test_selection_band_closed_forms():
    """Exact brackets (lo == hi) leave only the threshold's plateau
    undecided; a bracket covering everything leaves every unprotected index
    undecided; the protected tail is always decided (kept)."""
    g = torch.Generator().manual_seed(4)
    x = torch.rand(1, 2, 300, generator=g, dtype=torch.float64)
    und = R.selection_band(x, x, 1, 8, 30)
    assert int(und.sum()) == 2                                # per row: the threshold key itself
    pooled = R.pool_protect(x.float().clone(), 1, 8)
    T = torch.topk(pooled, 30, dim=-1).values[..., -1:]
    assert torch.equal(und, (pooled == T) & (torch.arange(300) < 292))
    und = R.selection_band(torch.zeros_like(x), torch.ones_like(x), 5, 8, 30)
    assert und[..., :292].all() and not und[..., 292:].any()
    und = R.selection_band(x, x, 5, 8, 8)                     # keep == protect: nothing else kept
    assert not und.any()


def test_gather_bit_exact():
    g = torch.Generator().manual_seed(12)
    K = torch.randn(2, 3, 50, 8, generator=g).to(torch.bfloat16)
    V = torch.randn(2, 3, 50, 8, generator=g).to(torch.bfloat16)
    idx = torch.sort(torch.randint(0, 50, (2, 3, 9), generator=g), -1).values
    k, v = R.gather_compressed(K, V, idx)
    for b in range(2):
        for h in range(3):
            assert torch.equal(k[b, h], K[b, h, idx[b, h]])
            assert torch.equal(v[b, h], V[b, h, idx[b, h]])


# ---------------------------------------------------------------------------
# golden fixtures (float64 brute force written by tests/golden/make_golden.py)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", golden_names())
def test_oracle_vs_golden(name):
    c = golden_case(name)
    B, Hq, Hkv, D, Lq, Lk, W, ks, keep = c["meta"]
    q, k, v = c["q"], c["k"], c["v"]
    if "exact" in c:
        assert_rel(R.dropkv_scores_reference(q, k, v, W, match_pytorch_precision=False), c["exact"], 1e-4)
        assert_rel(R.dropkv_scores_reference(q, k, v, W, match_pytorch_precision=True), c["bf16p"], 1e-4)
        assert torch.equal(R.topk_sorted(c["pooled_bf16p"], keep), c["keep_idx_bf16p"])
        assert torch.equal(R.pool_protect(torch.from_numpy(c["bf16p_np"].astype(np.float32)), ks, W),
                           c["pooled_bf16p"])
    assert_rel(R.fallback_scores(q, k, v, W), c["deployed"], 1e-4)
    assert torch.equal(R.topk_sorted(c["pooled_deployed"], keep), c["keep_idx_deployed"])
    assert R.keep_length(float(c["ratio"]), Lk, W) == keep


def test_binding_bars_bind():
    """The full-size score bars (conftest.assert_binding_scores) catch a
    2e-2 error on one key above 0.1x the keep threshold and a 1e-3 error on
    more than 1e-3 of those keys, and ignore any error on keys far below."""
    from conftest import assert_binding_scores, binding_keys
    Q, K, V = make_qkv(dict(B=1, Hq=4, Hkv=2, D=32), 600, seed=31)
    W, ks, keep = 8, 5, 60
    Qt = Q[:, :, -W:].contiguous()
    ref = R.dropkv_scores_reference(Qt, K, V, W, match_pytorch_precision=False)
    pooled = R.pool_protect(ref.clone(), ks, W)
    sel = binding_keys(ref, pooled, keep)
    assert 0 < int(sel.sum()) < sel.numel()
    n, worst, above, _ = assert_binding_scores(ref.clone(), ref, pooled, keep, Qt, K, V, W, None, 1e-4, 1e-4, 1.0,
                                               excuse_sinks=False)
    assert n == int(sel.sum()) and worst == 0.0 and above == 0
    far = (~sel).nonzero()[0].tolist()
    bad = ref.clone()
    bad[tuple(far)] *= 10.0                      # a key far below the threshold: not bound
    assert_binding_scores(bad, ref, pooled, keep, Qt, K, V, W, None, 1e-4, 1e-4, 1.0, excuse_sinks=False)
    hit = sel.nonzero()[0].tolist()
    bad = ref.clone()
    bad[tuple(hit)] *= 1.0 + 3e-2                # one binding key off by 3%
    with pytest.raises(AssertionError):
        assert_binding_scores(bad, ref, pooled, keep, Qt, K, V, W, None, 2e-2, 1e-3, 1e-3, excuse_sinks=False)
    bad = ref.clone()
    idx = sel.nonzero()[:2]
    for i in idx.tolist():
        bad[tuple(i)] *= 1.0 + 5e-3              # two binding keys off by 0.5%: above the 1e-3 share of ~100
    with pytest.raises(AssertionError):
        assert_binding_scores(bad, ref, pooled, keep, Qt, K, V, W, None, 2e-2, 1e-3, 1e-3, excuse_sinks=False)
