"""Write the golden fixtures in this directory (``dropkv_golden.npz``).

The expected outputs are computed here by an independent float64 NumPy brute
force of the DropKV eviction path, written from the mathematics rather than
from the oracle's code:

* score_j = (1/g) * sum over the g*W window rows m of
  (p/(1-p+eps))^2 * ||v_j - y_m||^2, with the *direct* squared distance
  (the oracle and the kernels use the expansion |v|^2 - 2<y,v> + |y|^2);
  p = softmax of q_m.k_j/sqrt(D) over keys j <= Lk-W+w, y_m = sum_j p v_j
  (reference: dropkv_triton.py:29-109);
* the bf16 variant rounds p to bfloat16 before the weight
  (dropkv_triton.py:88-92, :584-587); the deployed-path variant also rounds
  y = p@V to bfloat16 and uses W = min(window, Lq) (dropkv_cache.py:401-460);
* pool = sliding max with -inf padding, then the last `window` keys get
  max+1 in float32 (dropkv_cache.py:464-467);
* kept indices: key i is kept iff #{j: s_j > s_i} + #{j < i: s_j == s_i} < keep
  (the "lowest index first among ties" rule), ascending (:470-475).

Inputs are drawn with NumPy's PCG64 generator from fixed seeds and rounded to
bfloat16 (so the same bytes feed the bf16 GPU kernels and the float32
oracle).  Stored: the Q tail (only the last W query rows are ever read), K, V
as bfloat16 bit patterns, and the float64 expectations.

Run: ``python tests/golden/make_golden.py`` (rewrites the .npz).
"""

from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "dropkv_golden.npz")
EPS = 1e-6

# name: (B, Hq, Hkv, D, Lq, Lk, W, kernel_size, keep_ratio, seed, sink)
CASES = {
    # BASELINE config 0 (CPU plumbing shape), bf16-representable values
    "c1": (1, 8, 2, 64, 512, 512, 8, 11, 0.1, 1234, False),
    # chunked prefill: the query is a tail-aligned suffix (Lq < Lk)
    "chunk": (1, 4, 2, 64, 24, 300, 8, 11, 0.1, 99, False),
    # Qwen2 head grouping: M = 7*8 = 56 rows (not a multiple of 16/32)
    "qwen_rows": (1, 14, 2, 64, 200, 200, 8, 11, 0.1, 7, False),
    # one key per head made dominant (attention sink, p up to ~0.7): large
    # weights concentrated on one key; p stays far enough from 1 that float32
    # and float64 agree (at p -> 1 the float32 reference itself loses digits)
    "sink": (1, 4, 1, 128, 160, 160, 8, 5, 0.2, 5, True),
    # final chunk shorter than the window: only the deployed path applies,
    # with W = min(window, Lq) = 5 (dropkv_cache.py:407)
    "short": (1, 8, 2, 64, 5, 96, 8, 11, 0.3, 21, False),
}


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (uint16)."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def from_bf16_bits(u: np.ndarray) -> np.ndarray:
    return (u.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return from_bf16_bits(to_bf16_bits(np.asarray(x, dtype=np.float32))).astype(np.float64)


def brute_scores(q, k, v, W, mode):
    """q [B,Hq,W,D] (the tail), k/v [B,Hkv,Lk,D]; float64.
    mode: 'exact' | 'bf16_p' | 'deployed' (p and y rounded to bf16)."""
    B, Hq, _, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    g = Hq // Hkv
    out = np.zeros((B, Hkv, Lk))
    for b in range(B):
        for h in range(Hkv):
            kh, vh = k[b, h], v[b, h]
            for gi in range(g):
                for w in range(W):
                    qv = q[b, h * g + gi, q.shape[2] - W + w]
                    bound = Lk - W + w
                    logit = kh[: bound + 1] @ qv / np.sqrt(D)
                    e = np.exp(logit - logit.max())
                    p = e / e.sum()
                    if mode in ("bf16_p", "deployed"):
                        p = round_bf16(p)
                    y = p @ vh[: bound + 1]
                    if mode == "deployed":
                        y = round_bf16(y)
                    wt = (p / (1.0 - p + EPS)) ** 2
                    dist2 = ((vh[: bound + 1] - y[None, :]) ** 2).sum(axis=1)
                    out[b, h, : bound + 1] += wt * dist2
            out[b, h] /= g
    return out


def pool_protect(scores, ks, window):
    """float32 arithmetic, like the reference's fp32 tensors."""
    s = scores.astype(np.float32)
    B, H, L = s.shape
    h = ks // 2
    pad = np.full((B, H, L + 2 * h), -np.inf, dtype=np.float32)
    pad[:, :, h:h + L] = s
    pooled = np.max(np.stack([pad[:, :, t:t + L] for t in range(ks)], axis=0), axis=0)
    big = pooled.max(axis=-1, keepdims=True) + np.float32(1.0)
    pooled[:, :, L - window:] = np.broadcast_to(big, pooled[:, :, L - window:].shape)
    return pooled


def keep_by_rank(pooled, keep):
    B, H, L = pooled.shape
    out = np.zeros((B, H, keep), dtype=np.int64)
    for b in range(B):
        for h in range(H):
            x = pooled[b, h]
            kept = []
            for i in range(L):
                rank = np.count_nonzero(x > x[i]) + np.count_nonzero(x[:i] == x[i])
                if rank < keep:
                    kept.append(i)
            assert len(kept) == keep
            out[b, h] = kept
    return out


def make_case(B, Hq, Hkv, D, Lq, Lk, W, ks, ratio, seed, sink):
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.standard_normal((B, Hq, Lq, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Lk, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, Lk, D)).astype(np.float32)
    if sink:
        # key 3 of every head aligned with the mean window query of its group
        g = Hq // Hkv
        for b in range(B):
            for h in range(Hkv):
                mq = q[b, h * g:(h + 1) * g, Lq - W:].reshape(-1, D).mean(axis=0)
                k[b, h, 3] = 3.0 * mq / np.linalg.norm(mq) * np.sqrt(D) / 2.0
    Wq = min(W, Lq)
    qb, kb, vb = to_bf16_bits(q[:, :, Lq - Wq:]), to_bf16_bits(k), to_bf16_bits(v)
    qf, kf, vf = (from_bf16_bits(x).astype(np.float64) for x in (qb, kb, vb))
    keep = min(Lk, max(int(ratio * Lk), W, 1))
    out = dict(q_tail=qb, k=kb, v=vb, meta=np.array([B, Hq, Hkv, D, Lq, Lk, W, ks, keep], dtype=np.int64),
               ratio=np.array(ratio))
    out["deployed"] = brute_scores(qf, kf, vf, Wq, "deployed")
    out["pooled_deployed"] = pool_protect(out["deployed"], ks, W)
    out["keep_idx_deployed"] = keep_by_rank(out["pooled_deployed"], keep)
    if Lq >= W:
        out["exact"] = brute_scores(qf, kf, vf, W, "exact")
        out["bf16p"] = brute_scores(qf, kf, vf, W, "bf16_p")
        out["pooled_bf16p"] = pool_protect(out["bf16p"], ks, W)
        out["keep_idx_bf16p"] = keep_by_rank(out["pooled_bf16p"], keep)
    return out


def main():
    arrays = {}
    for name, args in CASES.items():
        for key, val in make_case(*args).items():
            arrays[f"{name}/{key}"] = val
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
