// Device-side pieces of the DropKV scoring kernels (dkv_score.hip): tile
// geometry, the online-softmax step, operand loads, the candidate order, one
// row of the cross-split merge and the pooling-tail parameters.
#pragma once

#include "dkv_common.h"
#include "dkv_select_dev.h"

#include <climits>
#include <type_traits>

namespace dkv {

constexpr int kTile = 32;           // keys per wave tile
constexpr int kRows = 32;           // query rows per row-chunk (2 MFMA row blocks)
constexpr int kMB = kRows / 16;
// The fp32 attention output y enters pass 2's G^T = V Y^T as two bf16/fp16
// MFMA operands y = hi + lo (lo the rounded remainder), ~16 significant bits:
// <v,y> then carries a relative error of ~2^-17 |v||y|, below 1e-4 of
// dist2 = |v|^2 - 2<v,y> + |y|^2 wherever no key takes half of the row's
// attention.  Where one does (p_k >= 1/2, at most one key per row), dist2 at
// that key cancels heavily (y -> v_k), so the merge computes that one pair's
// distance directly, |v_k - y|^2 from the fp32 y, and pass 2 uses it there.
constexpr int kYParts = 2;
constexpr int kOpSlots = 1 + kYParts;  // Q and the parts of Y, per row block and k-step
constexpr int kStatWords = 64;         // per 16-row block: lse, |y|^2, sink key, -dist2/2 at it
// Candidate keys per (row, split) for merge's rounding correction of y: the
// keys holding the largest logits among those of individual lanes.
constexpr int kCand = 4;


__device__ __forceinline__ int row_bound(int m, int M, int W, int Lk) {
  return m < M ? Lk - W + (m % W) : -1;
}

// Online-softmax step (base 2) of one 32-key tile starting at key t0, for
// the lane's kMB row blocks: applies the causal bound to the raw logits s in
// place (kMasked: tiles that reach it, or padding rows), updates the running
// maximum m2 and sum lsum (log2 units: logits times scale_log2), rescales
// the y accumulators when a maximum moved, keeps the largest logit among the
// lane's own keys and the lowest key holding it (lmax, larg: the candidates
// of merge's correction of y), and returns the tile's P as two parts in the
// element type, hi and the rounded remainder lo (~16 significant bits
// together).
template <typename T, int D, bool kMasked>
__device__ __forceinline__ void softmax_tile(f32x4 (&s)[2][kMB], float (&m2)[kMB], float (&lsum)[kMB],
                                             float (&lmax)[kMB], int (&larg)[kMB], f32x4 (&yacc)[D / 16][kMB],
                                             typename Elem<T>::v8 (&phi)[kMB], typename Elem<T>::v8 (&plo)[kMB],
                                             const int (&bound)[kMB], int t0, int lg, float scale_log2) {
  constexpr int DT = D / 16;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    // The largest raw logit of the lane (IEEE maximum: no canonicalising
    // copies of the MFMA results); scaled once below.  Scaling by a
    // positive factor keeps the order, so the scaled maximum is the maximum
    // of the scaled logits.
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = s[kb][mb][r];
        if (kMasked) x = (t0 + 16 * kb + 4 * lg + r) <= bound[mb] ? x : -INFINITY;
        s[kb][mb][r] = x;
        tmax = __builtin_elementwise_maximum(tmax, x);
      }
    {
      // The lane's own maximum so far and the lowest of its keys holding it
      // (key t0 + 16 kb + 4 lg + r; scanned downwards so the lowest wins).
      int off = 0;
#pragma unroll
      for (int kb = 1; kb >= 0; --kb)
#pragma unroll
        for (int r = 3; r >= 0; --r) off = s[kb][mb][r] == tmax ? 16 * kb + r : off;
      tmax *= scale_log2;
      const bool up = tmax > lmax[mb];
      lmax[mb] = up ? tmax : lmax[mb];
      larg[mb] = up ? t0 + 4 * lg + off : larg[mb];
    }
    tmax = max_xor32(max_xor16(tmax));
    const float mnew = fmaxf(m2[mb], tmax);
    const bool empty = mnew == -INFINITY;
    const float alpha = empty ? 1.f : __builtin_amdgcn_exp2f(m2[mb] - mnew);
    // An empty row (every logit -inf so far) subtracts 0, so that its p are
    // exp2(-inf) = 0 without a select per element.  p = 2^(s scale - max)
    // with one rounding of the exponent.
    const float msub = empty ? 0.f : mnew;
    float psum = 0.f, pv[8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pv[4 * kb + r] = __builtin_amdgcn_exp2f(fmaf(s[kb][mb][r], scale_log2, -msub));
        psum += pv[4 * kb + r];
      }
    // P in the element type, two values per packed conversion.
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef T t2 __attribute__((ext_vector_type(2)));
    t2 h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = __builtin_convertvector((f2{pv[2 * e], pv[2 * e + 1]}), t2);
    phi[mb] = __builtin_bit_cast(typename Elem<T>::v8,
                                 __builtin_shufflevector(__builtin_shufflevector(h[0], h[1], 0, 1, 2, 3),
                                                         __builtin_shufflevector(h[2], h[3], 0, 1, 2, 3), 0, 1, 2,
                                                         3, 4, 5, 6, 7));
    {
      t2 l[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        l[e] = __builtin_convertvector((f2{pv[2 * e] - static_cast<float>(h[e][0]),
                                           pv[2 * e + 1] - static_cast<float>(h[e][1])}), t2);
      plo[mb] = __builtin_bit_cast(typename Elem<T>::v8,
                                   __builtin_shufflevector(__builtin_shufflevector(l[0], l[1], 0, 1, 2, 3),
                                                           __builtin_shufflevector(l[2], l[3], 0, 1, 2, 3), 0, 1,
                                                           2, 3, 4, 5, 6, 7));
    }
    lsum[mb] = lsum[mb] * alpha + psum;
    m2[mb] = mnew;
    // Rescale only when some row's maximum moved (rare after a few tiles).
    if (wave_any(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) yacc[dt][mb] *= alpha;
    }
  }
}

// One lane's Q^T operand: 8 consecutive head-dim values from column d0 of
// query row m (zeros for padding rows).  With `qvec` (head-dim stride 1 and
// 16-byte aligned rows, checked by the host) one 16-byte load; otherwise
// eight element loads, so Q may have any strides.
template <typename T>
__device__ __forceinline__ typename Elem<T>::v8 load_q_op(const T* __restrict__ q, int64_t q_sb, int64_t q_sh,
                                                        int64_t q_ss, int64_t q_sd, bool qvec, int b, int hkv,
                                                        int g, int W, int Lq, int M, int m, int d0) {
  typedef typename Elem<T>::v8 v8;
  const bool valid = m < M;
  const int mm = valid ? m : 0;  // padding rows read row 0, then zero it
  const int gi = mm / W, w = mm % W;
  const T* base = q + (int64_t)b * q_sb + (int64_t)(hkv * g + gi) * q_sh + (int64_t)(Lq - W + w) * q_ss;
  v8 x;
  if (qvec) {
    x = *reinterpret_cast<const v8*>(base + d0);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = base[(int64_t)(d0 + e) * q_sd];
  }
  if (!valid) x = v8{};
  return x;
}

// Load the Q^T operands of one 16-row block (lane row m, lane group lg).
template <typename T, int D>
__device__ __forceinline__ void load_q_ops(typename Elem<T>::v8 (&qop)[D / 32], const T* __restrict__ q,
                                           int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, bool qvec,
                                           int b, int hkv, int g, int W, int Lq, int M, int m, int lg) {
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk)
    qop[kk] = load_q_op<T>(q, q_sb, q_sh, q_ss, q_sd, qvec, b, hkv, g, W, Lq, M, m, 32 * kk + 8 * lg);
}

// Next tile for this wave from the workgroup's LDS counter: waves that get
// their data sooner take more of the workgroup's tiles, so the waves of a
// workgroup finish together.  Wave-uniform result.
__device__ __forceinline__ int grab_tile(uint32_t* ctr) {
  uint32_t v = 0u;
  if ((threadIdx.x & 63) == 0) v = atomicAdd(ctr, 1u);
  return __builtin_amdgcn_readfirstlane(v);
}

// Candidate order: the larger logit first, the lower key among equal logits;
// no candidate (key < 0) last.
__device__ __forceinline__ bool cand_before(float va, int ka, float vb, int kb) {
  return ka >= 0 && (kb < 0 || va > vb || (va == vb && ka < kb));
}

// Sorts the four (logit, key) candidates of a row held by the lanes of its
// four lane groups (lg = lane / 16) into candidate order along lg (a bitonic
// network over lane swaps).
__device__ __forceinline__ void sort_lane_groups(float& v, int& k, int lg) {
  const int lane = lg << 4;  // (only bits 4 and 5 are read)
  auto step = [&](int mask, bool keep_first) {
    const float ov = __uint_as_float(mask == 16 ? from_xor16(__float_as_uint(v), lane)
                                                : from_xor32(__float_as_uint(v), lane));
    const int ok = (int)(mask == 16 ? from_xor16((uint32_t)k, lane) : from_xor32((uint32_t)k, lane));
    const bool mine_first = cand_before(v, k, ov, ok);
    if (mine_first != keep_first) {
      v = ov;
      k = ok;
    }
  };
  step(16, ((lg & 1) == 0) == ((lg & 2) == 0));  // pairs: (0,1) descending, (2,3) ascending
  step(32, (lg & 2) == 0);
  step(16, (lg & 1) == 0);
}

// Merges the WAVES waves' candidate lists of one row (4 per wave, each in
// candidate order, at sm_cs / sm_ck[(w * kRows + row) * 4 ..]) into the
// row's kCand first: each step takes the best head and advances that list.
// All lists are read up front (one 16-byte LDS read each), so the merge
// itself waits on no LDS round trip.
template <int WAVES>
__device__ __forceinline__ void merge_wave_cands(const float* sm_cs, const int* sm_ck, int row,
                                                 float (&cs)[kCand], int (&ck)[kCand]) {
  static_assert(kCand <= 4, "at most one list's length");
  f32x4 lv[WAVES];
  i32x4 lk[WAVES];
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    lv[w] = *reinterpret_cast<const f32x4*>(sm_cs + (w * kRows + row) * 4);
    lk[w] = *reinterpret_cast<const i32x4*>(sm_ck + (w * kRows + row) * 4);
  }
  float hv[WAVES];
  int hk[WAVES], hp[WAVES];
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    hp[w] = 0;
    hv[w] = lv[w][0];
    hk[w] = lk[w][0];
  }
#pragma unroll
  for (int j = 0; j < kCand; ++j) {
    int bw = 0;
#pragma unroll
    for (int w = 1; w < WAVES; ++w) bw = cand_before(hv[w], hk[w], hv[bw], hk[bw]) ? w : bw;
    float bv = hv[0];
    int bk = hk[0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      bv = bw == w ? hv[w] : bv;
      bk = bw == w ? hk[w] : bk;
    }
    cs[j] = bv;
    ck[j] = bk;
    if (j + 1 < kCand) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        if (bw == w) {
          ++hp[w];
          // (hp <= j + 1 <= 3 here: the list has an entry at hp.)
          hv[w] = hp[w] == 1 ? lv[w][1] : hp[w] == 2 ? lv[w][2] : lv[w][3];
          hk[w] = hp[w] == 1 ? lk[w][1] : hp[w] == 2 ? lk[w][2] : lk[w][3];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Tile loads shared by the two passes.  A workgroup reads the rows
// [k_begin, k_end) of one head through buffer views (make_rsrc) that end at
// k_end, so rows past the range (a wave's tiles after its last one, the tail
// past Lk) read as zeros without memory traffic; the callers mask those keys.
// Offsets are bytes relative to row k_begin; per-lane parts are computed once
// and the tile offset is one add.
// ---------------------------------------------------------------------------
// 32 key rows as an MFMA A operand: lane (li, lg) holds row t+16kb+li,
// head-dim columns 32kk+8lg .. +7.  `lane_off` = (li*D + 8*lg) * sizeof(T).
template <typename T, int D>
__device__ __forceinline__ void load_rows_op(typename Elem<T>::v8 (&op)[2][D / 32], rsrc_t rs, uint32_t lane_off,
                                             int t) {
  typedef typename Elem<T>::v8 v8;
  const uint32_t base = lane_off + (uint32_t)t * (D * sizeof(T));
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk)
      op[kb][kk] = bitcast_u4<v8>(buf_load16(rs, base + (16 * kb * D + 32 * kk) * sizeof(T)));
}

template <typename T>
__device__ __forceinline__ float sumsq8(typename Elem<T>::v8 x, float acc);
template <>
__device__ __forceinline__ float sumsq8<__bf16>(Elem<__bf16>::v8 x, float acc) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const bf2 t = {x[e], x[e + 1]};
    acc = __builtin_amdgcn_fdot2_f32_bf16(t, t, acc, false);
  }
  return acc;
}
template <>
__device__ __forceinline__ float sumsq8<_Float16>(Elem<_Float16>::v8 x, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const h2 t = {x[e], x[e + 1]};
    acc = __builtin_amdgcn_fdot2(t, t, acc, false);
  }
  return acc;
}

// One row of the cross-split merge (merge_kernel; one wave, lane = threadIdx.x % 64).
constexpr int kMergeRows = 1;  // waves (rows) per workgroup
constexpr int kMaxSplits = 1024;
// Candidates whose final p is at least this get their rounding error
// (round(p) - p) v added to y; below it, that error is under 2^-20 |v|.
constexpr float kCorrMinP = 1.0f / 4096.0f;
constexpr float kCorrMinLog2P = -12.0f;  // log2(kCorrMinP)
constexpr int kCorrKeys = 8;  // candidates corrected per row (the largest p)

template <typename T, int D>
__device__ __forceinline__ void merge_row(int rid, const float* __restrict__ part_ml, const float* __restrict__ part_y,
                                          const int2* __restrict__ part_cand, int n_mc, int n_splits, int M,
                                          int n_rows, int p_round, int y_round, const T* __restrict__ q,
                                          int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd,
                                          const T* __restrict__ vp, int kv_ld, int Lk, int Hkv, int g, int W, int Lq,
                                          u32x4* __restrict__ opblk, float* __restrict__ stblk,
                                          float* __restrict__ ystat, float* __restrict__ yf32) {
  constexpr int DPL = D >= 64 ? D / 64 : 1;  // columns per lane (D = 32: lanes 32..63 hold none)
  constexpr int KK = D / 32;
  constexpr int OPS = kOpSlots * kMB * KK;
  constexpr int kPre = 64 / DPL;  // splits whose partial y is loaded up front (64 registers)
  const int lane = threadIdx.x & 63;

  const int mpad = n_mc * kRows;
  if (rid >= n_rows) return;
  const int head = rid / mpad;
  const int gr = rid % mpad;
  const int mc = gr / kRows, row = gr % kRows;
  const int64_t slot0 = ((int64_t)head * n_mc + mc) * n_splits;
  const int d0 = lane * DPL;
  const bool col = d0 < D;  // this lane holds head-dim columns

  // Every load up front: the partial y columns of the first kPre splits, the
  // query row, the per-split statistics and the candidates.  They go through
  // buffer views of this row-chunk's partials, where loads past the last
  // split return zeros without a memory request: every load is
  // unconditional, so all are in flight before the first wait.
  typedef float fv __attribute__((ext_vector_type(DPL)));
  static_assert(DPL == 1 || DPL == 2, "columns per lane");
  const uint32_t nsr = (uint32_t)n_splits * kRows;  // (split, row) slots of the row-chunk
  const rsrc_t ry = make_rsrc(part_y + slot0 * kRows * D, nsr * D * 4);
  const rsrc_t rml = make_rsrc(part_ml + slot0 * kRows * 2, nsr * 8);
  const rsrc_t rcd = make_rsrc(part_cand + slot0 * kRows * kCand, nsr * kCand * 8);
  // First the statistics and the candidates (needed first: a wait for a
  // load also waits for every load issued before it), then the y columns.
  const f32x2 ml_raw = buf_load8f(rml, ((uint32_t)lane * kRows + row) * 8);
  auto cand_at = [&](int c) __attribute__((always_inline)) {
    const uint32_t idx = (((uint32_t)(c / kCand)) * kRows + row) * kCand + c % kCand;
    return buf_load8i(rcd, idx * 8);
  };
  constexpr int kCandPre = 4;  // candidates per lane loaded up front
  i32x2 kcp[kCandPre];
#pragma unroll
  for (int j = 0; j < kCandPre; ++j) kcp[j] = cand_at(lane + 64 * j);
  auto load_y = [&](int s) __attribute__((always_inline)) {
    const uint32_t off = col ? (((uint32_t)s * kRows + row) * D + d0) * 4 : nsr * D * 4;
    if constexpr (DPL == 1)
      return __builtin_bit_cast(fv, buf_load4(ry, off));
    else
      return __builtin_bit_cast(fv, buf_load8f(ry, off));
  };
  fv yv[kPre];
#pragma unroll
  for (int s = 0; s < kPre; ++s) yv[s] = load_y(s);
  T qv[DPL];
  {
    const bool valid = gr < M;
    const int b = head / Hkv, hkv = head % Hkv, gi = valid ? gr / W : 0, w = valid ? gr % W : 0;
    const T* qrow = q + (int64_t)b * q_sb + (int64_t)(hkv * g + gi) * q_sh + (int64_t)(Lq - W + w) * q_ss;
#pragma unroll
    for (int e = 0; e < DPL; ++e) qv[e] = qrow[(int64_t)(col ? d0 + e : 0) * q_sd];  // padding rows: zeroed at the store
  }
  // The row's (key, logit) candidates, kCand per split, loaded with the
  // partials: lane l reads candidates l, l + 64, ... and keeps its two
  // largest (lowest key first among equal logits).  Once the lse is known,
  // the wave takes the largest in turn (ranking by logit ranks by p) while
  // their p can matter, and loads their value rows together.
  const int ncand = n_splits * kCand;
  // Split statistics: lane s holds (m, l) of split s (the first 64 in
  // registers, any further ones re-read in the rare loops below).
  const float2 ml = lane < n_splits ? make_float2(ml_raw[0], ml_raw[1]) : make_float2(-INFINITY, 0.f);
  float mx = ml.x;
  for (int s = 64 + lane; s < n_splits; s += 64) mx = fmaxf(mx, part_ml[((slot0 + s) * kRows + row) * 2]);
  mx = wave_max_dpp(mx);
  const bool valid = gr < M && mx != -INFINITY;

  auto weight = [&](float m) { return (m == -INFINITY || mx == -INFINITY) ? 0.f : exp2f(m - mx); };
  const float f_lane = weight(ml.x);
  float lpart = ml.y * f_lane;
  for (int s = 64 + lane; s < n_splits; s += 64)
    lpart += part_ml[((slot0 + s) * kRows + row) * 2 + 1] * weight(part_ml[((slot0 + s) * kRows + row) * 2]);
  const float l = wave_sum_dpp(lpart);
  const float lse2 = mx + log2f(fmaxf(l, 1e-40f));

  // y from the probabilities rounded to the input dtype (the reference's
  // semantics with p rounding, dropkv_triton.py:88-93).  Pass 1 summed the
  // unrounded p (the rounded p needs the final lse).  Of the candidates (the
  // keys holding the largest logits of individual lanes of pass 1), the
  // kCorrKeys largest that take at least kCorrMinP of the row's attention
  // get (round(p) - p) v added here.  Each key's rounding error is at most
  // 2^-8 of its p, so these are the errors that can move a distance: a row
  // whose few largest keys went uncorrected would leave relative errors of
  // 1e-3 in other keys' scores.  The largest candidate is the row's top key
  // (the lowest key among those holding the maximum); when it takes at least
  // half of the attention its distance is also computed directly below.
  int ck[kCorrKeys];
  float cs[kCorrKeys];
  fv vb[kCorrKeys];
  {
    float sa = -INFINITY, sb = -INFINITY;
    int ka = -1, kb = -1;
    // Branch-free insertion into the lane's two best (selects only, so the
    // four values stay in registers).
    auto offer = [&](i32x2 kc) __attribute__((always_inline)) {
      const float sc = __int_as_float(kc.y);
      const int kx = (kc.x >= 0 && kc.x < Lk) ? kc.x : -1;
      const bool ga = cand_before(sc, kx, sa, ka);
      const bool gb = !ga && cand_before(sc, kx, sb, kb);
      const float nsb = ga ? sa : (gb ? sc : sb);
      const int nkb = ga ? ka : (gb ? kx : kb);
      sa = ga ? sc : sa;
      ka = ga ? kx : ka;
      sb = nsb;
      kb = nkb;
    };
#pragma unroll
    for (int j = 0; j < kCandPre; ++j) offer(lane + 64 * j < ncand ? kcp[j] : i32x2{-1, 0});
    for (int c = lane + 64 * kCandPre; c < ncand; c += 64) offer(cand_at(c));
    // Only candidates that can matter take part: p >= kCorrMinP with p
    // rounding, otherwise only a key with p >= 1/2 (its direct distance).
    const float s_min = !valid ? INFINITY : p_round ? lse2 + kCorrMinLog2P : lse2 - 1.0f;
    bool more = true;
#pragma unroll
    for (int u = 0; u < kCorrKeys; ++u) {
      ck[u] = -1;
      cs[u] = -INFINITY;
      if (!more) continue;
      const float best = wave_max_dpp(ka >= 0 ? sa : -INFINITY);
      more = best >= s_min && (p_round || u == 0);
      if (!more) continue;
      const uint64_t tie = __ballot(ka >= 0 && sa == best);
      int kmin = INT_MAX;
      if (tie) {
        kmin = __builtin_amdgcn_readlane(ka, __builtin_ctzll(tie));
        if (tie & (tie - 1)) kmin = wave_min_dpp((ka >= 0 && sa == best) ? ka : INT_MAX);  // equal logits
      }
      ck[u] = kmin == INT_MAX ? -1 : kmin;
      cs[u] = best;
      if (ka == kmin && kmin != INT_MAX) {
        sa = sb;
        ka = kb;
        sb = -INFINITY;
        kb = -1;
      }
    }
    // Their value rows, all loads unconditional (a row of no candidate reads
    // past the view: zeros, no memory request).
    const rsrc_t rv = make_rsrc(vp + (int64_t)head * kv_ld * D, (uint32_t)Lk * D * sizeof(T));
#pragma unroll
    for (int u = 0; u < kCorrKeys; ++u) {
      const uint32_t off =
          ck[u] >= 0 && col ? ((uint32_t)ck[u] * D + d0) * sizeof(T) : (uint32_t)Lk * D * sizeof(T);
      if constexpr (DPL == 1) {
        vb[u][0] = static_cast<float>(__builtin_bit_cast(T, buf_load2(rv, off)));
      } else {
        typedef T t2v __attribute__((ext_vector_type(2)));
        const t2v x = __builtin_bit_cast(t2v, buf_load4(rv, off));
        vb[u][0] = static_cast<float>(x[0]);
        vb[u][1] = static_cast<float>(x[1]);
      }
    }
  }
  int k_top = -1;
  fv vk = {}, corr = {};
  if (valid) {
    if (p_round) {
#pragma unroll
      for (int u = 0; u < kCorrKeys; ++u) {
        const float pc = ck[u] >= 0 ? fminf(__builtin_amdgcn_exp2f(cs[u] - lse2), 1.f) : 0.f;
        if (pc >= kCorrMinP) corr += (round_through<T>(pc) - pc) * vb[u];
      }
    }
    const float pk = fminf(__builtin_amdgcn_exp2f(mx - lse2), 1.f);
    if (pk >= 0.5f && ck[0] >= 0 && cs[0] == mx) {
      k_top = ck[0];
      vk = vb[0];
    }
  }

  // acc = sum_s f_s * y_s; lane s holds f_s of the first 64 splits.
  fv acc = {};
#pragma unroll
  for (int s = 0; s < kPre; ++s)
    if (s < n_splits) acc += read_lane_f(f_lane, s) * yv[s];
  // Further splits in batches of 8 whose loads are all issued before use.
  for (int s0 = kPre; s0 < n_splits; s0 += 8) {
    fv yb[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) yb[u] = load_y(s0 + u);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int s = s0 + u;
      if (s < n_splits) {
        const float fs = s < 64 ? read_lane_f(f_lane, s) : weight(part_ml[((slot0 + s) * kRows + row) * 2]);
        acc += fs * yb[u];
      }
    }
  }

  float ysq = 0.f, dsq = 0.f;
  const int64_t rbase = (int64_t)head * mpad + gr;
  T* ob = reinterpret_cast<T*>(opblk + ((int64_t)head * n_mc + mc) * OPS * 64);
  const int mb = row / 16, li = row % 16;
  float ye[DPL];
  T qe[DPL], he[DPL], le[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    float y = valid ? acc[e] / l + corr[e] : 0.f;
    const T hi = static_cast<T>(y);
    if (y_round) y = static_cast<float>(hi);
    const T lo = static_cast<T>(y - static_cast<float>(hi));
    if (col) {
      ysq += y * y;
      const float dv = vk[e] - y;
      dsq += dv * dv;
    }
    ye[e] = y;
    qe[e] = gr < M ? qv[e] : static_cast<T>(0.f);
    he[e] = hi;
    le[e] = lo;
  }
  // Operand block of this head: per row-chunk, the Q, Y-hi and Y-lo MFMA
  // operands in per-lane order (slot (which, mb, kk), lane li + 16*lg,
  // element e8), so that pass 2 stages them with one contiguous copy.
  auto op_at = [&](int which, int d) __attribute__((always_inline)) {
    const int kk = d / 32, lg = (d % 32) / 8, e8 = d % 8;
    return ob + ((size_t)((which * kMB + mb) * KK + kk) * 64 + li + 16 * lg) * 8 + e8;
  };
  if (col) {
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      yf32[rbase * D + d0 + e] = ye[e];
      *op_at(0, d0 + e) = qe[e];
      *op_at(1, d0 + e) = he[e];
      *op_at(2, d0 + e) = le[e];
    }
  }
  const float yn2 = wave_sum_dpp(ysq);
  const float nd2_top = -0.5f * wave_sum_dpp(dsq);
  if (lane == 0) {
    const float lse_row = valid ? lse2 : INFINITY;
    float* sb = stblk + (((int64_t)head * n_mc + mc) * kMB + row / 16) * kStatWords + (row % 16);
    ystat[rbase * 2 + 0] = lse_row;
    ystat[rbase * 2 + 1] = yn2;
    sb[0] = lse_row;
    sb[16] = yn2;
    sb[32] = __builtin_bit_cast(float, k_top);
    sb[48] = nd2_top;
  }
}

// The weight w = (p/(1-p+eps))^2 of pass 2 (dropkv_triton.py:589-591), in
// the reference's order of operations.
__device__ __forceinline__ float exact_weight(float p, float eps) {
  const float ratio = p * __builtin_amdgcn_rcpf(1.0f - p + eps);
  return ratio * ratio;
}

// Its small-p form.  With c = 1/(1+eps), w = c^2 p^2 / (1-cp)^2.  Where the
// caller has shown p <= 2^kSmallLog2P for every p of the wave's tile and the
// host has checked 0 <= eps <= kSmallMaxEps, (p + p^2)^2 = p^2 (1+p)^2
// stands for p^2 / (1-cp)^2: their ratio is ((1+p)(1-cp))^2 =
// (1 + p(1-c) - cp^2)^2 with 0 <= p(1-c) <= p eps <= 2^-25 and
// cp^2 <= 2^-26, so within 2^-24 of 1 (under one fp32 ulp).  The caller
// multiplies the tile's sums by c^2 (small_c2, computed on the host).  Two
// operations, where the exact form takes four and a quarter-rate
// reciprocal.
constexpr float kSmallLog2P = -13.0f;
constexpr float kSmallMaxEps = 0x1p-12f;
__device__ __forceinline__ float small_weight_over_c2(float p) {
  const float q = fmaf(p, p, p);
  return q * q;
}

// The largest of a lane's values of a 32-key tile, x[kb][mb][r] over every
// key block, row block and element; NaN if any is NaN.  (IEEE maximum: gfx950
// has a three-operand form of it, where fmaxf first canonicalises each
// operand with a copy.)
__device__ __forceinline__ float fmax_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float tile_max(const f32x4 (&x)[2][kMB]) {
  float t[2 * kMB];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
      t[kb * kMB + mb] = fmax_nan(fmax_nan(x[kb][mb][0], x[kb][mb][1]), fmax_nan(x[kb][mb][2], x[kb][mb][3]));
#pragma unroll
  for (int n = 2 * kMB; n > 1; n >>= 1)
#pragma unroll
    for (int i = 0; i < n / 2; ++i) t[i] = fmax_nan(t[i], t[i + n / 2]);
  return t[0];
}

// ---------------------------------------------------------------------------
// Pooling epilogue of pass 2 (a layer-call's score -> select).  Every pass-2
// workgroup owns the key range [k_begin, k_end) of one row and, once its
// scores are stored, pools the keys whose whole window lies in that range
// (its interior) into the pooled row, the row maximum and the top-digit
// histogram (pool_range).  The selection's resolve stage pools the keys next to
// the split boundaries.  The kernel boundary is the only synchronisation: an
// in-kernel handoff between workgroups would need agent-scope
// release/acquire, which on gfx950 writes back and invalidates an XCD's whole
// L2 per workgroup and costs far more than a launch.
// ---------------------------------------------------------------------------
struct SelFuse {
  SelWs ws;    // selection workspace; its per-row words were zeroed by merge
  int enabled;
  int ks, window;
  int sc_lds;  // the workgroup's scores are also kept in LDS (kps <= kScLds)
  // The whole selection in the tail (dkv_tail_dev.h) instead of pooling only.
  int full;
  int keep;
  int spin;    // polls at the tail's barrier A before a workgroup gives up
  int spin_b;  // polls at barrier B before a workgroup finishes the row alone
  int64_t* out_idx;
  CompactArgs ca;
};
constexpr int kScLds = 4096;  // longest split range whose scores pass 2 keeps in LDS

}  // namespace dkv
