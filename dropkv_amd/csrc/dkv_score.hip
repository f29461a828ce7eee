// DropKV scoring on gfx950: split-K flash partials, cross-split merge and the
// per-key residual-output perturbation score.
//
// Math (one KV head; g = Hq/Hkv query heads, W window rows each, M = g*W):
//   row m = gi*W + w is query head hkv*g+gi at position Lq-W+w, aligned to key
//   position Lk-W+w (dropkv_triton.py:225-231);  l[m,j] = q_m.k_j/sqrt(D) for
//   j <= Lk-W+w;  p = softmax_j(l);  y_m = sum_j p[m,j] v_j;
//   w = (p/(1-p+eps))^2;  score_j = (1/g) sum_m w[m,j] * max(|v_j|^2 - 2<y_m,v_j> + |y_m|^2, 0)
//   (dropkv_triton.py:29-109 and :574-606).
//
// Matrix-core mapping (v_mfma_f32_16x16x32_{bf16,f16}, wave64):
//   operand A[i][k] lives in lane i + 16*g, element e, where (g, e) names the
//   contraction slot; operand B[k][j] likewise in lane j + 16*g; the result
//   C[i][j] lives in lane j + 16*(i/4), element i%4.  Any bijection between
//   contraction slots and the real contraction index works as long as A and B
//   use the same one, which the kernels exploit to keep P in registers.
//   * logits are computed transposed, S^T = K Q^T: a lane then holds one query
//     row m = lane%16 for keys 4*(lane/16)+r, so row max / row sum are mostly
//     lane-local;
//   * Y^T = V^T P^T: B = P^T comes straight from the S^T registers; A = V^T
//     comes from a per-wave LDS tile written transposed (V rows are contiguous
//     along D in HBM, but the contraction here runs along keys).
#include "dkv_common.h"
#include "dkv_internal.h"
#include "dkv_score_dev.h"
#include "dkv_select_dev.h"
#include "dkv_tail_dev.h"

#include <algorithm>
#include <climits>
#include <atomic>
#include <mutex>
#include <type_traits>

namespace dkv {

// Makes a kernel argument live in scalar registers at this point, so that the
// compiler issues every argument load of the prologue at once instead of one
// dependent round trip per branch that first needs an argument.
#define DKV_ARG_NOW(x) __asm__ volatile("" ::"s"(x))

// ---------------------------------------------------------------------------
// Pass 1: split-K flash partials.  Workgroup = (head, row-chunk, key split);
// each of its WAVES waves streams its own 32-key tiles, issuing the loads of
// its next tile as soon as the current tile's K/V registers are consumed, so
// they overlap the softmax and P.V work.  The waves are merged in LDS at the
// end.  Output per (head, chunk, split, row): running max (log2 domain),
// running sum, and the unnormalised fp32 y row.
// ---------------------------------------------------------------------------
template <typename T, int D, int WAVES, int MINW>
__global__ void __launch_bounds__(64 * WAVES, MINW)
pass1_kernel(const T* __restrict__ q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, bool qvec,
             const T* __restrict__ kp, const T* __restrict__ vp, int kv_ld,
             int Hkv, int Lq, int Lk, int W, int g, int M, int n_mc, int n_splits, int kps,
             float scale_log2, float* __restrict__ part_ml, float* __restrict__ part_y,
             int2* __restrict__ part_cand) {
  typedef typename Elem<T>::v8 v8;
  constexpr int KK = D / 32;
  constexpr int DT = D / 16;
  constexpr int CPR = D / 8;           // 16-byte chunks per key row
  constexpr int GRP = 64 / CPR;        // key rows covered per load round
  constexpr int NVC = kTile / GRP;     // V chunks per lane and tile
  constexpr int NT = 64 * WAVES;
  // A wave's V tile in LDS: its rows as loaded, padded so that the
  // transposing reads (16 lanes: 4 rows x 32 bytes) hit no bank twice.
  constexpr int kVPitch = D + 16;
  constexpr int kVTileWords = kTile * kVPitch / 2;

  constexpr int kYPitch = D + 4;  // fp32 row pitch of the merge buffer
  constexpr int kLdsTiles = WAVES * kVTileWords;
  constexpr int kLdsMerge = 3 * WAVES * kRows + 8 * WAVES * kRows + WAVES * kRows * kYPitch;
  __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsTiles > kLdsMerge ? kLdsTiles : kLdsMerge];

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int mc = lid % n_mc;
  const int split = (lid / n_mc) % n_splits;
  const int head = lid / (n_mc * n_splits);
  const int b = head / Hkv, hkv = head % Hkv;

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;

  v8 qop[kMB][KK];
  int bound[kMB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const int m = mc * kRows + mb * 16 + li;
    load_q_ops<T, D>(qop[mb], q, q_sb, q_sh, q_ss, q_sd, qvec, b, hkv, g, W, Lq, M, m, lg);
    bound[mb] = row_bound(m, M, W, Lk);
  }
  // Tiles wholly below every row's causal bound need no masking (unless this
  // chunk holds padding rows).
  const bool pad_chunk = mc * kRows + kRows > M;
  const int unmasked_end = Lk - W + 1;

  const int k_begin = split * kps;
  const int k_end = min(k_begin + kps, Lk);
  const int64_t roff = ((int64_t)head * kv_ld + k_begin) * D;
  const uint32_t range = (uint32_t)(k_end - k_begin) * (D * sizeof(T));
  const rsrc_t krs = make_rsrc(kp + roff, range), vrs = make_rsrc(vp + roff, range);
  const uint32_t k_lane = (li * D + 8 * lg) * sizeof(T);
  // V chunk i of a lane: row lane / CPR + i * GRP of the tile, columns
  // 8 (lane % CPR) .. +7.
  const uint32_t v_lane = ((lane / CPR) * D + 8 * (lane % CPR)) * sizeof(T);
  const int v_row = lane / CPR, v_col = 8 * (lane % CPR);
  uint32_t* vt = lds + wv * kVTileWords;
  auto load_v = [&](u32x4 (&vc)[NVC], int t) __attribute__((always_inline)) {
    const uint32_t base = v_lane + (uint32_t)t * (D * sizeof(T));
#pragma unroll
    for (int i = 0; i < NVC; ++i) vc[i] = buf_load16(vrs, base + (uint32_t)(i * GRP * D * sizeof(T)));
  };

  float m2[kMB], lsum[kMB];
  // Per lane: the largest logit among its own keys and the lowest key
  // holding it (-1: none yet).
  float lmax[kMB];
  int larg[kMB];
  f32x4 yacc[DT][kMB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    m2[mb] = -INFINITY;
    lsum[mb] = 0.f;
    lmax[mb] = -INFINITY;
    larg[mb] = -1;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) yacc[dt][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  v8 kop[2][KK];
  u32x4 vch[NVC];
  const int stride = WAVES * kTile;

  // One tile (t0 absolute, tn relative to k_begin): consume the K/V
  // registers, refill them with tile tn (zeros past the range), then the
  // softmax and P.V work, which overlaps both tiles' loads.
  auto tile = [&](v8 (&kop)[2][KK], u32x4 (&vch)[NVC], int t0, int tn)
      __attribute__((always_inline)) {
    // S^T = K Q^T.
    f32x4 s[2][kMB];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) acc = Elem<T>::mfma(kop[kb][kk], qop[mb][kk], acc);
        s[kb][mb] = acc;
      }
    // The K registers are free again: start the K loads of tile tn (zeros
    // past the range; unconditional, so that the compiler's wait counts stay
    // exact) before waiting for this tile's V.
    load_rows_op<T, D>(kop, krs, k_lane, tn);

    // The V rows -> LDS, as loaded.
#pragma unroll
    for (int i = 0; i < NVC; ++i)
      *reinterpret_cast<u32x4*>(vt + ((v_row + i * GRP) * kVPitch + v_col) / 2) = vch[i];

    // The V registers are free again: start the V loads of tile tn.
    load_v(vch, tn);

    // Online softmax.  P enters the MFMA as hi + lo: the p of a tile is
    // relative to the running maximum, so rounding it to the input dtype
    // here would not be the reference's rounding of the final p (merge
    // applies that one to the keys where it matters).
    v8 phi[kMB], plo[kMB];
    if (pad_chunk || t0 + kTile > unmasked_end)
      softmax_tile<T, D, true>(s, m2, lsum, lmax, larg, yacc, phi, plo, bound, t0, lg, scale_log2);
    else
      softmax_tile<T, D, false>(s, m2, lsum, lmax, larg, yacc, phi, plo, bound, t0, lg, scale_log2);

    // Y^T += V^T P^T, V^T read transposed from the V rows in LDS: lane
    // (li, lg) needs V[key][16dt + li] for keys 4lg + e and 16 + 4lg + e
    // (e = 0..3, the keys of its P^T operand).  A transposing read gives
    // output lane i of each 16-lane group element e of input lane 4e + i/4's
    // 8 bytes, element i % 4; so input lane li reads key base + li/4,
    // columns 16dt + 4(li % 4) .. +3.
    const int tr_row = 4 * lg + li / 4, tr_col = 4 * (li % 4);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      typedef short s4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) s4 lds_s4;
      const T* vrow = reinterpret_cast<const T*>(vt);
      const s4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(vrow + tr_row * kVPitch + 16 * dt + tr_col));
      const s4 x1 =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(vrow + (16 + tr_row) * kVPitch + 16 * dt + tr_col));
      const v8 aop = __builtin_bit_cast(v8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        yacc[dt][mb] = Elem<T>::mfma(aop, phi[mb], yacc[dt][mb]);
        yacc[dt][mb] = Elem<T>::mfma(aop, plo[mb], yacc[dt][mb]);
      }
    }
  };

  // Static tile order (wave w takes tiles w, w+WAVES, ...): the summation
  // order, and so every bit of the result, is the same on every call.
  const int nrel = k_end - k_begin;
  int t = wv * kTile;  // relative to k_begin
  load_rows_op<T, D>(kop, krs, k_lane, t);  // zeros if t >= nrel
  load_v(vch, t);
  for (; t < nrel; t += stride) tile(kop, vch, k_begin + t, t + stride);

  // Row sums are per lane-group partials; fold the four groups.  The lanes'
  // candidates of a row go into candidate order along the lane groups (lane
  // swaps, no LDS: done before the barrier).
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    lsum[mb] = add_xor32(add_xor16(lsum[mb]));
    sort_lane_groups(lmax[mb], larg[mb], lg);
  }

  // Cross-wave merge in LDS (the V tiles are dead now): every wave stores
  // its unscaled accumulator once; then all threads combine the waves with
  // weights 2^(m_w - max_w m_w) and write the workgroup's partial.  The
  // lanes' (logit, key) candidates of a row (4 per wave) are reduced to the
  // kCand largest (the lowest key first among equal logits).
  __syncthreads();
  float* sm_m = reinterpret_cast<float*>(lds);
  float* sm_l = sm_m + WAVES * kRows;
  float* sm_f = sm_l + WAVES * kRows;
  float* sm_cs = sm_f + WAVES * kRows;                       // [WAVES][kRows][4]
  int* sm_ck = reinterpret_cast<int*>(sm_cs + 4 * WAVES * kRows);
  float* wbuf = sm_cs + 8 * WAVES * kRows;                   // [WAVES][kRows][kYPitch]
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const int ci = (wv * kRows + 16 * mb + li) * 4 + lg;
    sm_cs[ci] = lmax[mb];
    sm_ck[ci] = larg[mb];
    if (lg == 0) {
      sm_m[wv * kRows + 16 * mb + li] = m2[mb];
      sm_l[wv * kRows + 16 * mb + li] = lsum[mb];
    }
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
      *reinterpret_cast<f32x4*>(wbuf + ((size_t)wv * kRows + 16 * mb + li) * kYPitch + 16 * dt + 4 * lg) =
          yacc[dt][mb];
  __syncthreads();
  // The partials go out with write-through stores (st_dev): none of them is
  // left dirty in the L2 for the write-back at the end of the kernel, which
  // the merge kernel's start waits for.
  const int64_t slot = ((int64_t)head * n_mc + mc) * n_splits + split;
  if (threadIdx.x < kRows) {
    const int row = threadIdx.x;
    float mx = -INFINITY;
    for (int w = 0; w < WAVES; ++w) mx = fmaxf(mx, sm_m[w * kRows + row]);
    float l = 0.f;
    for (int w = 0; w < WAVES; ++w) {
      const float mw = sm_m[w * kRows + row];
      const float f = (mw == -INFINITY) ? 0.f : exp2f(mw - mx);
      sm_f[w * kRows + row] = f;
      l += sm_l[w * kRows + row] * f;
    }
    st_dev(&part_ml[(slot * kRows + row) * 2 + 0], mx);
    st_dev(&part_ml[(slot * kRows + row) * 2 + 1], l);
    float cs[kCand];
    int ck[kCand];
    merge_wave_cands<WAVES>(sm_cs, sm_ck, row, cs, ck);
#pragma unroll
    for (int j = 0; j < kCand; ++j)
      st_dev(reinterpret_cast<uint64_t*>(&part_cand[(slot * kRows + row) * kCand + j]),
             ((uint64_t)(uint32_t)__float_as_int(cs[j]) << 32) | (uint32_t)ck[j]);
  }
  __syncthreads();
  // y of the workgroup, 16 bytes a thread and step, every LDS read of a
  // thread issued before its first sum.
  constexpr int NV = kRows * D / 4;
  const rsrc_t yrs = make_rsrc(part_y + slot * kRows * D, (uint32_t)(kRows * D * sizeof(float)));
#pragma unroll
  for (int j = 0; j < (NV + NT - 1) / NT; ++j) {
    const int i = (int)threadIdx.x + j * NT;
    if (NV % NT == 0 || i < NV) {
      const int row = i / (D / 4), c4 = i % (D / 4);
      f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const f32x4 wb = *reinterpret_cast<const f32x4*>(wbuf + ((size_t)w * kRows + row) * kYPitch + 4 * c4);
        const float f = sm_f[w * kRows + row];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = fmaf(wb[e], f, y[e]);
      }
      st_dev16(yrs, (uint32_t)i * 16u, y);
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 1 for several row-chunks (n_mc >= 2: large GQA groups or windows).
// Workgroup = (head, key split) with 8 waves; wave w owns row-chunk w (waves
// past n_mc only load).  Each 32-key K/V tile is loaded once per workgroup,
// cooperatively, into LDS (K rows padded, V transposed), and every wave
// applies it to its own rows.  With one workgroup per row-chunk instead,
// every tile would be streamed n_mc times.  Tiles move in groups of kWideG:
// the loads of the next group are in flight (in registers) while the waves
// work on the current one, double-buffered in LDS with one barrier per group,
// so that ~64 KB per CU are on their way at any time (one tile in flight
// does not cover the memory latency).
// Writes the same per-(head, chunk, split, row) partials as pass1_kernel.
// ---------------------------------------------------------------------------
constexpr int kWideWaves = 8;

template <typename T, int D, int kWideG>
__global__ void __launch_bounds__(64 * kWideWaves, 1)
pass1w_kernel(const T* __restrict__ q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, bool qvec,
              const T* __restrict__ kp, const T* __restrict__ vp, int kv_ld,
              int Hkv, int Lq, int Lk, int W, int g, int M, int n_mc, int n_splits, int kps,
              float scale_log2, float* __restrict__ part_ml, float* __restrict__ part_y,
              int2* __restrict__ part_cand) {
  typedef typename Elem<T>::v8 v8;
  constexpr int KK = D / 32;
  constexpr int DT = D / 16;
  constexpr int NT = 64 * kWideWaves;
  constexpr int CPR = D / 8;                 // 16-byte chunks per key row
  constexpr int KCH = kTile * CPR;           // K (and V) chunks per tile
  static_assert(KCH <= NT, "one K chunk and one V chunk per thread");
  constexpr int kKPitch = D + 8;             // elements per padded K row in LDS
  constexpr int kKWords = kTile * kKPitch / 2;
  // V rows as loaded, padded so that the transposing reads below (16 lanes:
  // 4 rows x 32 bytes) cover the banks without conflicts.
  constexpr int kVPitch = D + 16;
  constexpr int kVWords = kTile * kVPitch / 2;
  constexpr int kTileWords = kKWords + kVWords;
  constexpr int kStage = kWideG * kTileWords;  // dwords per buffer stage
  __shared__ __attribute__((aligned(16))) uint32_t lds[2 * kStage];

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int split = lid % n_splits;
  const int head = lid / n_splits;
  const int b = head / Hkv, hkv = head % Hkv;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int mc = wv;
  const bool active = mc < n_mc;

  v8 qop[kMB][KK];
  int bound[kMB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const int m = mc * kRows + mb * 16 + li;
    load_q_ops<T, D>(qop[mb], q, q_sb, q_sh, q_ss, q_sd, qvec, b, hkv, g, W, Lq, M, m, lg);
    bound[mb] = row_bound(m, M, W, Lk);
  }
  const bool pad_chunk = mc * kRows + kRows > M;
  const int unmasked_end = Lk - W + 1;

  const int k_begin = split * kps;
  const int k_end = min(k_begin + kps, Lk);
  const int64_t roff = ((int64_t)head * kv_ld + k_begin) * D;
  const uint32_t range = (uint32_t)(k_end - k_begin) * (D * sizeof(T));
  const rsrc_t krs = make_rsrc(kp + roff, range), vrs = make_rsrc(vp + roff, range);
  // This thread's share of a tile: chunk tid of K and of V (row tid / CPR,
  // chunk tid % CPR).
  const int kr = tid / CPR, kc = tid % CPR;
  const uint32_t k_off = (uint32_t)(kr * D + 8 * kc) * sizeof(T);
  u32x4 kreg[kWideG], vreg[kWideG];
  // Loads of tile group grp (rows past the range read as zeros).
  auto issue = [&](int grp) __attribute__((always_inline)) {
#pragma unroll
    for (int gt = 0; gt < kWideG; ++gt) {
      const uint32_t base = (uint32_t)((grp * kWideG + gt) * kTile) * (D * sizeof(T));
      if (tid < KCH) {
        kreg[gt] = buf_load16(krs, base + k_off);
        vreg[gt] = buf_load16(vrs, base + k_off);
      }
    }
  };
  auto stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int gt = 0; gt < kWideG; ++gt) {
      uint32_t* kl = lds + buf * kStage + gt * kTileWords;
      uint32_t* vt = kl + kKWords;
      if (tid < KCH) {
        *reinterpret_cast<u32x4*>(kl + (kr * kKPitch + 8 * kc) / 2) = kreg[gt];
        *reinterpret_cast<u32x4*>(vt + (kr * kVPitch + 8 * kc) / 2) = vreg[gt];
      }
    }
  };

  float m2[kMB], lsum[kMB], lmax[kMB];
  int larg[kMB];
  f32x4 yacc[DT][kMB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    m2[mb] = -INFINITY;
    lsum[mb] = 0.f;
    lmax[mb] = -INFINITY;
    larg[mb] = -1;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) yacc[dt][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int nrel = k_end - k_begin;
  const int ntiles = (nrel + kTile - 1) / kTile;
  const int ngroups = (ntiles + kWideG - 1) / kWideG;
  // One group of tiles from LDS stage `st` (a compile-time constant in
  // both calls below, so that the LDS addresses fold into instruction
  // offsets).
  auto group = [&](int grp, auto st_c) __attribute__((always_inline)) {
    constexpr int st = decltype(st_c)::value;
    if (grp + 1 < ngroups) issue(grp + 1);
    for (int gt = 0; gt < kWideG && active; ++gt) {
      const int it = grp * kWideG + gt;
      if (it >= ntiles) break;
      const int t0 = k_begin + it * kTile;
      const uint32_t* kl = lds + st * kStage + gt * kTileWords;
      const uint32_t* vt = kl + kKWords;
      // S^T = K Q^T with K from LDS.
      f32x4 s[2][kMB];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        v8 kop[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          kop[kk] = bitcast_u4<v8>(
              *reinterpret_cast<const u32x4*>(kl + ((16 * kb + li) * kKPitch + 32 * kk + 8 * lg) / 2));
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) acc = Elem<T>::mfma(kop[kk], qop[mb][kk], acc);
          s[kb][mb] = acc;
        }
      }
      v8 phi[kMB], plo[kMB];
      if (pad_chunk || t0 + kTile > unmasked_end)
        softmax_tile<T, D, true>(s, m2, lsum, lmax, larg, yacc, phi, plo, bound, t0, lg, scale_log2);
      else
        softmax_tile<T, D, false>(s, m2, lsum, lmax, larg, yacc, phi, plo, bound, t0, lg, scale_log2);
      // Y^T += V^T P^T with V^T read transposed from the V rows in LDS: lane
      // (li, lg) needs V[key][16dt + li] for keys 4lg + e and 16 + 4lg + e
      // (e = 0..3, the keys of its P^T operand).  A transposing read gives
      // output lane i of each 16-lane group element e of input lane 4e + i/4's
      // 8 bytes, element i % 4; so input lane li reads key base + li/4,
      // columns 16dt + 4(li % 4) .. +3.
      const int tr_row = 4 * lg + li / 4, tr_col = 4 * (li % 4);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        typedef short s4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s4 lds_s4;
        const T* vrow = reinterpret_cast<const T*>(vt);
        const s4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s4*)(vrow + tr_row * kVPitch + 16 * dt + tr_col));
        const s4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s4*)(vrow + (16 + tr_row) * kVPitch + 16 * dt + tr_col));
        const v8 aop = __builtin_bit_cast(v8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
          yacc[dt][mb] = Elem<T>::mfma(aop, phi[mb], yacc[dt][mb]);
          yacc[dt][mb] = Elem<T>::mfma(aop, plo[mb], yacc[dt][mb]);
        }
      }
    }
    if (grp + 1 < ngroups) stage(1 - st);
    __syncthreads();
  };
  issue(0);
  stage(0);
  __syncthreads();
  for (int grp = 0; grp < ngroups; grp += 2) {
    group(grp, std::integral_constant<int, 0>{});
    if (grp + 1 < ngroups) group(grp + 1, std::integral_constant<int, 1>{});
  }
  if (!active) return;

  // This wave's rows are complete for the split: write the partials, and
  // each lane its (logit, key) candidate of the row (kCand = 4 lanes a row).
  static_assert(kCand == 4, "one candidate per lane group");
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    lsum[mb] = add_xor32(add_xor16(lsum[mb]));
  }
  const int64_t slot = ((int64_t)head * n_mc + mc) * n_splits + split;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const int row = 16 * mb + li;
    part_cand[(slot * kRows + row) * kCand + lg] = make_int2(larg[mb], __float_as_int(lmax[mb]));
    if (lg == 0) {
      part_ml[(slot * kRows + row) * 2 + 0] = m2[mb];
      part_ml[(slot * kRows + row) * 2 + 1] = lsum[mb];
    }
    float* py = part_y + (slot * kRows + row) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(py + 16 * dt + 4 * lg) = yacc[dt][mb];
  }
}

// ---------------------------------------------------------------------------
// Merge: one wave per (head, padded row), kMergeRows rows per workgroup; no
// workgroup barrier.  Lane l owns head-dim columns l*DPL .. +DPL-1 and split
// l's statistics; the split weights f_s = 2^(m_s - max_s m_s) are broadcast
// with lane shuffles and the weighted partial y rows summed with every load
// in flight.  Writes, for the score pass, the row's Q / Y-hi / Y-lo operands
// into the head's operand block (in the order pass 2's lanes read them from
// LDS) and its statistics (lse in log2 units, |y|^2, the key holding at least
// half of the row's attention if any, and -dist2/2 at that key), plus an fp32
// copy of y for inspection.  Optionally clears `zero_words` words at `zero_ptr` (the
// selection workspace of a fused layer-call), so that needs no launch of its
// own.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ void __launch_bounds__(64 * kMergeRows)
merge_kernel(const float* __restrict__ part_ml, const float* __restrict__ part_y, const int2* __restrict__ part_cand,
             int n_mc, int n_splits, int M, int n_rows, int p_round, int y_round, const T* __restrict__ q,
             int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, const T* __restrict__ vp, int kv_ld, int Lk,
             int Hkv, int g, int W, int Lq, u32x4* __restrict__ opblk, float* __restrict__ stblk,
             float* __restrict__ ystat, float* __restrict__ yf32, uint32_t* __restrict__ zero_ptr,
             int64_t zero_words) {
  DKV_ARG_NOW(gridDim.x);
  DKV_ARG_NOW(part_ml);
  DKV_ARG_NOW(part_y);
  DKV_ARG_NOW(part_cand);
  DKV_ARG_NOW(n_splits);
  DKV_ARG_NOW(n_mc);
  DKV_ARG_NOW(n_rows);
  DKV_ARG_NOW(q);
  DKV_ARG_NOW(q_sb);
  DKV_ARG_NOW(q_sh);
  DKV_ARG_NOW(q_ss);
  DKV_ARG_NOW(M);
  // (head, padded row); a head's rows on the XCD whose pass-1 workgroups
  // wrote its partials (pass 1 maps heads to XCDs the same way).
  const int rid =
      __builtin_amdgcn_readfirstlane(xcd_remap(blockIdx.x, gridDim.x) * kMergeRows + (threadIdx.x >> 6));
  merge_row<T, D>(rid, part_ml, part_y, part_cand, n_mc, n_splits, M, n_rows, p_round, y_round, q, q_sb, q_sh,
                  q_ss, q_sd, vp, kv_ld, Lk, Hkv, g, W, Lq, opblk, stblk, ystat, yf32);
  // Last, so that the argument loads it needs do not delay the row's first loads.
  if (zero_ptr)
    for (int64_t i = (int64_t)blockIdx.x * (64 * kMergeRows) + threadIdx.x; i < zero_words;
         i += (int64_t)gridDim.x * (64 * kMergeRows))
      zero_ptr[i] = 0u;
}

// ---------------------------------------------------------------------------
// Pass 2: per-key score.  Workgroup = (head, key split); each of its WAVES
// waves streams 32-key tiles, recomputes S^T = K Q^T and G^T = V Y^T (Y as
// hi+lo) and folds w * dist2 over all query rows.  The next tile's loads are
// issued right after the last MFMA of the current tile, overlapping the
// per-element work.  The Q^T / Y^T operands of up to `cg` row-chunks are
// staged in LDS in per-lane order (one conflict-free 16-byte read per
// operand); more row-chunks are processed in groups, the partial per-key sums
// being carried in the output array.
// ---------------------------------------------------------------------------

template <typename T, int D, int WAVES, int MINW, bool PR>
__global__ void __launch_bounds__(64 * WAVES, MINW)
pass2_kernel(const T* __restrict__ kp, const T* __restrict__ vp, int kv_ld,
             int Hkv, int Lq, int Lk, int W, int g, int M, int n_mc, int cg, int n_splits, int kps,
             float scale_log2, float eps, float small_c2,
             const u32x4* __restrict__ opblk, const float* __restrict__ stblk, float* __restrict__ scores,
             SelFuse fz) {
  typedef typename Elem<T>::v8 v8;
  constexpr int KK = D / 32;
  constexpr int OPS = kOpSlots * kMB * KK;  // operand slots per row-chunk (Q, Yhi, Ylo)
  constexpr int NT = 64 * WAVES;
  extern __shared__ u32x4 opnd[];    // [cg][OPS][64] then float stats [cg][kMB][kStatWords]
  float* stat = reinterpret_cast<float*>(opnd + (size_t)cg * OPS * 64);
  float* sc_row = stat + cg * kMB * kStatWords;  // [kps] this workgroup's scores (fused pooling only)
  // Top-digit histogram of the fused pooling (after sc_row), zeroed now.
  uint32_t* hist_l = reinterpret_cast<uint32_t*>(sc_row + kps);

  DKV_ARG_NOW(gridDim.x);
  DKV_ARG_NOW(kp);
  DKV_ARG_NOW(vp);
  DKV_ARG_NOW(opblk);
  DKV_ARG_NOW(stblk);
  DKV_ARG_NOW(n_splits);
  DKV_ARG_NOW(kps);
  DKV_ARG_NOW(kv_ld);
  DKV_ARG_NOW(Lk);
  DKV_ARG_NOW(n_mc);
  DKV_ARG_NOW(cg);
  DKV_ARG_NOW(g);
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int split = lid % n_splits;
  const int head = lid / n_splits;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;

  // The per-key sums hold sum_m w * (-dist2/2): scale by -2/g at the end.
  const float out_scale = -2.0f * (1.0f / static_cast<float>(g));
  const int k_begin = split * kps;
  const int k_end = min(k_begin + kps, Lk);
  const int64_t roff = ((int64_t)head * kv_ld + k_begin) * D;
  const uint32_t range = (uint32_t)(k_end - k_begin) * (D * sizeof(T));
  const rsrc_t krs = make_rsrc(kp + roff, range), vrs = make_rsrc(vp + roff, range);
  const uint32_t k_lane = (li * D + 8 * lg) * sizeof(T);
  const int ntiles = (k_end - k_begin + kTile - 1) / kTile;
  __shared__ uint32_t s_next;
  const int unmasked_end = Lk - W + 1;

  v8 kop[2][KK], vop[2][KK];
  for (int c0 = 0; c0 < n_mc; c0 += cg) {
    const int cn = min(cg, n_mc - c0);
    const bool first = c0 == 0, last = c0 + cn >= n_mc;
    // Operands of row-chunks c0 .. c0+cn-1 (written by the merge kernel in
    // LDS order): issue their loads, then the first tile's K/V loads, so both
    // round trips overlap; the LDS writes wait only for the former.  Every
    // wave issues its operand loads before any wave issues K/V loads (the
    // barrier between them): otherwise the later waves' operand loads queue
    // behind the earlier waves' 16 KB of K/V each, and the operand block
    // reaches LDS ~2 us later.
    constexpr int SPW = (2 * OPS * 64 + NT - 1) / NT;
    const int nw = cn * OPS * 64, ns = cn * kMB * kStatWords;
    static_assert(4 * kMB * kStatWords <= NT, "one statistics word per thread");
    const u32x4* gop = opblk + ((size_t)head * n_mc + c0) * OPS * 64;
    const float* gst = stblk + ((size_t)head * n_mc + c0) * kMB * kStatWords;
    u32x4 sv[SPW];
#pragma unroll
    for (int i = 0; i < SPW; ++i) sv[i] = gop[min((int)threadIdx.x + i * NT, nw - 1)];
    const float stv = gst[min((int)threadIdx.x, ns - 1)];
    // Tiles are handed out dynamically: wave w starts with tile w, then
    // takes the next unclaimed one from s_next (relative to k_begin).  Each
    // key's score is computed by one wave in a fixed order, so the results do
    // not depend on the assignment.
    const int tw = wv;
    __syncthreads();  // the previous group's LDS operands and s_next are dead
    load_rows_op<T, D>(kop, krs, k_lane, tw * kTile);
    load_rows_op<T, D>(vop, vrs, k_lane, tw * kTile);
    if (threadIdx.x == 0) s_next = WAVES;
    // The pooling histogram, zeroed once the first loads are out.
    if (first && fz.enabled && fz.sc_lds)
      for (int i = threadIdx.x; i < kBins1; i += NT) hist_l[i] = 0u;
#pragma unroll
    for (int i = 0; i < SPW; ++i)
      if ((int)threadIdx.x + i * NT < nw) opnd[threadIdx.x + i * NT] = sv[i];
    // Groups of four row-chunks copy the second pair directly.
    for (int i = SPW * NT + (int)threadIdx.x; i < nw; i += NT) opnd[i] = gop[i];
    if ((int)threadIdx.x < ns) stat[threadIdx.x] = stv;
    __syncthreads();

    // The chunk count NC of the unrolled body is a compile-time constant so
    // that the refill loads stay unconditional; groups of four row-chunks run
    // that body for two pairs (`npairs`) on the same K/V registers.
    auto run = [&](auto nc_const, int npairs) __attribute__((always_inline)) {
    constexpr int NC = decltype(nc_const)::value;
    auto tile = [&](v8 (&kop)[2][KK], v8 (&vop)[2][KK], int t0, int tn) __attribute__((always_inline)) {
      // The MFMAs put rows on the result registers and keys on the lanes:
      // lane (lg, li) holds rows 16mb + 4lg + r (r = 0..3) of key t0 + 16kb +
      // li, so a key's sum over the rows is in-lane but for the four lane
      // groups.  |v|^2 of key t0+16kb+li: fp32 dot of the exact operand
      // values.
      float vn2[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float part = 0.f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) part = sumsq8<T>(vop[kb][kk], part);
        vn2[kb] = add_xor32(add_xor16(part));
      }
      // (Padding rows need no mask: merge gives them lse = +inf and zero Q,
      // so their p is 0.)
      const bool masked = t0 + kTile > unmasked_end;

      float sc[2] = {0.f, 0.f};

#pragma unroll 1
      for (int cp = 0; cp < npairs; ++cp)
#pragma unroll
      for (int c1 = 0; c1 < NC; ++c1) {
        const int c = cp * NC + c1;
        f32x4 sacc[2][kMB], gacc[2][kMB];
        const u32x4* ob = opnd + (size_t)(c * OPS) * 64 + lane;
        const float* cst = stat + (size_t)c * kMB * kStatWords;
        // G starts at -(|v|^2 + |y|^2)/2, so that after the MFMAs it holds
        // <v,y> - (|v|^2 + |y|^2)/2 = -dist2/2 of every (key, row) pair.
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
          const f32x4 y4 = *reinterpret_cast<const f32x4*>(cst + mb * kStatWords + 16 + 4 * lg);
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            sacc[kb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < 4; ++r) gacc[kb][mb][r] = fmaf(vn2[kb], -0.5f, -0.5f * y4[r]);
          }
        }
        // S first: after the last row-chunk's S MFMAs the K registers are
        // free, and the K loads of tile tn (relative; zeros past the range)
        // start while G is computed; then the same for V.
        const bool refill = c1 == NC - 1 && cp == npairs - 1;
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) {
            const v8 qo = __builtin_bit_cast(v8, ob[(size_t)((0 * kMB + mb) * KK + kk) * 64]);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) sacc[kb][mb] = Elem<T>::mfma(qo, kop[kb][kk], sacc[kb][mb]);
          }
        if (refill) load_rows_op<T, D>(kop, krs, k_lane, tn);
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) {
            const v8 yh = __builtin_bit_cast(v8, ob[(size_t)((1 * kMB + mb) * KK + kk) * 64]);
            const v8 yl = __builtin_bit_cast(v8, ob[(size_t)((2 * kMB + mb) * KK + kk) * 64]);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
              gacc[kb][mb] = Elem<T>::mfma(yh, vop[kb][kk], gacc[kb][mb]);
              gacc[kb][mb] = Elem<T>::mfma(yl, vop[kb][kk], gacc[kb][mb]);
            }
          }
        if (refill) load_rows_op<T, D>(vop, vrs, k_lane, tn);
        // sc accumulates w * (-dist2/2).  The causal bound, and the direct
        // distance at a row's dominant key (merge), are applied only in
        // tiles that reach the bound or hold such a key (and with padding
        // rows), so that the other tiles carry no per-element selects.
        bool sink_here = false;
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb)
          sink_here |= (uint32_t)(__builtin_bit_cast(int, cst[mb * kStatWords + 32 + li]) - t0) < (uint32_t)kTile;
        // log2 p of every element, in place of its logit.
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(cst + mb * kStatWords + 4 * lg);
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) sacc[kb][mb][r] = sacc[kb][mb][r] * scale_log2 - l4[r];
        }
        auto epilogue = [&](auto masked_c, auto small_c, float (&acc)[2]) __attribute__((always_inline)) {
          constexpr bool kMasked = decltype(masked_c)::value;
          constexpr bool kSmall = decltype(small_c)::value;
#pragma unroll
          for (int mb = 0; mb < kMB; ++mb) {
            int bound[4] = {0, 0, 0, 0}, sk[4] = {-1, -1, -1, -1};
            float sn[4] = {0.f, 0.f, 0.f, 0.f};
            if (kMasked) {
              const u32x4 k4 = *reinterpret_cast<const u32x4*>(cst + mb * kStatWords + 32 + 4 * lg);
              const f32x4 n4 = *reinterpret_cast<const f32x4*>(cst + mb * kStatWords + 48 + 4 * lg);
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                bound[r] = row_bound((c0 + c) * kRows + mb * 16 + 4 * lg + r, M, W, Lk);
                sk[r] = (int)k4[r];
                sn[r] = n4[r];
              }
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
              const int key = t0 + 16 * kb + li;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                float p = __builtin_amdgcn_exp2f(sacc[kb][mb][r]);
                if (kMasked) p = key <= bound[r] ? p : 0.f;
                if (!kSmall) p = min_one_nonneg(p);  // (small p: p <= 2^-13 already)
                if (PR) p = round_through<T>(p);
                float nd2 = min_zero(gacc[kb][mb][r]);  // -dist2/2, dist2 clamped at 0
                if (kMasked) nd2 = key == sk[r] ? sn[r] : nd2;
                acc[kb] = fmaf(kSmall ? small_weight_over_c2(p) : exact_weight(p, eps), nd2, acc[kb]);
              }
            }
          }
        };
        if (masked || wave_any(sink_here)) {
          epilogue(std::true_type{}, std::false_type{}, sc);
        } else if (small_c2 > 0.f && !wave_any(!(tile_max(sacc) <= kSmallLog2P))) {
          // This chunk's sums carry w / c^2: scaled back as they join sc.
          float st[2] = {0.f, 0.f};
          epilogue(std::false_type{}, std::true_type{}, st);
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) sc[kb] = fmaf(st[kb], small_c2, sc[kb]);
        } else {
          epilogue(std::false_type{}, std::false_type{}, sc);
        }
      }

      // The four lane groups lg hold the same keys for different rows: their
      // sum, stored by the lanes of group 0.
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float v = add_xor16(add_xor32(sc[kb]));
        const int n = t0 + 16 * kb + li;
        if (lg == 0 && n < k_end) {
          float* dst = scores + (int64_t)head * Lk + n;
          if (!first) v += *dst;
          *dst = last ? v * out_scale : v;
          if (last && fz.sc_lds) sc_row[n - k_begin] = v * out_scale;
        }
      }
    };

    for (int tc = tw; tc < ntiles;) {
      const int tn = grab_tile(&s_next);
      tile(kop, vop, k_begin + tc * kTile, tn * kTile);
      tc = tn;
    }
    };
    if (cn % 2 == 0)
      run(std::integral_constant<int, 2>{}, cn / 2);
    else
      run(std::integral_constant<int, 1>{}, 1);
  }
  if (fz.enabled) {
    __syncthreads();  // this workgroup's score stores are done; the LDS operands are dead
    if (fz.full) {
      fused_tail<NT>(fz, sc_row, hist_l, head, split, n_splits, kps, Lk);
      return;
    }
    const int h = fz.ks / 2;
    const int i0 = split == 0 ? 0 : k_begin + h;
    const int i1 = k_end >= Lk ? Lk : k_end - h;
    uint32_t* L = reinterpret_cast<uint32_t*>(opnd);  // below sc: the operand region is dead
    float* prow = fz.ws.pooled + (int64_t)head * Lk;
    uint32_t* rw = fz.ws.rowws + (int64_t)head * kRowWords;
    if (fz.sc_lds)
      pool_range_lds<NT>(sc_row, k_begin, prow, rw, Lk, h, Lk - fz.window, i0, i1, hist_l, hist_l + kBins1);
    else
      pool_range<NT>(scores + (int64_t)head * Lk, prow, rw, Lk, h, Lk - fz.window, i0, i1,
                     reinterpret_cast<float*>(L), L + kSub + 2 * kMaxHalo, L + kSub + 2 * kMaxHalo + kBins1);
  }
}

// ---------------------------------------------------------------------------
// Pass 2 for several row-chunks (3 <= n_mc <= 8: large GQA groups or
// windows), in one sweep over K/V.  Workgroup = (head, key split) with 8
// waves; wave w holds row-chunk w's Q / Y-hi / Y-lo operands and statistics
// in registers (waves past n_mc only stage).  Each 32-key tile of K and V is
// loaded once per workgroup into LDS (rows padded against bank conflicts,
// with |v|^2 of each row), kG tiles per stage, double-buffered: the loads of
// the next stage are in flight while the waves work on the current one.
// Each wave's per-key sums over its 32 rows go to LDS, and after the stage's
// one barrier the keys' totals are summed over the waves in wave order, so
// the result does not depend on timing.  With one workgroup per row-chunk
// group instead, K/V would be streamed once per group.
// ---------------------------------------------------------------------------
template <int CPR>
__device__ __forceinline__ float sum_over_row_lanes(float x) {
  x += dpp_f<kDppQuadSwap1>(x);
  x += dpp_f<kDppQuadSwap2>(x);
  if (CPR >= 8) x += dpp_f<kDppHalfMirror>(x);
  if (CPR >= 16) x += dpp_f<kDppMirror>(x);
  return x;
}

template <typename T, int D, int kG, bool PR>
__global__ void __launch_bounds__(64 * kWideWaves, 1)
pass2w_kernel(const T* __restrict__ kp, const T* __restrict__ vp, int kv_ld, int Hkv, int Lq, int Lk, int W, int g,
              int M, int n_mc, int n_splits, int kps, float scale_log2, float eps, float small_c2,
              const u32x4* __restrict__ opblk, const float* __restrict__ stblk, float* __restrict__ scores, SelFuse fz) {
  typedef typename Elem<T>::v8 v8;
  constexpr int KK = D / 32;
  constexpr int OPS = kOpSlots * kMB * KK;
  constexpr int NT = 64 * kWideWaves;
  constexpr int RB = D * (int)sizeof(T);
  constexpr int CPR = RB / 16;                // 16-byte chunks per row
  constexpr int KCH = kTile * CPR;            // chunks per tile and tensor
  static_assert(KCH <= NT && KCH % 64 == 0, "one K and one V chunk per thread, whole waves");
  static_assert(CPR == 4 || CPR == 8 || CPR == 16, "a row's chunks in one DPP row");
  constexpr int kRowPitch = D + 8;            // elements per padded row in LDS
  constexpr int kTensorWords = kTile * kRowPitch / 2;
  constexpr int kTileWords = 2 * kTensorWords + kTile;  // K rows, V rows, |v|^2
  constexpr int kStage = kG * kTileWords;
  __shared__ __attribute__((aligned(16))) uint32_t lds[2 * kStage > kPoolLdsWords ? 2 * kStage : kPoolLdsWords];
  __shared__ float red[2][kWideWaves][kG * kTile];  // per-wave key sums of a stage, double-buffered
  __shared__ __attribute__((aligned(16))) float sc_row[kScLds];
  __shared__ uint32_t hist_l[kBins1 + 16];

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int split = lid % n_splits;
  const int head = lid / n_splits;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int mc = wv;
  const bool active = mc < n_mc;
  const bool sc_lds = fz.enabled && fz.sc_lds;
  if (sc_lds)
    for (int i = tid; i < kBins1; i += NT) hist_l[i] = 0u;

  const float out_scale = -2.0f * (1.0f / static_cast<float>(g));
  const int k_begin = split * kps;
  const int k_end = min(k_begin + kps, Lk);
  const int64_t roff = ((int64_t)head * kv_ld + k_begin) * D;
  const uint32_t range = (uint32_t)(k_end - k_begin) * RB;
  const rsrc_t krs = make_rsrc(kp + roff, range), vrs = make_rsrc(vp + roff, range);
  const int nrel = k_end - k_begin;
  const int ntiles = (nrel + kTile - 1) / kTile;
  const int ngroups = (ntiles + kG - 1) / kG;

  // This wave's operands (merge wrote them in pass 2's LDS order) and row
  // statistics.  The MFMAs put rows on the result registers and keys on the
  // lanes: lane (lg, li) holds rows 16mb + 4lg + r (r = 0..3) of key 16kb + li,
  // so a key's sum over the wave's rows is mostly in-lane.  Per lane: lse
  // (log2 units) and -|y|^2/2 of its rows; the dominant key of row 16mb + li
  // and -dist2/2 there (read by the other lanes through shuffles where a
  // tile needs them).
  const int c = active ? mc : 0;
  v8 qo[kMB][KK], yh[kMB][KK], yl[kMB][KK];
  float lse2[kMB][4], nyh[kMB][4], snd2[kMB];
  int skey[kMB];
  {
    const u32x4* ob = opblk + ((size_t)head * n_mc + c) * OPS * 64 + lane;
    const float* st = stblk + ((size_t)head * n_mc + c) * kMB * kStatWords;
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        qo[mb][kk] = __builtin_bit_cast(v8, ob[(size_t)((0 * kMB + mb) * KK + kk) * 64]);
        yh[mb][kk] = __builtin_bit_cast(v8, ob[(size_t)((1 * kMB + mb) * KK + kk) * 64]);
        yl[mb][kk] = __builtin_bit_cast(v8, ob[(size_t)((2 * kMB + mb) * KK + kk) * 64]);
      }
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(st + mb * kStatWords + 4 * lg);
      const f32x4 y4 = *reinterpret_cast<const f32x4*>(st + mb * kStatWords + 16 + 4 * lg);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        lse2[mb][r] = l4[r];
        nyh[mb][r] = -0.5f * y4[r];
      }
      skey[mb] = __builtin_bit_cast(int, st[mb * kStatWords + 32 + li]);
      snd2[mb] = st[mb * kStatWords + 48 + li];
    }
  }
  const int unmasked_end = Lk - W + 1;

  // Staging: thread tid < KCH owns chunk tid % CPR of row tid / CPR of each
  // tile, of K and of V.
  const int sr = tid / CPR, scn = tid % CPR;
  const uint32_t s_off = (uint32_t)(sr * D + 8 * scn) * sizeof(T);
  u32x4 kreg[kG], vreg[kG];
  auto issue = [&](int grp) __attribute__((always_inline)) {
#pragma unroll
    for (int gt = 0; gt < kG; ++gt) {
      const uint32_t base = (uint32_t)((grp * kG + gt) * kTile) * RB;
      if (tid < KCH) {
        kreg[gt] = buf_load16(krs, base + s_off);
        vreg[gt] = buf_load16(vrs, base + s_off);
      }
    }
  };
  auto stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int gt = 0; gt < kG; ++gt) {
      uint32_t* kl = lds + buf * kStage + gt * kTileWords;
      uint32_t* vl = kl + kTensorWords;
      float* vn = reinterpret_cast<float*>(vl + kTensorWords);
      if (tid < KCH) {
        *reinterpret_cast<u32x4*>(kl + (sr * kRowPitch + 8 * scn) / 2) = kreg[gt];
        *reinterpret_cast<u32x4*>(vl + (sr * kRowPitch + 8 * scn) / 2) = vreg[gt];
        // |v|^2 of the row: fp32 sum of the exact element values.
        const float ss = sum_over_row_lanes<CPR>(sumsq8<T>(bitcast_u4<v8>(vreg[gt]), 0.f));
        if (scn == 0) vn[sr] = ss;
      }
    }
  };

  // One tile in two parts.  mma: S and G of this wave's rows for the tile
  // whose K/V rows are at kl (G starts at -(|v|^2 + |y|^2)/2, so that after
  // the MFMAs it holds <v,y> - (|v|^2 + |y|^2)/2 = -dist2/2); epi: the
  // per-element work on them and this wave's per-key sums over its rows into
  // red[buf][wv][gt * kTile ..].
  auto mma = [&](const uint32_t* kl, f32x4 (&sacc)[2][kMB], f32x4 (&gacc)[2][kMB]) __attribute__((always_inline)) {
    const uint32_t* vl = kl + kTensorWords;
    const float* vn = reinterpret_cast<const float*>(vl + kTensorWords);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const float vn2 = vn[16 * kb + li];
      v8 kop[KK], vop[KK];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int w = ((16 * kb + li) * kRowPitch + 32 * kk + 8 * lg) / 2;
        kop[kk] = bitcast_u4<v8>(*reinterpret_cast<const u32x4*>(kl + w));
        vop[kk] = bitcast_u4<v8>(*reinterpret_cast<const u32x4*>(vl + w));
      }
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        f32x4 sa = {0.f, 0.f, 0.f, 0.f};
        f32x4 ga;
#pragma unroll
        for (int r = 0; r < 4; ++r) ga[r] = fmaf(vn2, -0.5f, nyh[mb][r]);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) sa = Elem<T>::mfma(qo[mb][kk], kop[kk], sa);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          ga = Elem<T>::mfma(yh[mb][kk], vop[kk], ga);
          ga = Elem<T>::mfma(yl[mb][kk], vop[kk], ga);
        }
        sacc[kb][mb] = sa;
        gacc[kb][mb] = ga;
      }
    }
  };
  auto epi = [&](f32x4 (&sacc)[2][kMB], const f32x4 (&gacc)[2][kMB], int t0, int buf, int gt)
                 __attribute__((always_inline)) {
    float sc[2] = {0.f, 0.f};
    // log2 p of every element, in place of its logit.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) sacc[kb][mb][r] = sacc[kb][mb][r] * scale_log2 - lse2[mb][r];
    bool sink_here = false;
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) sink_here |= (uint32_t)(skey[mb] - t0) < (uint32_t)kTile;
    auto epilogue = [&](auto masked_c, auto small_c) __attribute__((always_inline)) {
      constexpr bool kMasked = decltype(masked_c)::value;
      constexpr bool kSmall = decltype(small_c)::value;
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        int bound[4] = {0, 0, 0, 0}, sk[4] = {-1, -1, -1, -1};
        float sn[4] = {0.f, 0.f, 0.f, 0.f};
        if (kMasked)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            bound[r] = row_bound(mc * kRows + mb * 16 + 4 * lg + r, M, W, Lk);
            sk[r] = __shfl(skey[mb], 4 * lg + r);
            sn[r] = __shfl(snd2[mb], 4 * lg + r);
          }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int key = t0 + 16 * kb + li;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float p = __builtin_amdgcn_exp2f(sacc[kb][mb][r]);
            if (kMasked) p = key <= bound[r] ? p : 0.f;
            if (!kSmall) p = min_one_nonneg(p);  // (small p: p <= 2^-13 already)
            if (PR) p = round_through<T>(p);
            float nd2 = min_zero(gacc[kb][mb][r]);  // -dist2/2, dist2 clamped at 0
            if (kMasked) nd2 = key == sk[r] ? sn[r] : nd2;
            sc[kb] = fmaf(kSmall ? small_weight_over_c2(p) : exact_weight(p, eps), nd2, sc[kb]);
          }
        }
      }
    };
    // The small-p tiles' sums carry w / c^2: scaled back below.
    float tile_scale = 1.0f;
    // (Padding rows need no mask: merge gives them lse = +inf and zero Q, so
    // their p is 0.)
    if (t0 + kTile > unmasked_end || wave_any(sink_here)) {
      epilogue(std::true_type{}, std::false_type{});
    } else if (small_c2 > 0.f && !wave_any(!(tile_max(sacc) <= kSmallLog2P))) {
      epilogue(std::false_type{}, std::true_type{});
      tile_scale = small_c2;
    } else {
      epilogue(std::false_type{}, std::false_type{});
    }
    // The four lane groups lg hold the same keys for different rows.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const float v = add_xor16(add_xor32(sc[kb]));
      if (lg == 0) red[buf][wv][gt * kTile + 16 * kb + li] = v * tile_scale;
    }
  };

  // The keys' totals of a stage over the active waves, in wave order, after
  // the barrier that follows the stage's red writes.
  auto finish = [&](int grp) __attribute__((always_inline)) {
    if (tid < kG * kTile) {
      const int buf = grp & 1;
      const int it = grp * kG + tid / kTile;
      float v = red[buf][0][tid];
      for (int w = 1; w < n_mc; ++w) v += red[buf][w][tid];
      const int n = k_begin + it * kTile + tid % kTile;
      if (it < ntiles && n < k_end) {
        scores[(int64_t)head * Lk + n] = v * out_scale;
        if (sc_lds) sc_row[n - k_begin] = v * out_scale;
      }
    }
  };

  auto group = [&](int grp, auto st_c) __attribute__((always_inline)) {
    constexpr int st = decltype(st_c)::value;
    if (grp + 1 < ngroups) issue(grp + 1);
    if (active) {
#pragma unroll
      for (int gt = 0; gt < kG; ++gt) {
        const int it = grp * kG + gt;
        if (it < ntiles) {
          f32x4 sacc[2][kMB], gacc[2][kMB];
          mma(lds + st * kStage + gt * kTileWords, sacc, gacc);
          epi(sacc, gacc, k_begin + it * kTile, grp & 1, gt);
        }
      }
    }
    if (grp + 1 < ngroups) stage(1 - st);
    __syncthreads();
    finish(grp);
  };
  issue(0);
  stage(0);
  __syncthreads();
  for (int grp = 0; grp < ngroups; grp += 2) {
    group(grp, std::integral_constant<int, 0>{});
    if (grp + 1 < ngroups) group(grp + 1, std::integral_constant<int, 1>{});
  }

  if (fz.enabled) {
    // The stage loop ended with a barrier, but the last stage's key totals
    // (finish) were stored after it.
    __syncthreads();
    const int h = fz.ks / 2;
    const int i0 = split == 0 ? 0 : k_begin + h;
    const int i1 = k_end >= Lk ? Lk : k_end - h;
    float* prow = fz.ws.pooled + (int64_t)head * Lk;
    uint32_t* rw = fz.ws.rowws + (int64_t)head * kRowWords;
    if (sc_lds)
      pool_range_lds<NT>(sc_row, k_begin, prow, rw, Lk, h, Lk - fz.window, i0, i1, hist_l, hist_l + kBins1);
    else
      pool_range<NT>(scores + (int64_t)head * Lk, prow, rw, Lk, h, Lk - fz.window, i0, i1,
                     reinterpret_cast<float*>(lds), lds + kSub + 2 * kMaxHalo, lds + kSub + 2 * kMaxHalo + kBins1);
  }
}

// ---------------------------------------------------------------------------
// Host-side launch helpers (called from dkv_capi.hip).
// ---------------------------------------------------------------------------


static inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Launch shapes (from sweeps on MI355X).  Fixed per build: the split
// geometry sets the floating-point summation order, so the same inputs give
// the same bits on every call.  The -D overrides exist for sweeps only.
#ifndef DKV_TARGET_WG
#define DKV_TARGET_WG 256      // workgroups per pass: one per CU
#endif
#ifndef DKV_TARGET_P1_BW
#define DKV_TARGET_P1_BW 160   // pass-1 workgroups of a bandwidth-bound call
#endif
#ifndef DKV_P1_WAVES
#define DKV_P1_WAVES 4         // waves per pass-1 workgroup (4 or 8)
#endif
#ifndef DKV_P1_WIDE_MIN
#define DKV_P1_WIDE_MIN 3      // row-chunks from which pass 1 shares tiles across chunks (0: never)
#endif
#ifndef DKV_P1_WIDE_GROUP
#define DKV_P1_WIDE_GROUP 2    // tiles per LDS stage of the wide pass 1 (1, 2 or 4)
#endif
#ifndef DKV_P2_WIDE_GROUP
#define DKV_P2_WIDE_GROUP 3    // tiles per LDS stage of the wide pass 2 (1 to 3)
#endif

ScorePlan make_score_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t Lk, int64_t D, int64_t W,
                          int64_t splits) {
  ScorePlan p;
  p.heads = (int)(B * Hkv);
  p.g = (int)(Hq / Hkv);
  p.M = p.g * (int)W;
  p.n_mc = ceil_div(p.M, kRows);
  p.mpad = p.n_mc * kRows;
  p.p1_waves = DKV_P1_WAVES == 8 ? 8 : 4;
  p.p2_waves = 8;
  const int target = DKV_TARGET_WG;
  const int max_by_work = max(1, (int)(Lk / 256));
  // Several row-chunks share each K/V tile in one workgroup (pass1w) from
  // n_mc >= DKV_P1_WIDE_MIN up to one chunk per wave.
  // p1_wide is 0 or the pass1w tile group (1, 2 or 4 tiles per LDS stage).
  p.p1_wide = (DKV_P1_WIDE_MIN > 0 && p.n_mc >= DKV_P1_WIDE_MIN && p.n_mc <= kWideWaves) ? DKV_P1_WIDE_GROUP : 0;
  const int64_t p1_groups = p.p1_wide ? (int64_t)p.heads : (int64_t)p.heads * p.n_mc;
  // Pass 1 of a bandwidth-bound call (a K/V stream of 32 MiB or more) runs
  // fewer, longer splits: the memory system is already saturated with
  // ~160 workgroups, and the merge then combines fewer partials (C2: 20
  // splits per head, 75.3 us per layer-call against 76.9 us with 32).  A
  // small call is latency-bound and keeps one workgroup per CU.
  const bool p1_bw = (int64_t)p.heads * Lk * D * 2 * 2 >= (int64_t(32) << 20);
  const int target1 = (p1_bw && !p.p1_wide) ? DKV_TARGET_P1_BW : target;
  int s1 = splits > 0 ? (int)splits : ceil_div(target1, p1_groups);
  s1 = max(1, min(min(s1, max_by_work), kMaxSplits));
  p.kps1 = ceil_div(ceil_div(Lk, s1), kTile) * kTile;
  p.s1 = ceil_div(Lk, p.kps1);
  // Pass 2: at most one workgroup per CU in all (rounded down), so that the
  // grid runs in one wave and the selection tail's barriers can hold.
  int s2 = splits > 0 ? (int)splits : max(1, target / p.heads);
  s2 = max(1, min(s2, max_by_work));
  p.kps2 = ceil_div(ceil_div(Lk, s2), kTile) * kTile;
  p.s2 = ceil_div(Lk, p.kps2);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += (bytes + 255) & ~size_t(255);
    return o;
  };
  // The call counters first, at a fixed offset, so that no other layout
  // ever writes over them.
  p.off_sync = take(kSyncBytes);
  const size_t slots = (size_t)p.heads * p.n_mc * p.s1;
  p.off_ml = take(slots * kRows * 2 * sizeof(float));
  p.off_y = take(slots * kRows * D * sizeof(float));
  p.off_cand = take(slots * kRows * kCand * sizeof(int2));
  p.off_op = take((size_t)p.heads * p.n_mc * kOpSlots * kMB * (D / 32) * 64 * 16);
  p.off_stb = take((size_t)p.heads * p.n_mc * kMB * kStatWords * sizeof(float));
  p.off_stat = take((size_t)p.heads * p.mpad * 2 * sizeof(float));
  p.off_yf = take((size_t)p.heads * p.mpad * D * sizeof(float));
  p.total = off;
  return p;
}

namespace {
// Process-wide settings of the selection tail, read once per call (relaxed:
// a call in flight on another thread sees either the old or the new value).
std::atomic<int> g_tail_mode{1};          // 1: selection in pass 2's tail whenever the call allows it
std::atomic<int> g_tail_spin{1 << 16};    // polls at the tail's barrier A before a workgroup gives up
std::atomic<int> g_tail_spin_b{1 << 22};  // polls at barrier B before a workgroup finishes the row alone

// Whether `grid` workgroups of `fn` (threads, dynamic LDS bytes) fit on the
// current GPU at once: the tail's barriers need every workgroup of a row
// running.  Looked up once per (device, kernel, LDS size).
bool tail_fits(const void* fn, int threads, size_t lds, int64_t grid) {
  struct Entry {
    int dev;
    const void* fn;
    size_t lds;
    int64_t cap;
  };
  static std::mutex mu;
  static Entry cache[64];
  static int n_cache = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_cache; ++i)
    if (cache[i].dev == dev && cache[i].fn == fn && cache[i].lds == lds) return grid <= cache[i].cap;
  int per_cu = 0, cus = 0, max_lds = 0;
  int64_t cap = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
      lds <= (size_t)max_lds)
    cap = (int64_t)per_cu * cus;
  (void)hipGetLastError();
  if (n_cache < 64) cache[n_cache++] = Entry{dev, fn, lds, cap};
  return grid <= cap;
}
}  // namespace

void set_tail_select(int mode, int spin, int spin_b) {
  g_tail_mode.store(mode, std::memory_order_relaxed);
  if (spin >= 0) g_tail_spin.store(spin, std::memory_order_relaxed);
  if (spin_b >= 0) g_tail_spin_b.store(spin_b, std::memory_order_relaxed);
}

template <typename T, int D>
static hipError_t launch_scores_t(const ScorePlan& p, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                                  int64_t q_sd, const void* k, const void* v, int kv_ld, int Hkv, int Lq, int Lk,
                                  int W, float eps, int p_round, int y_round, float* scores, char* ws,
                                  uint32_t* zero_ptr, int64_t zero_words, const FuseSelect* fuse, hipStream_t st) {
  const float scale_log2 = 1.4426950408889634f / sqrtf((float)D);
  // c^2 = 1/(1+eps)^2 for pass 2's small-p weight, or 0 where eps is outside
  // the range that form is exact for (then every tile takes the exact one).
  const float small_c2 =
      (eps >= 0.f && eps <= kSmallMaxEps) ? (float)(1.0 / ((1.0 + (double)eps) * (1.0 + (double)eps))) : 0.f;
  float* part_ml = reinterpret_cast<float*>(ws + p.off_ml);
  float* part_y = reinterpret_cast<float*>(ws + p.off_y);
  u32x4* opblk = reinterpret_cast<u32x4*>(ws + p.off_op);
  float* stblk = reinterpret_cast<float*>(ws + p.off_stb);
  float* ystat = reinterpret_cast<float*>(ws + p.off_stat);
  float* yf = reinterpret_cast<float*>(ws + p.off_yf);
  int2* part_cand = reinterpret_cast<int2*>(ws + p.off_cand);
  const T* qq = static_cast<const T*>(q);
  const T* kk = static_cast<const T*>(k);
  const T* vv = static_cast<const T*>(v);

  const bool qvec = q_sd == 1 && (q_sb % 8) == 0 && (q_sh % 8) == 0 && (q_ss % 8) == 0 &&
                    (reinterpret_cast<uintptr_t>(q) & 15u) == 0;
  const dim3 g1(p.heads * p.n_mc * p.s1);
  if (p.p1_wide) {
    launch((pass1w_kernel<T, D, DKV_P1_WIDE_GROUP>), dim3(p.heads * p.s1), dim3(64 * kWideWaves), 0, st, qq, q_sb,
           q_sh, q_ss, q_sd, qvec, kk, vv, kv_ld, Hkv, Lq, Lk, W, p.g, p.M, p.n_mc, p.s1, p.kps1, scale_log2, part_ml,
           part_y, part_cand);
  } else if (p.p1_waves == 8) {
    launch((pass1_kernel<T, D, 8, 1>), g1, dim3(512), 0, st, qq, q_sb, q_sh, q_ss, q_sd, qvec, kk, vv, kv_ld, Hkv,
           Lq, Lk, W, p.g, p.M, p.n_mc, p.s1, p.kps1, scale_log2, part_ml, part_y, part_cand);
  } else {
    launch((pass1_kernel<T, D, 4, 1>), g1, dim3(256), 0, st, qq, q_sb, q_sh, q_ss, q_sd, qvec, kk, vv, kv_ld, Hkv,
           Lq, Lk, W, p.g, p.M, p.n_mc, p.s1, p.kps1, scale_log2, part_ml, part_y, part_cand);
  }
  const int n_rows = p.heads * p.mpad;
  launch((merge_kernel<T, D>), dim3((n_rows + kMergeRows - 1) / kMergeRows), dim3(64 * kMergeRows), 0, st,
                     part_ml, part_y, part_cand, p.n_mc, p.s1, p.M, n_rows, p_round, y_round, qq, q_sb, q_sh, q_ss,
                     q_sd, vv, kv_ld, Lk, Hkv, p.g, W, Lq, opblk, stblk, ystat, yf, zero_ptr, zero_words);
  // Named here, right after merge, so that the compiler lays pass 2's code
  // out next to pass 1's and merge's: the three run back to back, and their
  // code shares each CU pair's instruction cache.
  const auto k2 = p_round ? pass2_kernel<T, D, 8, 1, true> : pass2_kernel<T, D, 8, 1, false>;
  SelFuse fz{};
  // Row-chunks whose operands share LDS in one sweep over the keys (every
  // further group streams the workgroup's K/V range again): four when they
  // divide n_mc (as pairs of the two-chunk body: unrolling four chunks pushes
  // pass 2 into register spills), else up to two.
  const int cg = (p.n_mc % 4 == 0) ? 4 : min(p.n_mc, 2);
  size_t lds2 = (size_t)cg * kOpSlots * kMB * (D / 32) * 64 * 16 + (size_t)cg * kMB * kStatWords * sizeof(float);
  if (fuse) {
    fz.enabled = 1;
    fz.ws = sel_layout(fuse->ws, p.heads, Lk, nullptr);
    fz.ks = fuse->ks;
    fz.window = fuse->window;
    fz.sc_lds = p.kps2 <= kScLds;
    // sc_row[] and the histogram after the operands and statistics.
    if (fz.sc_lds) lds2 += (size_t)p.kps2 * 4 + (size_t)(kBins1 + 16) * 4;
    lds2 = std::max(lds2, (size_t)kPoolLdsWords * 4);
  }
  const dim3 g2(p.heads * p.s2);
  if (p.p1_wide) {
    // One sweep over K/V for all row-chunks (pass2w); its LDS is static.
    if (p_round)
      launch((pass2w_kernel<T, D, DKV_P2_WIDE_GROUP, true>), g2, dim3(64 * kWideWaves), 0, st, kk, vv, kv_ld, Hkv, Lq,
             Lk, W, p.g, p.M, p.n_mc, p.s2, p.kps2, scale_log2, eps, small_c2, opblk, stblk, scores, fz);
    else
      launch((pass2w_kernel<T, D, DKV_P2_WIDE_GROUP, false>), g2, dim3(64 * kWideWaves), 0, st, kk, vv, kv_ld, Hkv,
             Lq, Lk, W, p.g, p.M, p.n_mc, p.s2, p.kps2, scale_log2, eps, small_c2, opblk, stblk, scores, fz);
    return hipGetLastError();
  }
  // The whole selection in pass 2's tail: needs the scores in LDS, an
  // output to emit into, and every workgroup of the grid running at once.
  if (fuse && fz.sc_lds && fuse->keep_idx && fuse->cp && g_tail_mode.load(std::memory_order_relaxed) &&
      p.s2 <= kFuseMaxSplits) {
    const size_t lds_t = (size_t)cg * kOpSlots * kMB * (D / 32) * 64 * 16 + (size_t)cg * kMB * kStatWords * 4 +
                         (size_t)p.kps2 * 4 + (size_t)tail_lds_words(512, p.kps2) * 4;
    if (tail_fits(reinterpret_cast<const void*>(k2), 512, lds_t, (int64_t)p.heads * p.s2)) {
      fz.full = 1;
      fz.keep = fuse->keep;
      fz.spin = g_tail_spin.load(std::memory_order_relaxed);
      fz.spin_b = g_tail_spin_b.load(std::memory_order_relaxed);
      fz.out_idx = fuse->keep_idx;
      fz.ca = compact_args(fuse->cp);
      lds2 = std::max(lds2, lds_t);
      if (fuse->tail_done) *fuse->tail_done = 1;
    }
  }
  launch(k2, g2, dim3(512), lds2, st, kk, vv, kv_ld, Hkv, Lq, Lk, W, p.g, p.M, p.n_mc, cg, p.s2, p.kps2, scale_log2,
         eps, small_c2, opblk, stblk, scores, fz);
  return hipGetLastError();
}

hipError_t launch_scores(const ScorePlan& p, int dtype, int D, const void* q, int64_t q_sb, int64_t q_sh,
                         int64_t q_ss, int64_t q_sd, const void* k, const void* v, int kv_ld, int Hkv, int Lq,
                         int Lk, int W, float eps, int p_round, int y_round, float* scores, char* ws,
                         uint32_t* zero_ptr, int64_t zero_words, const FuseSelect* fuse, hipStream_t st) {
  if (scores_generic(dtype, D, p.M)) {
    if (fuse) return hipErrorInvalidValue;  // the generic kernels have no pooling tail
    return launch_scores_generic(p, dtype, D, q, q_sb, q_sh, q_ss, q_sd, k, v, kv_ld, Hkv, Lq, Lk, W, eps, p_round,
                                 y_round, scores, ws, zero_ptr, zero_words, st);
  }
#define DKV_CASE(TT, DD)                                                                                   \
  return launch_scores_t<TT, DD>(p, q, q_sb, q_sh, q_ss, q_sd, k, v, kv_ld, Hkv, Lq, Lk, W, eps, p_round, \
                                 y_round, scores, ws, zero_ptr, zero_words, fuse, st)
  if (dtype == kDtypeBf16) {
    if (D == 32) DKV_CASE(__bf16, 32);
    if (D == 64) DKV_CASE(__bf16, 64);
    if (D == 128) DKV_CASE(__bf16, 128);
  } else if (dtype == kDtypeFp16) {
    if (D == 32) DKV_CASE(_Float16, 32);
    if (D == 64) DKV_CASE(_Float16, 64);
    if (D == 128) DKV_CASE(_Float16, 128);
  }
#undef DKV_CASE
  return hipErrorInvalidValue;
}

// Debug: copy lse (natural log) and fp32 y for the valid rows out of the workspace.
__global__ void debug_state_kernel(const float* __restrict__ ystat, const float* __restrict__ yf, int heads,
                                   int mpad, int M, int D, float* __restrict__ lse_out, float* __restrict__ y_out) {
  const int head = blockIdx.x / M, m = blockIdx.x % M;
  const int64_t rbase = (int64_t)head * mpad + m;
  for (int d = threadIdx.x; d < D; d += blockDim.x) y_out[((int64_t)head * M + m) * D + d] = yf[rbase * D + d];
  if (threadIdx.x == 0) lse_out[(int64_t)head * M + m] = ystat[rbase * 2] * 0.69314718055994531f;
}

hipError_t launch_debug_state(const ScorePlan& p, const char* ws, int D, float* lse_out, float* y_out,
                              hipStream_t st) {
  hipLaunchKernelGGL(debug_state_kernel, dim3(p.heads * p.M), dim3(64), 0, st,
                     reinterpret_cast<const float*>(ws + p.off_stat), reinterpret_cast<const float*>(ws + p.off_yf),
                     p.heads, p.mpad, p.M, D, lse_out, y_out);
  return hipGetLastError();
}

// Matrix-core layout self-test: A[i][k] = i + k/32, B[k][j] = (k%4)-j/16 ... small exact integers.
__global__ void mfma_selftest_kernel(float* out) {
  typedef Elem<__bf16>::v8 v8;
  const int lane = threadIdx.x;
  const int li = lane & 15, lg = lane >> 4;
  v8 a, bop;
  for (int e = 0; e < 8; ++e) {
    const int kidx = 8 * lg + e;
    a[e] = static_cast<__bf16>((float)((li * 3 + kidx) % 7) - 3.0f);
    bop[e] = static_cast<__bf16>((float)((li * 5 + 2 * kidx) % 5) - 2.0f);
  }
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
  c = Elem<__bf16>::mfma(a, bop, c);
  for (int r = 0; r < 4; ++r) out[(4 * lg + r) * 16 + li] = c[r];
}

hipError_t launch_mfma_selftest(float* out, hipStream_t st) {
  hipLaunchKernelGGL(mfma_selftest_kernel, dim3(1), dim3(64), 0, st, out);
  return hipGetLastError();
}

}  // namespace dkv
