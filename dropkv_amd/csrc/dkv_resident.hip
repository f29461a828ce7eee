// Resident layer-call scoring on gfx950: pass 1, the cross-split merge and
// pass 2 in ONE kernel whose workgroups keep their K/V slice's V rows and
// fp32 logits on chip between the passes, so that K and V are streamed from
// memory once instead of twice.
//
// It applies when the whole call fits on chip: D = 128, one row-chunk
// (g * W <= 32 query rows per KV head), bf16/fp16, and at most 1024 keys per
// workgroup with one workgroup per CU (B * Hkv * ceil(Lk / 1024) <= CUs; a
// Llama-3.1-8B layer up to Lk = 32768 on MI355X's 256 CUs).  Per workgroup
// (4 waves, 1024 keys of one head, wave w owning the 32-key tiles w, w+4, ..):
//   V rows       8 tiles x 32 keys x 128 x 2 B per wave, in registers
//                (accumulation registers as storage; 256 per lane);
//   logits       S^T of every (key, row) pair, fp32: 128 KiB of LDS;
//   work area    32 KiB of LDS: the V tile transposed for P.V during the
//                first pass, the waves' merge, then the operand block.
// Phases, per head (its S workgroups):
//   1. stream K and V once: S^T = K Q^T, online softmax, Y^T += V^T P^T
//      (as pass1_kernel), logits kept in LDS; one (m, l, y, candidates)
//      partial per workgroup;
//   2. barrier 1 (all partials of the head written), then the workgroups
//      merge the head's rows (merge_row, one wave per row);
//   3. barrier 2 (all rows merged), then every wave scores its own keys
//      from its registers and the LDS logits (G^T = V Y^T as pass2_kernel)
//      and the workgroup pools its interior (the pass-2 pooling tail).
// The split geometry (S splits of kpw keys) is then that of the selection's
// resolve stage, as after pass 2.
//
// Barriers: per head, counters in the caller's workspace (zero on entry,
// zero again when the call ends).  What a workgroup publishes (its partial,
// its merged rows, the cleared selection words) it writes with
// device-coherent stores (st_dev), waits for them and adds its arrival; the
// others poll with agent-scope atomic loads and acquire.  (An agent-scope
// release fence would write back the XCD's whole L2 instead; those
// write-backs queue up per XCD and cost 2-8 us per barrier.)  Every workgroup of the grid is resident at once when the
// GPU runs nothing else (one workgroup per CU, grid <= CUs), but nothing
// guarantees it: a workgroup that waits at barrier 1 longer than `spin1`
// polls marks the head abandoned (a flag bit in the counter, set by
// compare-and-swap only while some partial is still missing) and exits, as
// do the others when they see the flag; the head's last workgroup to arrive
// then finishes the head alone: it merges every row and scores every key by
// streaming K/V from memory (same instructions on the same operands, so the
// same bits).  Barrier 2 is reached only by workgroups that all passed
// barrier 1 together, so all are resident; its wait is bounded as a hang
// guard that sets the status word.
#include "dkv_common.h"
#include "dkv_internal.h"
#include "dkv_score_dev.h"
#include "dkv_select_dev.h"

namespace dkv {

namespace {

constexpr int kResD = 128;
constexpr int kResWaves = 4;
constexpr int kResNT = 64 * kResWaves;
constexpr int kResTiles = 8;                                          // 32-key tiles per wave
constexpr int kLogitBytes = kResWaves * kResTiles * 2 * kMB * 64 * 16;  // 128 KiB
constexpr int kAuxBytes = kResWaves * kTile * kResD * 2;              // 32 KiB
constexpr int kResOps = kOpSlots * kMB * (kResD / 32);                // operand slots (Q, Y-hi, Y-lo)
constexpr int kYPitchR = kResD + 4;                                   // fp32 row pitch of the waves' merge
// Work-area offsets (bytes).
constexpr int kAuxOps = 0;                                     // operand block, phase 3
constexpr int kAuxStat = kAuxOps + kResOps * 64 * 16;          // statistics
constexpr int kAuxSc = kAuxStat + kMB * kStatWords * 4;        // this workgroup's scores
constexpr int kAuxRed = kAuxSc + kResKeys * 4;                 // 16 words for block reductions
constexpr int kAuxState = kAuxRed + 64;                        // barrier outcome
static_assert(kAuxState + 16 <= kAuxBytes, "work area");
constexpr int kAuxMergeY = 5632;                               // the waves' merge: y rows after the stats
static_assert(kAuxMergeY + kRows * kYPitchR * 4 <= kAuxBytes, "merge area");
static_assert(kPoolLdsWords * 4 <= kLogitBytes, "pooling scratch of the lone-finish path");

constexpr uint32_t kPoison = 0x80000000u;
constexpr int kStGo = 0, kStLeave = 1, kStAlone = 2, kStFail = 3;
constexpr int kSpin2 = 1 << 22;  // polls at barrier 2 before the hang guard gives up

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every wave's device-coherent stores complete (the caller adds its arrival
// right after).  On the other side one acquire by thread 0 followed by a
// workgroup barrier covers the workgroup's later loads (the fence
// invalidates the CU's and the XCD's caches, which every wave shares).
__device__ __forceinline__ void publish() {
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// Thread 0 at barrier 1: arrival, then the wait (see the file comment).
__device__ int barrier1(uint32_t* c1, int S, int spin) {
  const uint32_t old = atomicAdd(c1, 1u);
  if ((old & ~kPoison) == (uint32_t)S - 1u) return (old & kPoison) ? kStAlone : kStGo;
  if (old & kPoison) return kStLeave;
  for (int n = 0;; ++n) {
    const uint32_t c = ld_agent(c1);
    if (c & kPoison) return kStLeave;
    if (c == (uint32_t)S) return kStGo;
    if (n >= spin) {
      uint32_t expect = c;
      if (__hip_atomic_compare_exchange_strong(c1, &expect, c | kPoison, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        return kStLeave;
      continue;  // the counter moved: look again
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

struct ResArgs {
  const void* q;
  int64_t q_sb, q_sh, q_ss, q_sd;
  int qvec;
  const void* k;
  const void* v;
  int kv_ld;
  int Hkv, Lq, Lk, W, g, M;
  int S, kpw;  // workgroups per head, keys per workgroup
  float scale_log2, eps;
  int p_round, y_round;
  float* part_ml;
  float* part_y;
  int2* part_cand;
  u32x4* opblk;
  float* stblk;
  float* ystat;
  float* yf32;
  float* scores;
  SelFuse fz;
  uint32_t* sync;  // [heads][4]: barrier-1 arrivals, barrier-2 arrivals, departures, status
  int spin1;
};

// One 32-key tile of the score pass (pass2_kernel's tile for one row-chunk):
// S^T given (sacc, the raw K Q^T products), V as the MFMA A operand (vop),
// the operand block and statistics in LDS.  Stores the keys' scores below
// k_end to srow and, when sc is given, to sc[n - k_begin].
template <typename T, bool PR>
__device__ __forceinline__ void score_tile(const f32x4 (&sacc)[2][kMB], const typename Elem<T>::v8 (&vop)[2][kResD / 32],
                                           const u32x4* opnd, const float* stat, int t0, int k_begin, int k_end,
                                           int M, int W, int Lk, bool pad_rows, float scale_log2, float eps,
                                           float out_scale, float* __restrict__ srow, float* sc) {
  typedef typename Elem<T>::v8 v8;
  constexpr int KK = kResD / 32;
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  float vn2[2][4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    float part = 0.f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) part = sumsq8<T>(vop[kb][kk], part);
    part = add_xor32(add_xor16(part));
#pragma unroll
    for (int r = 0; r < 4; ++r) vn2[kb][r] = __shfl(part, 4 * lg + r);
  }
  f32x4 gacc[2][kMB];
  const u32x4* ob = opnd + lane;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const float nyh = -0.5f * stat[mb * kStatWords + 16 + li];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) gacc[kb][mb][r] = fmaf(vn2[kb][r], -0.5f, nyh);
  }
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const v8 yh = __builtin_bit_cast(v8, ob[(size_t)((1 * kMB + mb) * KK + kk) * 64]);
      const v8 yl = __builtin_bit_cast(v8, ob[(size_t)((2 * kMB + mb) * KK + kk) * 64]);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        gacc[kb][mb] = Elem<T>::mfma(vop[kb][kk], yh, gacc[kb][mb]);
        gacc[kb][mb] = Elem<T>::mfma(vop[kb][kk], yl, gacc[kb][mb]);
      }
    }
  float sc2[2][4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r) sc2[kb][r] = 0.f;
  const float* cst = stat + li;
  bool sink_here = false;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
    sink_here |= (uint32_t)(__builtin_bit_cast(int, cst[mb * kStatWords + 32]) - t0) < (uint32_t)kTile;
  auto epilogue = [&](auto masked_c) __attribute__((always_inline)) {
    constexpr bool kMasked = decltype(masked_c)::value;
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
      const int m = mb * 16 + li;
      const int bound = kMasked ? row_bound(m, M, W, Lk) : 0;
      const int skey = kMasked ? __builtin_bit_cast(int, cst[mb * kStatWords + 32]) : -1;
      const float snd2 = kMasked ? cst[mb * kStatWords + 48] : 0.f;
      const float lse2 = cst[mb * kStatWords];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          float p[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            p[e] = __builtin_amdgcn_exp2f(sacc[kb][mb][r + e] * scale_log2 - lse2);
            if (kMasked) p[e] = (t0 + 16 * kb + 4 * lg + r + e) <= bound ? p[e] : 0.f;
            p[e] = min_one_nonneg(p[e]);
          }
          if (PR) round_through2<T>(p[0], p[1]);
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float ratio = p[e] * __builtin_amdgcn_rcpf(1.0f - p[e] + eps);
            float nd2 = min_zero(gacc[kb][mb][r + e]);  // -dist2/2, dist2 clamped at 0
            if (kMasked) nd2 = (t0 + 16 * kb + 4 * lg + r + e) == skey ? snd2 : nd2;
            sc2[kb][r + e] = fmaf(ratio * ratio, nd2, sc2[kb][r + e]);
          }
        }
    }
  };
  if (pad_rows || t0 + kTile > Lk - W + 1 || __any(sink_here))
    epilogue(std::true_type{});
  else
    epilogue(std::false_type{});
  // Sum over the 16 query rows of lanes li = 0..15 (a reduce-scatter: lane
  // li with li % 4 == 0 ends with the total of key r = li / 4).
  const bool h8 = li & 8, h4 = li & 4;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    float k0 = h8 ? sc2[kb][2] : sc2[kb][0];
    float k1 = h8 ? sc2[kb][3] : sc2[kb][1];
    k0 += __shfl_xor(h8 ? sc2[kb][0] : sc2[kb][2], 8);
    k1 += __shfl_xor(h8 ? sc2[kb][1] : sc2[kb][3], 8);
    float v = h4 ? k1 : k0;
    v += __shfl_xor(h4 ? k0 : k1, 4);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 1);
    const int n = t0 + 16 * kb + 4 * lg + (li >> 2);
    if ((li & 3) == 0 && n < k_end) {
      srow[n] = v * out_scale;
      if (sc) sc[n - k_begin] = v * out_scale;
    }
  }
}

// Two tiles of the score pass at once (tiles u = 0, 1 starting at keys
// t0[u]), in one basic block so that their dependency chains interleave: with
// one wave per SIMD nothing else hides the latencies.  The operands are read
// from LDS once for both.  kMasked: the causal bound and the rows' dominant
// keys are applied (chosen for the pair by the caller).  Keys at or past
// k_end are computed but not stored.
template <typename T, bool PR, bool kMasked>
__device__ __forceinline__ void score_pair(const f32x4 (&sacc)[2][2][kMB],
                                           const typename Elem<T>::v8 (&vA)[2][kResD / 32],
                                           const typename Elem<T>::v8 (&vB)[2][kResD / 32], const u32x4* opnd,
                                           const float* stat, const int (&t0)[2], int k_begin, int k_end, int M,
                                           int W, int Lk, float scale_log2, float eps, float out_scale,
                                           float* __restrict__ srow, float* sc) {
  typedef typename Elem<T>::v8 v8;
  constexpr int KK = kResD / 32;
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  auto both = [&](auto&& f) __attribute__((always_inline)) {
    f(std::integral_constant<int, 0>{});
    f(std::integral_constant<int, 1>{});
  };
  auto vop = [&](auto uc, int kb, int kk) __attribute__((always_inline)) -> v8 {
    if constexpr (decltype(uc)::value == 0)
      return vA[kb][kk];
    else
      return vB[kb][kk];
  };
  const float* cst = stat + li;
  float vn2[2][2][4];
  both([&](auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float part = 0.f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) part = sumsq8<T>(vop(uc, kb, kk), part);
      part = add_xor32(add_xor16(part));
#pragma unroll
      for (int r = 0; r < 4; ++r) vn2[u][kb][r] = __shfl(part, 4 * lg + r);
    }
  });
  f32x4 gacc[2][2][kMB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const float nyh = -0.5f * cst[mb * kStatWords + 16];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) gacc[u][kb][mb][r] = fmaf(vn2[u][kb][r], -0.5f, nyh);
  }
  const u32x4* ob = opnd + lane;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const v8 yh = __builtin_bit_cast(v8, ob[(size_t)((1 * kMB + mb) * KK + kk) * 64]);
      const v8 yl = __builtin_bit_cast(v8, ob[(size_t)((2 * kMB + mb) * KK + kk) * 64]);
      both([&](auto uc) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          gacc[u][kb][mb] = Elem<T>::mfma(vop(uc, kb, kk), yh, gacc[u][kb][mb]);
          gacc[u][kb][mb] = Elem<T>::mfma(vop(uc, kb, kk), yl, gacc[u][kb][mb]);
        }
      });
    }
  float sc2[2][2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) sc2[u][kb][r] = 0.f;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const int m = mb * 16 + li;
    const int bound = kMasked ? row_bound(m, M, W, Lk) : 0;
    const int skey = kMasked ? __builtin_bit_cast(int, cst[mb * kStatWords + 32]) : -1;
    const float snd2 = kMasked ? cst[mb * kStatWords + 48] : 0.f;
    const float lse2 = cst[mb * kStatWords];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          float p[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            p[e] = __builtin_amdgcn_exp2f(sacc[u][kb][mb][r + e] * scale_log2 - lse2);
            if (kMasked) p[e] = (t0[u] + 16 * kb + 4 * lg + r + e) <= bound ? p[e] : 0.f;
            p[e] = min_one_nonneg(p[e]);
          }
          if (PR) round_through2<T>(p[0], p[1]);
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float ratio = p[e] * __builtin_amdgcn_rcpf(1.0f - p[e] + eps);
            float nd2 = min_zero(gacc[u][kb][mb][r + e]);  // -dist2/2, dist2 clamped at 0
            if (kMasked) nd2 = (t0[u] + 16 * kb + 4 * lg + r + e) == skey ? snd2 : nd2;
            sc2[u][kb][r + e] = fmaf(ratio * ratio, nd2, sc2[u][kb][r + e]);
          }
        }
  }
  const bool h8 = li & 8, h4 = li & 4;
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float k0 = h8 ? sc2[u][kb][2] : sc2[u][kb][0];
      float k1 = h8 ? sc2[u][kb][3] : sc2[u][kb][1];
      k0 += __shfl_xor(h8 ? sc2[u][kb][0] : sc2[u][kb][2], 8);
      k1 += __shfl_xor(h8 ? sc2[u][kb][1] : sc2[u][kb][3], 8);
      float v = h4 ? k1 : k0;
      v += __shfl_xor(h4 ? k0 : k1, 4);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 1);
      const int n = t0[u] + 16 * kb + 4 * lg + (li >> 2);
      if ((li & 3) == 0 && n < k_end) {
        srow[n] = v * out_scale;
        if (sc) sc[n - k_begin] = v * out_scale;
      }
    }
}

// Operand block and statistics of `head` (written by merge_row) into LDS.
__device__ __forceinline__ void stage_operands(const ResArgs& a, int head, u32x4* opnd, float* stat) {
  const u32x4* gop = a.opblk + (size_t)head * kResOps * 64;
  const float* gst = a.stblk + (size_t)head * kMB * kStatWords;
  for (int i = threadIdx.x; i < kResOps * 64; i += kResNT) opnd[i] = gop[i];
  if ((int)threadIdx.x < kMB * kStatWords) stat[threadIdx.x] = gst[threadIdx.x];
}

// The pooling tail of one split [k_begin, k_end): its interior keys.
__device__ __forceinline__ void interior(int split, int k_begin, int k_end, int Lk, int h, int* i0, int* i1) {
  *i0 = split == 0 ? 0 : k_begin + h;
  *i1 = k_end >= Lk ? Lk : k_end - h;
}

// The head finished by one workgroup (barrier 1 abandoned): every row
// merged, every key scored from K/V streamed from memory, every split's
// interior pooled; then the counters cleared once the others have left.
template <typename T, bool PR>
__device__ void finish_alone(const ResArgs& a, int head, unsigned char* lds) {
  typedef typename Elem<T>::v8 v8;
  constexpr int D = kResD, KK = D / 32;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const T* q = static_cast<const T*>(a.q);
  const T* vp = static_cast<const T*>(a.v);
  const T* kp = static_cast<const T*>(a.k);
  const int heads_rows = (int)(gridDim.x / a.S) * kRows;  // every head's padded rows
  for (int r = wv; r < kRows; r += kResWaves)
    merge_row<T, D, true>(head * kRows + r, a.part_ml, a.part_y, a.part_cand, 1, a.S, a.M, heads_rows, a.p_round,
                          a.y_round, q, a.q_sb, a.q_sh, a.q_ss, a.q_sd, vp, a.kv_ld, a.Lk, a.Hkv, a.g, a.W, a.Lq,
                          a.opblk, a.stblk, a.ystat, a.yf32);
  publish();
  if (threadIdx.x == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __syncthreads();
  unsigned char* aux = lds + kLogitBytes;
  u32x4* opnd = reinterpret_cast<u32x4*>(aux + kAuxOps);
  float* stat = reinterpret_cast<float*>(aux + kAuxStat);
  stage_operands(a, head, opnd, stat);
  __syncthreads();
  const float out_scale = -2.0f * (1.0f / static_cast<float>(a.g));
  float* srow = a.scores + (int64_t)head * a.Lk;
  const uint32_t k_lane = (li * D + 8 * lg) * sizeof(T);
  const int h = a.fz.ks / 2;
  for (int s = 0; s < a.S; ++s) {
    const int k_begin = s * a.kpw;
    if (k_begin >= a.Lk) break;
    const int k_end = min(k_begin + a.kpw, a.Lk);
    const int64_t roff = ((int64_t)head * a.kv_ld + k_begin) * D;
    const uint32_t range = (uint32_t)(k_end - k_begin) * (D * sizeof(T));
    const rsrc_t krs = make_rsrc(kp + roff, range), vrs = make_rsrc(vp + roff, range);
    for (int t = wv * kTile; t < k_end - k_begin; t += kResWaves * kTile) {
      v8 kop[2][KK], vop[2][KK];
      load_rows_op<T, D>(kop, krs, k_lane, t);
      load_rows_op<T, D>(vop, vrs, k_lane, t);
      f32x4 sacc[2][kMB];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < KK; ++kk)
            acc = Elem<T>::mfma(kop[kb][kk], __builtin_bit_cast(v8, opnd[(size_t)(mb * KK + kk) * 64 + lane]), acc);
          sacc[kb][mb] = acc;
        }
      score_tile<T, PR>(sacc, vop, opnd, stat, k_begin + t, k_begin, k_end, a.M, a.W, a.Lk, kRows > a.M,
                        a.scale_log2, a.eps, out_scale, srow, nullptr);
    }
    if (a.fz.enabled) {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // the split's scores are stored
      int i0, i1;
      interior(s, k_begin, k_end, a.Lk, h, &i0, &i1);
      uint32_t* L = reinterpret_cast<uint32_t*>(lds);
      pool_range<kResNT>(srow, a.fz.ws.pooled + (int64_t)head * a.Lk, a.fz.ws.rowws + (int64_t)head * kRowWords,
                         a.Lk, h, a.Lk - a.fz.window, i0, i1, reinterpret_cast<float*>(L), L + kSub + 2 * kMaxHalo,
                         L + kSub + 2 * kMaxHalo + kBins1);
    }
  }
  if (threadIdx.x == 0) {
    uint32_t* sy = a.sync + (size_t)head * 4;
    int n = 0;
    while (ld_agent(sy + 2) != (uint32_t)a.S - 1u && n < kSpin2) {
      __builtin_amdgcn_s_sleep(2);
      ++n;
    }
    if (n >= kSpin2) atomicOr(sy + 3, 1u);
    st_agent(sy + 0, 0u);
    st_agent(sy + 1, 0u);
    st_agent(sy + 2, 0u);
  }
}

template <typename T, bool PR>
__global__ void __launch_bounds__(kResNT, 1) resident_kernel(ResArgs a) {
  typedef typename Elem<T>::v8 v8;
  constexpr int D = kResD, KK = D / 32, DT = D / 16;
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLogitBytes + kAuxBytes];
  unsigned char* aux = lds + kLogitBytes;

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int split = lid % a.S, head = lid / a.S;
  const int b = head / a.Hkv, hkv = head % a.Hkv;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const T* q = static_cast<const T*>(a.q);
  const T* kp = static_cast<const T*>(a.k);
  const T* vp = static_cast<const T*>(a.v);
  const int Lk = a.Lk, M = a.M;

  // ---- Phase 1 ----------------------------------------------------------
  v8 qop[kMB][KK];
  int bound[kMB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const int m = mb * 16 + li;
    load_q_ops<T, D>(qop[mb], q, a.q_sb, a.q_sh, a.q_ss, a.q_sd, a.qvec, b, hkv, a.g, a.W, a.Lq, M, m, lg);
    bound[mb] = row_bound(m, M, a.W, Lk);
  }
  const bool pad_rows = kRows > M;
  const int unmasked_end = Lk - a.W + 1;
  const int k_begin = split * a.kpw;
  const int k_end = min(k_begin + a.kpw, Lk);
  const int nrel = max(k_end - k_begin, 0);
  const int64_t roff = ((int64_t)head * a.kv_ld + k_begin) * D;
  const uint32_t range = (uint32_t)nrel * (D * sizeof(T));
  const rsrc_t krs = make_rsrc(kp + roff, range), vrs = make_rsrc(vp + roff, range);
  const uint32_t k_lane = (li * D + 8 * lg) * sizeof(T);
  // This wave's logits: slot (tile i, kb, mb), lane-contiguous 16 bytes.
  f32x4* logit = reinterpret_cast<f32x4*>(lds) + (size_t)wv * kResTiles * 2 * kMB * 64 + lane;
  // This wave's V tile, row-major with 8-byte chunks XOR-swizzled by row, for
  // the transposing reads (ds_read_b64_tr_b16).
  unsigned char* vt = aux + wv * (kTile * D * 2);
  auto trel = [&](int i) { return (i * kResWaves + wv) * kTile; };

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
  v8 vres[kResTiles][2][KK];  // this wave's V rows, for the whole kernel
  v8 kbuf[2][2][KK];          // K tiles, two in flight
  load_rows_op<T, D>(kbuf[0], krs, k_lane, trel(0));
  load_rows_op<T, D>(vres[0], vrs, k_lane, trel(0));
  load_rows_op<T, D>(kbuf[1], krs, k_lane, trel(1));
  load_rows_op<T, D>(vres[1], vrs, k_lane, trel(1));
#pragma unroll
  for (int i = 0; i < kResTiles; ++i) {
    const int tr0 = trel(i);
    if (tr0 >= nrel) break;
    v8 (&kop)[2][KK] = kbuf[i & 1];
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
    // Two tiles ahead (zeros past the range, no memory request).
    if (i + 2 < kResTiles) {
      load_rows_op<T, D>(kop, krs, k_lane, trel(i + 2));
      load_rows_op<T, D>(vres[i + 2], vrs, k_lane, trel(i + 2));
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) logit[(i * 2 * kMB + kb * kMB + mb) * 64] = s[kb][mb];
    // V rows into the wave's tile: lane (li, lg) holds row 16kb+li, columns
    // 32kk+8lg..+7 (16 bytes = 8-byte chunks 2c, 2c+1 of c = 4kk+lg).
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int r = 16 * kb + li;
        const int pc8 = (8 * kk + 2 * lg) ^ (4 * (r & 7));
        *reinterpret_cast<v8*>(vt + r * (D * 2) + pc8 * 8) = vres[i][kb][kk];
      }
    const int t0 = k_begin + tr0;
    v8 phi[kMB], plo[kMB];
    if (pad_rows || t0 + kTile > unmasked_end)
      softmax_tile<T, D, true>(s, m2, lsum, lmax, larg, yacc, phi, plo, bound, t0, lg, a.scale_log2);
    else
      softmax_tile<T, D, false>(s, m2, lsum, lmax, larg, yacc, phi, plo, bound, t0, lg, a.scale_log2);
    // Y^T += V^T P^T.  The A operand of lane (li, lg) is V^T[16dt+li][keys
    // 4lg..4lg+3, 16+4lg..+3]: two transposing reads, in which source lane
    // 4e + i/4 of each 16-lane group supplies row 4lg+e (+16), columns
    // 16dt + 4(i%4) .. +3.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      v4s hv[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int r = 16 * half + 4 * lg + (li >> 2);
        const int pc8 = (4 * dt + (li & 3)) ^ (4 * (r & 7));
        typedef __attribute__((address_space(3))) unsigned char lds_u8;
        hv[half] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(lds_u8*)(vt + r * (D * 2) + pc8 * 8));
      }
      const v8 aop = __builtin_bit_cast(v8, __builtin_shufflevector(hv[0], hv[1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        yacc[dt][mb] = Elem<T>::mfma(aop, phi[mb], yacc[dt][mb]);
        yacc[dt][mb] = Elem<T>::mfma(aop, plo[mb], yacc[dt][mb]);
      }
    }
  }
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) lsum[mb] = add_xor32(add_xor16(lsum[mb]));

  // The waves' partials merged in the work area (the V tiles are dead):
  // statistics and candidates first, then the y rows accumulated wave by
  // wave with weights 2^(m_w - max_w m_w).
  __syncthreads();
  float* sm_m = reinterpret_cast<float*>(aux);
  float* sm_l = sm_m + kResWaves * kRows;
  float* sm_cs = sm_l + kResWaves * kRows;                   // [waves][rows][4]
  int* sm_ck = reinterpret_cast<int*>(sm_cs + 4 * kResWaves * kRows);
  float* ybuf = reinterpret_cast<float*>(aux + kAuxMergeY);  // [rows][kYPitchR]
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const int ci = (wv * kRows + 16 * mb + li) * 4 + lg;
    sort_lane_groups(lmax[mb], larg[mb], lg);
    sm_cs[ci] = lmax[mb];
    sm_ck[ci] = larg[mb];
    if (lg == 0) {
      sm_m[wv * kRows + 16 * mb + li] = m2[mb];
      sm_l[wv * kRows + 16 * mb + li] = lsum[mb];
    }
  }
  __syncthreads();
  float fw[kMB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    const int row = 16 * mb + li;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kResWaves; ++w) mx = fmaxf(mx, sm_m[w * kRows + row]);
    fw[mb] = m2[mb] == -INFINITY ? 0.f : exp2f(m2[mb] - mx);
  }
#pragma unroll
  for (int w = 0; w < kResWaves; ++w) {
    if (wv == w) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
          f32x4* p = reinterpret_cast<f32x4*>(ybuf + (16 * mb + li) * kYPitchR + 16 * dt + 4 * lg);
          const f32x4 v = yacc[dt][mb] * fw[mb];
          *p = w == 0 ? v : *p + v;
        }
    }
    __syncthreads();
  }
  const int64_t slot = (int64_t)head * a.S + split;
  if (threadIdx.x < kRows) {
    const int row = threadIdx.x;
    float mx = -INFINITY;
    for (int w = 0; w < kResWaves; ++w) mx = fmaxf(mx, sm_m[w * kRows + row]);
    float l = 0.f;
    for (int w = 0; w < kResWaves; ++w) {
      const float mw = sm_m[w * kRows + row];
      l += sm_l[w * kRows + row] * ((mw == -INFINITY) ? 0.f : exp2f(mw - mx));
    }
    st_dev(reinterpret_cast<uint64_t*>(a.part_ml + (slot * kRows + row) * 2), __builtin_bit_cast(uint64_t, f32x2{mx, l}));
    float cs[kCand];
    int ck[kCand];
    merge_wave_cands<kResWaves>(sm_cs, sm_ck, row, cs, ck);
#pragma unroll
    for (int j = 0; j < kCand; ++j)
      st_dev(reinterpret_cast<uint64_t*>(a.part_cand + (slot * kRows + row) * kCand + j),
             __builtin_bit_cast(uint64_t, i32x2{ck[j], __float_as_int(cs[j])}));
  }
  float* py = a.part_y + slot * kRows * D;
  for (int i = 2 * threadIdx.x; i < kRows * D; i += 2 * kResNT) {
    const float* yr = ybuf + (i / D) * kYPitchR + i % D;
    st_dev(reinterpret_cast<uint64_t*>(py + i), __builtin_bit_cast(uint64_t, f32x2{yr[0], yr[1]}));
  }
  // The selection's per-row words start at zero (the pooling tail adds to them).
  if (a.fz.enabled && split == 0)
    for (int i = threadIdx.x; i < kRowWords; i += kResNT) st_dev(a.fz.ws.rowws + (int64_t)head * kRowWords + i, 0u);

  // ---- Barrier 1 ----------------------------------------------------------
  uint32_t* sy = a.sync + (size_t)head * 4;
  int* s_state = reinterpret_cast<int*>(aux + kAuxState);
  publish();
  if (threadIdx.x == 0) {
    const int st = barrier1(sy, a.S, a.spin1);
    if (st != kStLeave) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // for the whole workgroup
    s_state[0] = st;
  }
  __syncthreads();
  const int st1 = s_state[0];
  if (st1 == kStLeave) {
    if (threadIdx.x == 0) atomicAdd(sy + 2, 1u);
    return;
  }
  if (st1 == kStAlone) {
    __syncthreads();  // s_state read by every thread before the LDS is reused
    finish_alone<T, PR>(a, head, lds);
    return;
  }

  // ---- Merge: this workgroup's rows of the head, one wave each --------------
  const int heads_rows = (int)(gridDim.x / a.S) * kRows;
  for (int r = split + a.S * wv; r < kRows; r += a.S * kResWaves)
    merge_row<T, D, true>(head * kRows + r, a.part_ml, a.part_y, a.part_cand, 1, a.S, M, heads_rows, a.p_round,
                          a.y_round, q, a.q_sb, a.q_sh, a.q_ss, a.q_sd, vp, a.kv_ld, Lk, a.Hkv, a.g, a.W, a.Lq,
                          a.opblk, a.stblk, a.ystat, a.yf32);

  // ---- Barrier 2 ----------------------------------------------------------
  publish();
  if (threadIdx.x == 0) {
    atomicAdd(sy + 1, 1u);
    int st = kStGo, n = 0;
    while (ld_agent(sy + 1) != (uint32_t)a.S) {
      if (++n >= kSpin2) {
        st = kStFail;
        atomicOr(sy + 3, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    // Departure; the last one clears the counters for the next call.
    if (atomicAdd(sy + 2, 1u) == (uint32_t)a.S - 1u) {
      st_agent(sy + 0, 0u);
      st_agent(sy + 1, 0u);
      st_agent(sy + 2, 0u);
    }
    if (st == kStGo) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // for the whole workgroup
    s_state[0] = st;
  }
  __syncthreads();
  if (s_state[0] == kStFail) return;

  // ---- Phase 3: the scores of this workgroup's keys ------------------------
  u32x4* opnd = reinterpret_cast<u32x4*>(aux + kAuxOps);
  float* stat = reinterpret_cast<float*>(aux + kAuxStat);
  float* sc = reinterpret_cast<float*>(aux + kAuxSc);
  stage_operands(a, head, opnd, stat);
  __syncthreads();
  const float out_scale = -2.0f * (1.0f / static_cast<float>(a.g));
  float* srow = a.scores + (int64_t)head * Lk;
  // Tiles in pairs (i, i+1); a pair whose second tile lies past the range
  // computes it on stale logits and zero V rows and stores none of it.
  const float* cst = stat + li;
#pragma unroll
  for (int i = 0; i < kResTiles; i += 2) {
    if (trel(i) >= nrel) break;
    const int t0[2] = {k_begin + trel(i), k_begin + trel(i + 1)};
    f32x4 s[2][2][kMB];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) s[u][kb][mb] = logit[((i + u) * 2 * kMB + kb * kMB + mb) * 64];
    bool sink_here = false;
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
      const int sk = __builtin_bit_cast(int, cst[mb * kStatWords + 32]);
      sink_here |= (uint32_t)(sk - t0[0]) < (uint32_t)kTile || (uint32_t)(sk - t0[1]) < (uint32_t)kTile;
    }
    float* scp = a.fz.enabled ? sc : nullptr;
    if (pad_rows || t0[1] + kTile > unmasked_end || __any(sink_here))
      score_pair<T, PR, true>(s, vres[i], vres[i + 1], opnd, stat, t0, k_begin, k_end, M, a.W, Lk, a.scale_log2,
                              a.eps, out_scale, srow, scp);
    else
      score_pair<T, PR, false>(s, vres[i], vres[i + 1], opnd, stat, t0, k_begin, k_end, M, a.W, Lk, a.scale_log2,
                               a.eps, out_scale, srow, scp);
  }
  if (a.fz.enabled) {
    __syncthreads();  // scores in LDS; the logits are dead
    uint32_t* hist = reinterpret_cast<uint32_t*>(lds);
    for (int i = threadIdx.x; i < kBins1; i += kResNT) hist[i] = 0u;
    __syncthreads();
    const int h = a.fz.ks / 2;
    int i0, i1;
    interior(split, k_begin, k_end, Lk, h, &i0, &i1);
    pool_range_lds<kResNT>(sc, k_begin, a.fz.ws.pooled + (int64_t)head * Lk,
                           a.fz.ws.rowws + (int64_t)head * kRowWords, Lk, h, Lk - a.fz.window, i0, i1, hist,
                           reinterpret_cast<uint32_t*>(aux + kAuxRed));
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
namespace {
int g_res_mode = 0;            // 0: never, 1: when the call fits
int g_res_spin1 = 1 << 16;     // polls at barrier 1 before a workgroup gives up
constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices];        // CUs per device ordinal (0: not looked up yet)

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  if (!g_cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}
}  // namespace

void set_resident(int mode, int spin1) {
  g_res_mode = mode;
  if (spin1 >= 0) g_res_spin1 = spin1;
}

bool resident_plan(int dtype, int64_t D, int64_t M, int64_t heads, int64_t Lk, int64_t splits, int* S, int* kpw) {
  if (g_res_mode == 0 || splits != 0) return false;
  if ((dtype != kDtypeBf16 && dtype != kDtypeFp16) || D != kResD || M < 1 || M > kRows) return false;
  if (heads < 1 || heads > kResMaxHeads || Lk < 1) return false;
  const int64_t s = (Lk + kResKeys - 1) / kResKeys;
  const int cus = device_cus();
  if (cus <= 0 || heads * s > cus || heads * s > kResMaxHeads) return false;  // the plan sized its partials for this
  *S = (int)s;
  *kpw = kResKeys;
  return true;
}

hipError_t launch_resident(const ScorePlan& p, int dtype, int S, int kpw, const void* q, int64_t q_sb,
                           int64_t q_sh, int64_t q_ss, int64_t q_sd, const void* k, const void* v, int kv_ld,
                           int Hkv, int Lq, int Lk, int W, float eps, int p_round, int y_round, float* scores,
                           char* ws, const FuseSelect* fuse, hipStream_t st) {
  ResArgs a{};
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_ss = q_ss;
  a.q_sd = q_sd;
  a.qvec = q_sd == 1 && (q_sb % 8) == 0 && (q_sh % 8) == 0 && (q_ss % 8) == 0 &&
           (reinterpret_cast<uintptr_t>(q) & 15u) == 0;
  a.k = k;
  a.v = v;
  a.kv_ld = kv_ld;
  a.Hkv = Hkv;
  a.Lq = Lq;
  a.Lk = Lk;
  a.W = W;
  a.g = p.g;
  a.M = p.M;
  a.S = S;
  a.kpw = kpw;
  a.scale_log2 = 1.4426950408889634f / sqrtf((float)kResD);
  a.eps = eps;
  a.p_round = p_round;
  a.y_round = y_round;
  a.part_ml = reinterpret_cast<float*>(ws + p.off_ml);
  a.part_y = reinterpret_cast<float*>(ws + p.off_y);
  a.part_cand = reinterpret_cast<int2*>(ws + p.off_cand);
  a.opblk = reinterpret_cast<u32x4*>(ws + p.off_op);
  a.stblk = reinterpret_cast<float*>(ws + p.off_stb);
  a.ystat = reinterpret_cast<float*>(ws + p.off_stat);
  a.yf32 = reinterpret_cast<float*>(ws + p.off_yf);
  a.scores = scores;
  if (fuse) {
    a.fz.enabled = 1;
    a.fz.ws = sel_layout(fuse->ws, p.heads, Lk, nullptr);
    a.fz.ks = fuse->ks;
    a.fz.window = fuse->window;
    a.fz.sc_lds = 1;
  }
  a.sync = reinterpret_cast<uint32_t*>(ws + p.off_sync);
  a.spin1 = g_res_spin1;
  const dim3 grid((unsigned)(p.heads * S)), block(kResNT);
  if (dtype == kDtypeBf16) {
    if (p_round)
      launch(resident_kernel<__bf16, true>, grid, block, 0, st, a);
    else
      launch(resident_kernel<__bf16, false>, grid, block, 0, st, a);
  } else {
    if (p_round)
      launch(resident_kernel<_Float16, true>, grid, block, 0, st, a);
    else
      launch(resident_kernel<_Float16, false>, grid, block, 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace dkv
