// The selection of a layer-call run in the tail of the scoring pass
// (pass2_kernel): pooling, the top-k threshold, the ordered emit of the kept
// indices and the K/V gather happen in the launch that computes the scores,
// with two barriers among the S pass-2 workgroups of each row (one per key
// split), instead of two further kernels (resolve, emit) and their launch
// gaps.  Reference semantics as in dkv_select_dev.h (dropkv_cache.py:464-491).
//
//   0. Every workgroup pools its interior keys (whole window inside its
//      split) from its scores in LDS, into LDS and the pooled row, adds them
//      to the row's top-digit histogram and maximum, and publishes the raw
//      scores next to its split boundaries.
//   A. Barrier A: every contribution of the row is in.
//   1. Every workgroup loads the row's histogram, maximum and boundary raw
//      scores, pools all boundary keys of the row (the histogram needs every
//      key; its own boundary keys also go to LDS and the pooled row) and finds
//      the top-digit bin b1 of the keep-th largest key.
//   2. It counts its keys above b1 and appends its keys inside b1 (the
//      candidates) to the row's list.
//   B. Barrier B: every count and candidate is in.
//   3. Every workgroup resolves digits 2 and 3 over the candidate list (the
//      same threshold T everywhere), counts the kept keys above T and the keys
//      equal to T in the splits before its own, writes its kept indices in
//      index order and gathers their K/V rows.
//
// Publishing uses device-coherent stores (st_dev), a wait for them and then
// the arrival; the waiting side polls with agent-scope loads.
//
// Barrier A is the one place where a workgroup could wait for another that
// is not running: the host takes this path only when the whole grid fits on
// the GPU at once, but nothing guarantees that the GPU runs nothing else.  A
// workgroup that waits longer than `spin` polls marks the row abandoned (a
// flag bit set by compare-and-swap while an arrival is still missing) and
// leaves, as do the others when they see the flag; the row's last workgroup
// to arrive then finishes the row alone from the pooled row in memory (the
// same keys, so the same result).  Barrier B is reached only by workgroups
// that passed A together, all running, so its wait ends; it is still bounded
// (`spin_b` polls).  A workgroup that gives up there writes the pooled
// values of every boundary key of the row (it has them all) and finishes the
// whole row alone from the pooled row in memory, as at barrier A: every
// workgroup that finishes the row, alone or not, writes the same indices and
// rows, so the outputs are those of a call without the give-up.
#pragma once

#include "dkv_common.h"
#include "dkv_score_dev.h"
#include "dkv_select_dev.h"

namespace dkv {

constexpr uint32_t kTailPoison = 0x80000000u;
constexpr int kTailGo = 0, kTailLeave = 1, kTailAlone = 2;
constexpr int kEmitPer = 4;          // consecutive keys per thread in one emit round
constexpr int kFuseCandCap = 2048;   // candidates resolved from LDS (more: the row is swept instead)
constexpr int kPre = 8;              // 16-byte units of K and of V per thread loaded ahead of barrier B

// LDS words of the tail, starting where pass 2's pooling histogram starts.
__host__ __device__ constexpr int tail_u_words(int nt) {
  return (kBndLds > 2 * kFuseCandCap ? kBndLds : 2 * kFuseCandCap) > 2 * nt * kEmitPer
             ? (kBndLds > 2 * kFuseCandCap ? kBndLds : 2 * kFuseCandCap)
             : 2 * nt * kEmitPer;
}
__host__ __device__ constexpr int tail_lds_words(int nt, int kps) {
  return kBins1 + 128 + 3 * ((kps + 3) & ~3) + tail_u_words(nt) + kBins2 + kBins3 + 3 * kFuseMaxSplits;
}

// max of x[u0 .. u1] (u0 <= u1) from LDS, with eight loads in flight at a
// time (indices past u1 repeat x[u1]).
__device__ __forceinline__ float lds_window_max(const float* x, int u0, int u1) {
  float m = -INFINITY;
#pragma unroll 2
  for (int u = u0; u <= u1; u += 8) {
    float a[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = x[min(u + e, u1)];
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, a[e]);
  }
  return m;
}

// Device-coherent loads (sc1: coherent across the XCDs' L2s, the form an
// agent-scope atomic load takes): what other workgroups published with st_dev
// is read with these after a barrier, so no acquire fence (which would
// invalidate the XCD's whole L2) is needed on the hot path.
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint2 ld_dev(const uint2* p) {
  const uint64_t v = ld_dev(reinterpret_cast<const uint64_t*>(p));
  return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}
constexpr int kCpolSc1 = 16;  // buffer-load cache policy: sc1
__device__ __forceinline__ u32x4 ld_dev16(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, kCpolSc1));
}

// Thread 0 at barrier A: the arrival, then the wait (see the file comment).
__device__ __forceinline__ int tail_barrier_a(uint32_t* c, int S, int spin) {
  const uint32_t old = atomicAdd(c, 1u);
  if ((old & ~kTailPoison) == (uint32_t)S - 1u) return (old & kTailPoison) ? kTailAlone : kTailGo;
  if (old & kTailPoison) return kTailLeave;
  for (int n = 0;; ++n) {
    const uint32_t v = ld_dev(c);
    if (v & kTailPoison) return kTailLeave;
    if (v == (uint32_t)S) return kTailGo;
    if (n >= spin) {
      uint32_t expect = v;
      if (__hip_atomic_compare_exchange_strong(c, &expect, v | kTailPoison, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        return kTailLeave;
      continue;  // the counter moved: look again
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Exclusive prefix sums of a and b over the threads of the block with their
// totals, and the totals of c and d, in one pass (two barriers).  wsum: 4*NT/64
// words of LDS.
template <int NT>
__device__ __forceinline__ void block_scan2_sum2(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t* pa,
                                                 uint32_t* pb, uint32_t* ta, uint32_t* tb, uint32_t* tc,
                                                 uint32_t* td, uint32_t* wsum) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t xa = wave_incl_scan(a), xb = wave_incl_scan(b);
  const uint32_t sc = wave_reduce_add(c), sd = wave_reduce_add(d);
  __syncthreads();
  if (lane == 63) {
    wsum[w] = xa;
    wsum[NW + w] = xb;
  }
  if (lane == 0) {
    wsum[2 * NW + w] = sc;
    wsum[3 * NW + w] = sd;
  }
  __syncthreads();
  uint32_t oa = 0, ob = 0, sa = 0, sb = 0, s3 = 0, s4 = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if (i < w) {
      oa += wsum[i];
      ob += wsum[NW + i];
    }
    sa += wsum[i];
    sb += wsum[NW + i];
    s3 += wsum[2 * NW + i];
    s4 += wsum[3 * NW + i];
  }
  *pa = oa + xa - a;
  *pb = ob + xb - b;
  *ta = sa;
  *tb = sb;
  *tc = s3;
  *td = s4;
}

// Copies nk kept rows (source row s_src[i] to output row s_dst[i]) of one
// (batch, head) row with 16-byte units spread over the block.  The outputs
// here and in fused_tail are written with non-temporal stores: they stream
// to memory instead of waiting, dirty in the L2, for the write-back at the
// end of the kernel.
template <int NT>
__device__ __forceinline__ void tail_gather(const CompactArgs& ca, int row, int nk, const int* s_src,
                                            const int* s_dst) {
  const int b = row / ca.H, hh = row % ca.H;
  const int total = nk * ca.units;
  const uint8_t* kb = ca.k + b * ca.sb + hh * ca.sh;
  const uint8_t* vb = ca.v + b * ca.sb + hh * ca.sh;
  constexpr int kG = 4;  // 16-byte units of K and of V in flight per thread
  for (int t0 = threadIdx.x; t0 < total; t0 += kG * NT) {
    u32x4 kv[kG], vv[kG];
#pragma unroll
    for (int q = 0; q < kG; ++q) {
      const int t = t0 + q * NT;
      if (t < total) {
        const int64_t o = (int64_t)s_src[t / ca.units] * ca.sl + 16 * (t % ca.units);
        kv[q] = *reinterpret_cast<const u32x4*>(kb + o);
        vv[q] = *reinterpret_cast<const u32x4*>(vb + o);
      }
    }
#pragma unroll
    for (int q = 0; q < kG; ++q) {
      const int t = t0 + q * NT;
      if (t < total) {
        const int64_t o = ((int64_t)row * ca.out_ld + s_dst[t / ca.units]) * ca.units * 16 + 16 * (t % ca.units);
        __builtin_nontemporal_store(kv[q], reinterpret_cast<u32x4*>(ca.ko + o));
        __builtin_nontemporal_store(vv[q], reinterpret_cast<u32x4*>(ca.vo + o));
      }
    }
  }
}

// Digits 2 and 3 over the candidates (keys whose top digit is b1, visited by
// for_cands), given the rank k1 of the keep-th key among them: the threshold
// key T and how many keys equal to T are kept.  hist2 / hist3 zeroed and
// visible on entry; fb: 8 words of LDS.
template <typename ForCands>
__device__ __forceinline__ void tail_digits(ForCands&& for_cands, uint32_t b1, uint32_t k1, uint32_t* hist2,
                                            uint32_t* hist3, uint32_t* fb, uint32_t* T, uint32_t* take_eq) {
  for_cands([&](uint32_t key, int) { atomicAdd(&hist2[(key >> kShift2) & (kBins2 - 1)], 1u); });
  __syncthreads();
  if (threadIdx.x < 64) wave_find_bin<kBins2>(hist2, nullptr, k1, fb);
  __syncthreads();
  const uint32_t b2 = fb[0];
  const uint32_t k2 = k1 - fb[1];
  const uint32_t pre = (b1 << kBits2) | b2;
  const uint32_t m = hist2[b2];  // candidates left in the two top digits
  if (m <= 64u) {
    // Few: rank them directly (one wave, one key per lane) against each
    // other; the k2-th largest is T.  hist3 serves as their list.
    if (threadIdx.x == 0) fb[7] = 0u;
    __syncthreads();
    for_cands([&](uint32_t key, int) {
      if ((key >> kShift2) == pre) hist3[atomicAdd(&fb[7], 1u)] = key;
    });
    __syncthreads();
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      const uint32_t mine = (uint32_t)l < m ? hist3[l] : 0u;
      uint32_t g = 0u, e = 0u;
      for (uint32_t i = 0; i < m; ++i) {
        const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)mine, (int)i);  // lane i's key
        g += o > mine ? 1u : 0u;
        e += o == mine ? 1u : 0u;
      }
      if ((uint32_t)l < m && g < k2 && k2 <= g + e) {
        fb[4] = mine;
        fb[5] = k2 - g;
      }
    }
    __syncthreads();
    *T = fb[4];
    *take_eq = fb[5];
    return;
  }
  for_cands([&](uint32_t key, int) {
    if ((key >> kShift2) == pre) atomicAdd(&hist3[key & (kBins3 - 1)], 1u);
  });
  __syncthreads();
  if (threadIdx.x < 64) wave_find_bin<kBins3>(hist3, nullptr, k2, fb + 4);
  __syncthreads();
  *T = (pre << kBits3) | fb[4];
  *take_eq = k2 - fb[5];
}

// Emits the kept keys of [j0, j1) of a row in index order, given the kept
// keys above T (gt0) and the keys equal to T (eq0) before j0, and gathers
// their K/V rows.  pooled_of(j) gives key j's pooled value (unprotected).
// Rounds of NT * kEmitPer keys; s_src / s_dst: NT * kEmitPer ints each.
template <int NT, typename PooledOf>
__device__ __forceinline__ void tail_emit(const SelFuse& fz, int row, int j0, int j1, uint32_t gt0, uint32_t eq0,
                                          uint32_t T, uint32_t take_eq, uint32_t kbig, int prot,
                                          PooledOf&& pooled_of, int* s_src, int* s_dst, uint32_t* wsum) {
  const uint32_t keep = (uint32_t)fz.keep;
  for (int r0 = j0; r0 < j1; r0 += NT * kEmitPer) {
    const int jt = r0 + kEmitPer * (int)threadIdx.x;
    uint32_t keys[kEmitPer];
    uint32_t ng = 0u, ne = 0u;
#pragma unroll
    for (int i = 0; i < kEmitPer; ++i) {
      const int j = jt + i;
      keys[i] = 0u;
      if (j < j1) {
        keys[i] = j >= prot ? kbig : float_key(pooled_of(j));
        ng += keys[i] > T ? 1u : 0u;
        ne += keys[i] == T ? 1u : 0u;
      }
    }
    uint32_t pg, pe, tg, te;
    block_excl_scan2<NT>(ng, ne, &pg, &pe, &tg, &te, wsum);
    const uint32_t start = gt0 + min(eq0, take_eq);  // first output slot of this round
    uint32_t g_before = gt0 + pg, e_before = eq0 + pe;
#pragma unroll
    for (int i = 0; i < kEmitPer; ++i) {
      const int j = jt + i;
      if (j < j1) {
        const bool gt = keys[i] > T, eq = keys[i] == T;
        if (gt || (eq && e_before < take_eq)) {
          const uint32_t pos = g_before + min(e_before, take_eq);
          if (pos < keep) {
            fz.out_idx[(int64_t)row * keep + pos] = j;
            s_src[pos - start] = j;
            s_dst[pos - start] = (int)pos;
          }
        }
        g_before += gt ? 1u : 0u;
        e_before += eq ? 1u : 0u;
      }
    }
    __syncthreads();
    const uint32_t last = min(gt0 + tg + min(eq0 + te, take_eq), keep);
    const int nk = last > start ? (int)(last - start) : 0;
    tail_gather<NT>(fz.ca, row, nk, s_src, s_dst);
    gt0 += tg;
    eq0 += te;
    __syncthreads();  // s_src / s_dst are rewritten by the next round
  }
}

// The whole selection of one row by the pass-2 workgroup of split `split`
// (keys [split*kps, min((split+1)*kps, Lk))) once its scores are in LDS (sc).
// L: tail_lds_words(NT, kps) words of LDS (pass 2's operands are dead).
// Global loads that one phase needs are issued together, so each phase
// costs one round trip to memory.
template <int NT>
__device__ void fused_tail(const SelFuse& fz, const float* __restrict__ sc, uint32_t* L, int row, int split, int S,
                           int kps, int Lk) {
  static_assert(NT * 4 == kBins1, "one 16-byte histogram load per thread");
  static_assert(NT >= kFuseMaxSplits, "one split header per thread");
  constexpr int kEdge4 = kBndLds / 4 / NT;                   // 16-byte edge loads per thread
  constexpr int kPeekPer = kPeekTotal / NT;  // peeked candidates per thread
  const int tid = threadIdx.x;
  const int k_begin = split * kps, k_end = min(k_begin + kps, Lk);
  const int h = fz.ks / 2, w2 = 2 * h, w4 = 4 * h;
  const int prot = Lk - fz.window;
  const int nb = S - 1;
  uint32_t* rw = fz.ws.rowws + (int64_t)row * kRowWords;
  float* prow = fz.ws.pooled + (int64_t)row * Lk;
  float* edge = fz.ws.edge + (int64_t)row * kBndLds;
  uint2* hdr = fz.ws.shdr + (int64_t)row * kFuseMaxSplits;
  uint2* cregion = fz.ws.scand + (int64_t)row * (Lk + kScandPad);
  uint32_t* hist1 = L;
  uint32_t* small = hist1 + kBins1;  // [0, 16) block scans, [64, 72) bin searches, [96, 112) max, 120 state
  float* pl = reinterpret_cast<float*>(small + 128);
  uint32_t* U = small + 128 + ((kps + 3) & ~3);  // boundary raw scores, then candidates, then emit slots
  uint32_t* hist2 = U + tail_u_words(NT);
  uint32_t* hist3 = hist2 + kBins2;
  uint32_t* abv = hist3 + kBins3;     // per split: keys above b1
  uint32_t* ncs = abv + kFuseMaxSplits;  // per split: candidates
  uint32_t* soff = ncs + kFuseMaxSplits; // per split: first slot of its candidates in the list
  int* s_pot = reinterpret_cast<int*>(soff + kFuseMaxSplits);  // this split's keys at or above b1
  int* pos_of = s_pot + ((kps + 3) & ~3);                        // output row of each key of the split, or -1

  // 0. Boundary raw scores out; the interior pooled into LDS, the pooled row,
  // the row histogram and maximum.  Boundary i (between splits i and i+1)
  // keeps raw scores [(i+1)*kps - 2h, (i+1)*kps + 2h) (past Lk: -inf).
  for (int i = tid; i < kBins1; i += NT) hist1[i] = 0u;
  if (tid == 0) small[127] = 0u;
  if (split > 0)
    for (int t = tid; t < w2; t += NT) {
      const int u = k_begin + t;
      st_dev(edge + (split - 1) * w4 + w2 + t, u < k_end ? sc[u - k_begin] : -INFINITY);
    }
  if (split < nb)
    for (int t = tid; t < w2; t += NT) st_dev(edge + split * w4 + t, sc[k_end - w2 + t - k_begin]);
  __syncthreads();
  const int i0 = split == 0 ? 0 : k_begin + h;
  const int i1 = k_end >= Lk ? Lk : k_end - h;
  uint32_t kmax = 0u;
  // Keys j, j+1 per thread: their windows share [j-h+1, j+h].
  for (int j = i0 + 2 * tid; j < i1; j += 2 * NT) {
    const int mlo = max(j - h + 1, 0), mhi = min(j + h, Lk - 1);
    const float mid = mlo <= mhi ? lds_window_max(sc, mlo - k_begin, mhi - k_begin) : -INFINITY;
    const float m0 = fmaxf(mid, j - h >= 0 ? sc[j - h - k_begin] : -INFINITY);
    const bool two = j + 1 < i1;
    const float m1 = two ? fmaxf(mid, j + h + 1 <= Lk - 1 ? sc[j + h + 1 - k_begin] : -INFINITY) : -INFINITY;
    pl[j - k_begin] = m0;
    st_dev(reinterpret_cast<uint32_t*>(prow + j), __float_as_uint(m0));
    const uint32_t key0 = float_key(m0);
    kmax = max(kmax, key0);
    if (j < prot) atomicAdd(&hist1[key0 >> kShift1], 1u);
    if (two) {
      pl[j + 1 - k_begin] = m1;
      st_dev(reinterpret_cast<uint32_t*>(prow + j + 1), __float_as_uint(m1));
      const uint32_t key1 = float_key(m1);
      kmax = max(kmax, key1);
      if (j + 1 < prot) atomicAdd(&hist1[key1 >> kShift1], 1u);
    }
  }
  kmax = wave_reduce_max(kmax);
  if ((tid & 63) == 0 && kmax) atomicMax(&small[127], kmax);
  __syncthreads();  // every wave's histogram adds and maximum are in
  if (tid == 0 && small[127]) atomicMax(rw + kRowMax, small[127]);
  for (int i = tid; i < kBins1; i += NT)
    if (hist1[i]) atomicAdd(rw + kRowHist1 + i, hist1[i]);

  // A.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) small[120] = (uint32_t)tail_barrier_a(rw + kRowBarA, S, fz.spin);
  __syncthreads();
  const int state = (int)small[120];
  if (state == kTailLeave) return;
  const bool alone = state == kTailAlone;

  // 1. One round trip: the row's histogram, maximum and boundary raw scores.
  {
    const rsrc_t hrs = make_rsrc(rw + kRowHist1, kBins1 * 4u);
    const rsrc_t ers = make_rsrc(edge, kBndLds * 4u);
    const u32x4 hv = ld_dev16(hrs, (uint32_t)tid * 16u);
    const uint32_t rm = ld_dev(rw + kRowMax);
    const int n4 = (nb * w4 + 3) / 4;
    u32x4 ev[kEdge4];
#pragma unroll
    for (int k = 0; k < kEdge4; ++k)
      if (tid + k * NT < n4) ev[k] = ld_dev16(ers, (uint32_t)(tid + k * NT) * 16u);
    reinterpret_cast<u32x4*>(hist1)[tid] = hv;
#pragma unroll
    for (int k = 0; k < kEdge4; ++k)
      if (tid + k * NT < n4) reinterpret_cast<u32x4*>(U)[tid + k * NT] = ev[k];
    if (tid == 0) {
      small[121] = rm;   // row maximum, then with the boundary keys
      small[124] = 0u;   // slots taken in the candidate regions / in s_pot
      small[125] = 0u;
    }
  }
  __syncthreads();
  const uint32_t rmax = small[121];
  const float* ex = reinterpret_cast<const float*>(U);
  uint32_t bmax = 0u;
  for (int t = tid; t < nb * w2; t += NT) {
    const int bi = t / w2, k = t % w2;
    const int j = (bi + 1) * kps - h + k;
    if (j < Lk) {
      const float m = lds_window_max(ex, bi * w4 + k, bi * w4 + k + w2);  // raw scores [j - h, j + h]
      const uint32_t key = float_key(m);
      bmax = max(bmax, key);
      if (j < prot) atomicAdd(&hist1[key >> kShift1], 1u);
      const bool own = j >= k_begin && j < k_end;
      if (own) pl[j - k_begin] = m;
      // the pooled row is read back by sweeps (many candidates, or alone)
      if (own || alone) st_dev(reinterpret_cast<uint32_t*>(prow + j), __float_as_uint(m));
    }
  }
  bmax = wave_reduce_max(bmax);
  if ((tid & 63) == 0 && bmax > rmax) atomicMax(&small[121], bmax);
  __syncthreads();
  const uint32_t gmax = small[121];
  const uint32_t kbig = float_key(key_float(gmax) + 1.0f);
  if (tid < 64) {
    // (one wave: its own LDS operations stay in order)
    if (tid == 0) hist1[kbig >> kShift1] += (uint32_t)fz.window;
    wave_find_bin<kBins1>(hist1, nullptr, (uint32_t)fz.keep, small + 64);
  }
  __syncthreads();
  const uint32_t b1 = small[64];
  const uint32_t k1 = (uint32_t)fz.keep - small[65];
  int* s_src = reinterpret_cast<int*>(U);
  int* s_dst = s_src + NT * kEmitPer;
  for (int i = tid; i < kBins2; i += NT) hist2[i] = 0u;
  for (int i = tid; i < kBins3; i += NT) hist3[i] = 0u;
  const rsrc_t prs = make_rsrc(prow, (uint32_t)Lk * 4u);
  // Every key of the row inside b1, from the pooled row in memory.
  auto sweep = [&](auto&& f) __attribute__((always_inline)) {
    for (int j0 = 4 * tid; j0 < Lk; j0 += 4 * NT) {
      const u32x4 xv = buf_load16(prs, (uint32_t)j0 * 4u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = j0 + e;
        const uint32_t key = pooled_key(xv[e], j, prot, kbig);
        if (j < Lk && (key >> kShift1) == b1) f(key, j);
      }
    }
  };

  // Every key of the row from the pooled row in memory: digits 2 and 3, then
  // the ordered emit and gather of the whole row.  The caller made the
  // pooled row complete and visible to this workgroup's loads.
  auto finish_alone = [&]() __attribute__((always_inline)) {
    uint32_t T, take_eq;
    tail_digits(sweep, b1, k1, hist2, hist3, small + 64, &T, &take_eq);
    tail_emit<NT>(fz, row, 0, Lk, 0u, 0u, T, take_eq, kbig, prot, [&](int j) { return prow[j]; }, s_src, s_dst,
                  small);
  };

  if (alone) {
    // The others left: finish the row from the pooled row in memory (every
    // interior came in before barrier A; this workgroup wrote the boundary
    // keys above and makes them visible to its own loads first).
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __syncthreads();
    finish_alone();
    return;
  }

  // 2. This split's keys above b1 (a count) and inside b1 (the candidates,
  // into the split's own region of the list: no atomics), then its header.
  // Every key at or above b1 may be kept: their list (s_pot) lets the
  // gather's loads start before barrier B.
  uint32_t na = 0u, nc = 0u;
  for (int j = k_begin + tid; j < k_end; j += NT) {
    const uint32_t d = (j >= prot ? kbig : float_key(pl[j - k_begin])) >> kShift1;
    na += d > b1 ? 1u : 0u;
    nc += d == b1 ? 1u : 0u;
  }
  // Slots: a wave-wide prefix, then one LDS atomic per wave.
  uint32_t pc, pp;
  {
    const uint32_t ic = wave_incl_scan(nc), ip = wave_incl_scan(na + nc);
    const uint32_t tc = (uint32_t)__builtin_amdgcn_readlane((int)ic, 63);
    const uint32_t tp = (uint32_t)__builtin_amdgcn_readlane((int)ip, 63);
    uint32_t bc = 0u, bp = 0u;
    if ((tid & 63) == 0) {
      if (tc) bc = atomicAdd(&small[124], tc);
      if (tp) bp = atomicAdd(&small[125], tp);
    }
    pc = (uint32_t)__builtin_amdgcn_readfirstlane((int)bc) + ic - nc;
    pp = (uint32_t)__builtin_amdgcn_readfirstlane((int)bp) + ip - (na + nc);
  }
  if (na + nc) {
    for (int j = k_begin + tid; j < k_end; j += NT) {
      const uint32_t key = j >= prot ? kbig : float_key(pl[j - k_begin]);
      const uint32_t d = key >> kShift1;
      if (d >= b1) s_pot[pp++] = j;
      if (d == b1) {
        st_dev(reinterpret_cast<uint64_t*>(cregion + k_begin + pc), (uint64_t)key | ((uint64_t)(uint32_t)j << 32));
        ++pc;
      }
    }
  }

  // B.  The K/V rows of the first keys of s_pot are loaded into registers
  // right after the arrival (workgroup barriers do not wait for them).
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const uint32_t nc_all = small[124], np_all = small[125];
  if (tid == 0) {
    st_dev(reinterpret_cast<uint64_t*>(hdr + split), (uint64_t)(np_all - nc_all) | ((uint64_t)nc_all << 32));
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    atomicAdd(rw + kRowBarB, 1u);
  }
  const CompactArgs& ca = fz.ca;
  const int units = ca.units;
  const int pre_rows = min((int)np_all, kPre * NT / units);
  const int bb = row / ca.H, hh = row % ca.H;
  const uint8_t* kbase = ca.k + bb * ca.sb + hh * ca.sh;
  const uint8_t* vbase = ca.v + bb * ca.sb + hh * ca.sh;
  u32x4 kpre[kPre], vpre[kPre];
#pragma unroll
  for (int q = 0; q < kPre; ++q) {
    const int u = tid + q * NT;
    if (u < pre_rows * units) {
      const int64_t o = (int64_t)s_pot[u / units] * ca.sl + 16 * (u % units);
      kpre[q] = *reinterpret_cast<const u32x4*>(kbase + o);
      vpre[q] = *reinterpret_cast<const u32x4*>(vbase + o);
    }
  }
  if (tid == 0) {
    bool ok = true;
    for (int n = 0; ld_dev(rw + kRowBarB) < (uint32_t)S; ++n) {
      if (n >= fz.spin_b) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    small[120] = ok ? 1u : 0u;
    small[122] = 0u;  // set below when a split has more candidates than were peeked
  }
  __syncthreads();
  if (!small[120]) {
    // Gave up at B: the boundary keys of every split (their raw scores are
    // still in U) into the pooled row, then the whole row alone.
    for (int t = tid; t < nb * w2; t += NT) {
      const int bi = t / w2, k = t % w2;
      const int j = (bi + 1) * kps - h + k;
      if (j < Lk)
        st_dev(reinterpret_cast<uint32_t*>(prow + j), __float_as_uint(lds_window_max(ex, bi * w4 + k, bi * w4 + k + w2)));
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __syncthreads();
    finish_alone();
    return;
  }

  // 3. One round trip: every split's header and its first `peek`
  // candidates (read blindly; kPeekTotal entries in all, the region is
  // padded for the last split).
  const int lpeek = 31 - __clz(min(kps, kPeekTotal / S));  // peek: a power of two
  const int peek = 1 << lpeek;
  constexpr int kHdrPer = kFuseMaxSplits / 64;  // split headers per lane of wave 0
  uint2 hv[kHdrPer];
  if (tid < 64) {
#pragma unroll
    for (int q = 0; q < kHdrPer; ++q) {
      const int sp = kHdrPer * tid + q;
      hv[q] = sp < S ? ld_dev(hdr + sp) : make_uint2(0u, 0u);
    }
  }
  uint2 pk[kPeekPer];
  const int npk = S * peek;
#pragma unroll
  for (int k = 0; k < kPeekPer; ++k) {
    const int e = tid + k * NT;
    if (e < npk) pk[k] = ld_dev(cregion + (e >> lpeek) * kps + (e & (peek - 1)));
  }
  if (tid < 64) {
    // Split counts -> first slots, by one wave (splits kHdrPer*lane ..).
    uint32_t n = 0u;
    bool over = false;
#pragma unroll
    for (int q = 0; q < kHdrPer; ++q) {
      n += hv[q].y;
      over |= hv[q].y > (uint32_t)peek;
    }
    const uint32_t inc = wave_incl_scan(n);
    uint32_t run = inc - n;
#pragma unroll
    for (int q = 0; q < kHdrPer; ++q) {
      const int sp = kHdrPer * tid + q;
      if (sp < S) {
        abv[sp] = hv[q].x;
        ncs[sp] = hv[q].y;
        soff[sp] = run;
      }
      run += hv[q].y;
    }
    if (tid == 63) small[126] = inc;
    if (__ballot(over)) small[122] = 1u;
  }
  __syncthreads();
  const uint32_t ncand = small[126];
  const bool in_lds = ncand <= (uint32_t)kFuseCandCap;
  uint2* cl = reinterpret_cast<uint2*>(U);  // the boundary raw scores are dead
  if (in_lds) {
    uint32_t pn[kPeekPer], po[kPeekPer];
#pragma unroll
    for (int k = 0; k < kPeekPer; ++k) {
      const int sp = min((tid + k * NT) >> lpeek, S - 1);
      pn[k] = ncs[sp];
      po[k] = soff[sp];
    }
#pragma unroll
    for (int k = 0; k < kPeekPer; ++k) {
      const int e = tid + k * NT;
      const uint32_t i = (uint32_t)(e & (peek - 1));
      if (e < npk && i < pn[k]) cl[po[k] + i] = pk[k];
    }
    // Splits with more candidates than were peeked: the rest (a second round trip).
    if (small[122])
      for (int sp = 0; sp < S; ++sp)
        for (uint32_t i = peek + tid; i < ncs[sp]; i += NT) cl[soff[sp] + i] = ld_dev(cregion + sp * kps + i);
  } else {
    // The row is swept from the pooled row in memory instead (plain loads):
    // acquire first.
    if (tid == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  auto for_cands = [&](auto&& f) __attribute__((always_inline)) {
    if (in_lds) {
      for (uint32_t p = tid; p < ncand; p += NT) {
        const uint2 cv = cl[p];
        f(cv.x, (int)cv.y);
      }
    } else {
      sweep(f);
    }
  };
  uint32_t T, take_eq;
  tail_digits(for_cands, b1, k1, hist2, hist3, small + 64, &T, &take_eq);
  // Kept keys above T and keys equal to T before this split: its
  // predecessors' keys above b1 and their candidates above / at T.
  uint32_t cgt = 0u, ceq = 0u;
  for_cands([&](uint32_t key, int j) {
    if (j < k_begin) {
      cgt += key > T ? 1u : 0u;
      ceq += key == T ? 1u : 0u;
    }
  });
  for (int sp = tid; sp < split; sp += NT) cgt += abv[sp];
  // (their block totals come out of the first emit round's scan)
  uint32_t gt0 = 0u, eq0 = 0u;
  // Output rows of this split's keys (pos_of), then the prefetched rows
  // stored where they go and the rest of the kept rows copied.
  const uint32_t keep = (uint32_t)fz.keep;
  for (int r0 = k_begin; r0 < k_end; r0 += NT * kEmitPer) {
    const int jt = r0 + kEmitPer * tid;
    uint32_t keys[kEmitPer];
    uint32_t ng = 0u, ne = 0u;
#pragma unroll
    for (int i = 0; i < kEmitPer; ++i) {
      const int j = jt + i;
      keys[i] = 0u;
      if (j < k_end) {
        keys[i] = j >= prot ? kbig : float_key(pl[j - k_begin]);
        ng += keys[i] > T ? 1u : 0u;
        ne += keys[i] == T ? 1u : 0u;
      }
    }
    uint32_t pg, pe, tg, te;
    if (r0 == k_begin)
      block_scan2_sum2<NT>(ng, ne, cgt, ceq, &pg, &pe, &tg, &te, &gt0, &eq0, small);
    else
      block_excl_scan2<NT>(ng, ne, &pg, &pe, &tg, &te, small);
    uint32_t g_before = gt0 + pg, e_before = eq0 + pe;
#pragma unroll
    for (int i = 0; i < kEmitPer; ++i) {
      const int j = jt + i;
      if (j < k_end) {
        const bool gt = keys[i] > T, eq = keys[i] == T;
        int pos = -1;
        if (gt || (eq && e_before < take_eq)) {
          const uint32_t p = g_before + min(e_before, take_eq);
          if (p < keep) {
            __builtin_nontemporal_store((int64_t)j, &fz.out_idx[(int64_t)row * keep + p]);
            pos = (int)p;
          }
        }
        pos_of[j - k_begin] = pos;
        g_before += gt ? 1u : 0u;
        e_before += eq ? 1u : 0u;
      }
    }
    gt0 += tg;
    eq0 += te;
  }
  __syncthreads();
  const int64_t orow = (int64_t)row * ca.out_ld;
#pragma unroll
  for (int q = 0; q < kPre; ++q) {
    const int u = tid + q * NT;
    if (u < pre_rows * units) {
      const int p = pos_of[s_pot[u / units] - k_begin];
      if (p >= 0) {
        const int64_t o = (orow + p) * units * 16 + 16 * (u % units);
        __builtin_nontemporal_store(kpre[q], reinterpret_cast<u32x4*>(ca.ko + o));
        __builtin_nontemporal_store(vpre[q], reinterpret_cast<u32x4*>(ca.vo + o));
      }
    }
  }
  for (int u = pre_rows * units + tid; u < (int)np_all * units; u += NT) {
    const int j = s_pot[u / units];
    const int p = pos_of[j - k_begin];
    if (p >= 0) {
      const int64_t os = (int64_t)j * ca.sl + 16 * (u % units);
      const int64_t o = (orow + p) * units * 16 + 16 * (u % units);
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(kbase + os), reinterpret_cast<u32x4*>(ca.ko + o));
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(vbase + os), reinterpret_cast<u32x4*>(ca.vo + o));
    }
  }
}

}  // namespace dkv
