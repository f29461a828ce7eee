// Device-side pieces of the selection (pool / protect / top-k threshold /
// ordered emit) shared by the selection kernels (dkv_select.hip) and the
// pooling epilogue of the scoring pass (dkv_score.hip).
//
// Reference semantics (dropkv_cache.py:464-475):
//   pooled[j] = max(scores[j-h .. j+h]), h = kernel_size/2, out of range = -inf
//   big = max_j pooled[j] + 1.0f ; pooled[Lk-window ..] = big
//   keep the `keep` largest pooled values; among values equal to the
//   threshold the lowest indices win (torch.topk leaves that order open).
//
// Floats are mapped to order-preserving uint32 keys and the keep-th largest
// key T is found by a radix select over 11 + 11 + 10 bits:
//   pool    (pass-2 epilogue, or the standalone pool kernel) pooled values of
//           the keys whose window lies inside one workgroup's range, the row
//           maximum and the top-digit histogram (device atomics);
//   resolve (up to 8 workgroups per row, each sweeping a part of it) pools
//           the few keys next to the scoring pass's split boundaries, which
//           completes the histogram and fixes the top-digit bin b1; sweeps
//           its part for the keys above b1 per chunk and the keys inside b1
//           (the candidates, a few percent of the row, appended to a list in
//           the workspace); the row's last part to finish resolves digits 2
//           and 3 from the candidates and writes per 1024-key chunk the kept
//           keys above T and the keys equal to T before it;
//   emit    (row, chunk) workgroups write the chunk's kept indices in index
//           order from those offsets and copy the K/V rows they name.
#pragma once

#include "dkv_common.h"

namespace dkv {

constexpr int kChunk = 1024;      // keys per emit workgroup (offset granularity)
constexpr int kBits1 = 11, kBits2 = 11, kBits3 = 10;  // radix digits, most significant first
constexpr int kShift1 = 32 - kBits1;                // digit 1 = key >> kShift1
constexpr int kShift2 = kBits3;                     // digit 2 = (key >> kShift2) & (kBins2 - 1)
constexpr int kBins1 = 1 << kBits1;                 // key bits 31..21
constexpr int kBins2 = 1 << kBits2;                 // key bits 20..10
constexpr int kBins3 = 1 << kBits3;                 // key bits 9..0
constexpr int kMaxHalo = 64;      // kernel_size <= 2*kMaxHalo+1
constexpr int kMaxChunks = 4096;  // Lk <= kMaxChunks * kChunk
constexpr int kBndLds = 4096;     // LDS words for the boundary keys' raw-score neighbourhoods
constexpr int kBndPoolLds = 2048; // LDS words for the boundary keys' pooled values

// Per-row words that must be zero on entry (the merge kernel or the zero
// kernel clears them every call), then results of the resolve stage:
constexpr int kRowMax = 0;                 // max pooled key of the interiors
constexpr int kRowB1 = 1;                  // T, keys equal to T that are kept, max key of the row (resolve)
constexpr int kRowArrive = 4;              // resolve parts of the row that have swept their chunks
constexpr int kRowNcand = 5;               // candidates the parts have found (may exceed kResCandCap)
constexpr int kRowBarA = 8;                // selection in the scoring tail: arrivals at barrier A (| poison bit)
constexpr int kRowBarB = 9;                //   arrivals at barrier B
constexpr int kRowHist1 = 16;              // top-digit histogram (unprotected interior keys), 16-byte aligned
constexpr int kRowWords = kRowHist1 + kBins1;
constexpr int kResCandCap = 4096;          // candidates (key, index) kept per row, in the workspace and in LDS
constexpr int kFuseMaxSplits = 256;        // scoring splits per row the selection tail takes
constexpr int kPeekTotal = 4096;           // candidates of a row the tail reads without knowing the counts
constexpr int kScandPad = 4096;            // entries past Lk in a row's candidate regions (the last split's peek)

struct SelWs {
  uint32_t* rowws;     // [rows][kRowWords]
  float* pooled;       // [rows][Lk]
  uint2* cnt;          // [rows][chunks] {kept keys above T, keys equal to T} in the chunks before each
  uint2* cand;         // [rows][kResCandCap] the resolve parts' candidates (key, index)
  // The selection in the scoring tail (dkv_tail_dev.h):
  float* edge;         // [rows][kBndLds] raw scores around each split boundary
  uint2* shdr;         // [rows][kFuseMaxSplits] per split {keys above the top-digit bin, candidates}
  uint2* scand;        // [rows][Lk + kScandPad] per split's key range: its candidates (key, index)
};

inline size_t sel_al256(size_t b) { return (b + 255) & ~size_t(255); }

inline SelWs sel_layout(char* base, int64_t rows, int64_t Lk, size_t* total) {
  const int64_t chunks = (Lk + kChunk - 1) / kChunk;
  SelWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += sel_al256(bytes);
    return p;
  };
  w.rowws = reinterpret_cast<uint32_t*>(take((size_t)rows * kRowWords * 4));
  w.pooled = reinterpret_cast<float*>(take((size_t)rows * Lk * 4));
  w.cnt = reinterpret_cast<uint2*>(take((size_t)rows * chunks * 8));
  w.cand = reinterpret_cast<uint2*>(take((size_t)rows * kResCandCap * 8));
  w.edge = reinterpret_cast<float*>(take((size_t)rows * kBndLds * 4));
  w.shdr = reinterpret_cast<uint2*>(take((size_t)rows * kFuseMaxSplits * 8));
  w.scand = reinterpret_cast<uint2*>(take((size_t)rows * (Lk + kScandPad) * 8));
  if (total) *total = off;
  return w;
}

// Sort key of a pooled value given as its bits (the buffer load's integer
// lanes), with the protected tail mapped to kbig.
__device__ __forceinline__ uint32_t pooled_key(uint32_t bits, int j, int prot, uint32_t kbig) {
  if (bits == 0x80000000u) bits = 0u;
  const uint32_t k = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return j >= prot ? kbig : k;
}

// The K/V gather of the emit stage: kept rows of the [B, H, L, D] sources go
// to rows of [B, H, out_ld, D] outputs, in 16-byte units.
struct CompactArgs {
  const uint8_t* k;
  const uint8_t* v;
  int64_t sb, sh, sl;  // source byte strides
  int H;
  int units;           // 16-byte units per row
  uint8_t* ko;
  uint8_t* vo;
  int64_t out_ld;      // rows per head in ko / vo
};

// Split geometry of the pooling stage: keys within h of j = i*kps
// (1 <= i < n_splits) were not pooled by it (their window straddles two
// workgroup ranges).  n_splits = 1 means every key was pooled.
struct SplitGeom {
  int n_splits, kps;
};

// Whether the resolve stage can hold the boundary keys of this geometry in LDS.
__host__ __device__ constexpr bool boundary_fits(int64_t n_splits, int64_t h) {
  return (n_splits - 1) * 4 * h <= kBndLds && (n_splits - 1) * 2 * h <= kBndPoolLds;
}

// ---------------------------------------------------------------------------
// Wave-level scans and reductions on DPP (a few cycles per step, against an
// LDS round trip per step for lane shuffles).
// ---------------------------------------------------------------------------
// DPP move of x with zeros where the source lane is out of the row or the
// destination lane is masked off (row_mask / bank_mask).
template <int kCtrl, int kRowMask, int kBankMask>
__device__ __forceinline__ uint32_t dpp_z(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kCtrl, kRowMask, kBankMask, true);
}
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr3 = 0x113, kDppRowShr4 = 0x114,
              kDppRowShr8 = 0x118, kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

// Inclusive prefix sum over the 64 lanes: within each row of 16 lanes by row
// shifts (1, 2, 3, then 4 into banks 1-3 and 8 into banks 2-3), then across
// rows by broadcasting lane 15 into rows 1 and 3 and lane 31 into rows 2-3.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  uint32_t t = x + dpp_z<kDppRowShr1, 0xf, 0xf>(x);
  t += dpp_z<kDppRowShr2, 0xf, 0xf>(x);
  t += dpp_z<kDppRowShr3, 0xf, 0xf>(x);
  t += dpp_z<kDppRowShr4, 0xf, 0xe>(t);
  t += dpp_z<kDppRowShr8, 0xf, 0xc>(t);
  t += dpp_z<kDppRowBcast15, 0xa, 0xf>(t);
  t += dpp_z<kDppRowBcast31, 0xc, 0xf>(t);
  return t;
}

// Sum and maximum over the 64 lanes (wave-uniform results).
__device__ __forceinline__ uint32_t wave_reduce_add(uint32_t x) {
  int v = (int)x;
  v += dpp_i<kDppQuadSwap1>(v);
  v += dpp_i<kDppQuadSwap2>(v);
  v += dpp_i<kDppHalfMirror>(v);
  v += dpp_i<kDppMirror>(v);
  return (uint32_t)((__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
                    (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48)));
}

__device__ __forceinline__ uint32_t wave_reduce_max(uint32_t x) {
  x = max(x, (uint32_t)dpp_i<kDppQuadSwap1>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppQuadSwap2>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppHalfMirror>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppMirror>((int)x));
  return max(max((uint32_t)__builtin_amdgcn_readlane((int)x, 0), (uint32_t)__builtin_amdgcn_readlane((int)x, 16)),
             max((uint32_t)__builtin_amdgcn_readlane((int)x, 32), (uint32_t)__builtin_amdgcn_readlane((int)x, 48)));
}

// ---------------------------------------------------------------------------
// Block-level helpers for NT threads (a multiple of 64).
// ---------------------------------------------------------------------------
// Exclusive prefix sums of two counters over the threads of the block, and
// optionally their block totals.  wsum: 2*NT/64 words of LDS.
template <int NT>
__device__ __forceinline__ void block_excl_scan2(uint32_t a, uint32_t b, uint32_t* pa, uint32_t* pb, uint32_t* ta,
                                                 uint32_t* tb, uint32_t* wsum) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t xa = wave_incl_scan(a), xb = wave_incl_scan(b);
  __syncthreads();
  if (lane == 63) {
    wsum[w] = xa;
    wsum[NW + w] = xb;
  }
  __syncthreads();
  uint32_t oa = 0, ob = 0, sa = 0, sb = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if (i < w) {
      oa += wsum[i];
      ob += wsum[NW + i];
    }
    sa += wsum[i];
    sb += wsum[NW + i];
  }
  *pa = oa + xa - a;
  *pb = ob + xb - b;
  if (ta) *ta = sa;
  if (tb) *tb = sb;
}

// Block sums of two counters (every thread gets them).  wsum: 2*NT/64 words.
template <int NT>
__device__ __forceinline__ void block_sum2(uint32_t a, uint32_t b, uint32_t* ta, uint32_t* tb, uint32_t* wsum) {
  constexpr int NW = NT / 64;
  a = wave_reduce_add(a);
  b = wave_reduce_add(b);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    wsum[threadIdx.x >> 6] = a;
    wsum[NW + (threadIdx.x >> 6)] = b;
  }
  __syncthreads();
  uint32_t sa = 0, sb = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    sa += wsum[i];
    sb += wsum[NW + i];
  }
  *ta = sa;
  *tb = sb;
}

// For a histogram of NB bins in LDS and 1 <= k <= total: the bin b with
// (count of keys in bins > b) < k <= (count in bins >= b), and the count in
// bins > b.  Results land in *s_bin / *s_above (LDS); ends with a barrier.
template <int NB, int NT>
__device__ void find_bin(const uint32_t* hist, uint32_t k, int* s_bin, uint32_t* s_above, uint32_t* wsum) {
  static_assert(NB % NT == 0, "bins must be a multiple of the block size");
  constexpr int per = NB / NT;
  const int tid = threadIdx.x;
  uint32_t loc[per];
  uint32_t tsum = 0u;
#pragma unroll
  for (int i = 0; i < per; ++i) {
    loc[i] = hist[NB - 1 - (tid * per + i)];  // thread order = descending bins
    tsum += loc[i];
  }
  uint32_t run, dummy;
  block_excl_scan2<NT>(tsum, 0u, &run, &dummy, nullptr, nullptr, wsum);
#pragma unroll
  for (int i = 0; i < per; ++i) {
    const uint32_t nxt = run + loc[i];
    if (run < k && nxt >= k) {
      *s_bin = NB - 1 - (tid * per + i);
      *s_above = run;
    }
    run = nxt;
  }
  __syncthreads();
}

// The same search done by one whole wave (no block barrier inside; the
// caller brackets it with barriers).  For a second histogram he over the same
// bins (optional), also its count in bins > b and in b.  Writes out[0..3] =
// {b, count in bins > b, he count in bins > b, he[b]}.  Lane l first sums the
// bins of its segment (NB/64 consecutive bins, lane order = descending bins;
// the reads are rotated per lane so that a wave's reads hit distinct banks),
// the lane holding the k-th key is found by a scan over lanes, and its
// segment is then scanned one bin per lane (both scans on DPP).
template <int NB>
__device__ void wave_find_bin(const uint32_t* hist, const uint32_t* he, uint32_t k, uint32_t* out) {
  constexpr int per = NB / 64;
  static_assert(per >= 1 && per <= 64 && (per & (per - 1)) == 0, "NB/64 must be a power of two up to 64");
  const int lane = threadIdx.x & 63;
  const int top = NB - 1 - lane * per;
  uint32_t th = 0u, te = 0u;
#pragma unroll
  for (int i = 0; i < per; ++i) {
    const int b = top - ((i + lane) & (per - 1));
    th += hist[b];
    if (he) te += he[b];
  }
  const uint32_t ih = wave_incl_scan(th), ie = he ? wave_incl_scan(te) : 0u;
  const uint64_t hit = __ballot(ih - th < k && ih >= k);
  const int lf = __ffsll((unsigned long long)hit) - 1;
  const uint32_t run0 = (uint32_t)__builtin_amdgcn_readlane((int)(ih - th), lf);
  const uint32_t rune0 = (uint32_t)__builtin_amdgcn_readlane((int)(ie - te), lf);
  const int b = NB - 1 - lf * per - lane;
  const uint32_t hv = lane < per ? hist[b] : 0u, ev = (lane < per && he) ? he[b] : 0u;
  const uint32_t jh = wave_incl_scan(hv), je = he ? wave_incl_scan(ev) : 0u;
  if (lane < per && run0 + jh - hv < k && run0 + jh >= k) {
    out[0] = (uint32_t)b;
    out[1] = run0 + jh - hv;
    out[2] = rune0 + je - ev;
    out[3] = ev;
  }
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t x, uint32_t* red) {
  x = wave_reduce_max(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  uint32_t m = 0u;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) m = max(m, red[i]);
  return m;
}

// Lanes below this one in the wave whose bit is set in `mask`.
__device__ __forceinline__ uint32_t lane_prefix(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// ---------------------------------------------------------------------------
// Pooling of the keys j in [i0, i1) of one row whose whole window lies in
// the scores this workgroup may read (the caller guarantees it), adding them
// to the row's maximum and top-digit histogram.  xs: kSub + 2*kMaxHalo
// floats, hist: kBins1 words, red: 16 words of LDS.
// ---------------------------------------------------------------------------
constexpr int kSub = 2048;  // keys pooled per round
constexpr int kPoolLdsWords = kSub + 2 * kMaxHalo + kBins1 + 16;

template <int NT>
__device__ void pool_range(const float* __restrict__ srow, float* __restrict__ prow, uint32_t* rw, int Lk, int h,
                           int prot, int i0, int i1, float* xs, uint32_t* hist, uint32_t* red) {
  const int tid = threadIdx.x;
  for (int i = tid; i < kBins1; i += NT) hist[i] = 0u;
  uint32_t kmax = 0u;
  for (int s0 = i0; s0 < i1; s0 += kSub) {
    const int s1 = min(s0 + kSub, i1);
    const int lo = s0 - h, n = s1 + h - lo;
    __syncthreads();
    for (int t = tid; t < n; t += NT) {
      const int j = lo + t;
      xs[t] = (j >= 0 && j < Lk) ? srow[j] : -INFINITY;
    }
    __syncthreads();
    for (int j = s0 + tid; j < s1; j += NT) {
      const float* w = xs + (j - s0);
      float m = -INFINITY;
      for (int t = 0; t <= 2 * h; ++t) m = fmaxf(m, w[t]);
      prow[j] = m;
      const uint32_t key = float_key(m);
      kmax = max(kmax, key);
      if (j < prot) atomicAdd(&hist[key >> kShift1], 1u);
    }
  }
  kmax = block_max_u32(kmax, red);
  if (tid == 0 && i0 < i1) atomicMax(&rw[kRowMax], kmax);
  for (int i = tid; i < kBins1; i += NT)
    if (hist[i]) atomicAdd(&rw[kRowHist1 + i], hist[i]);
}

// The same, when the workgroup's own scores [k_begin, k_end) are in LDS (sc)
// and every window of [i0, i1) lies inside them once clipped to [0, Lk).
// hist: kBins1 words of LDS, zeroed by the caller; red: 16 words of LDS; the
// caller has made sc and the zeroed hist visible.
template <int NT>
__device__ void pool_range_lds(const float* sc, int k_begin, float* __restrict__ prow, uint32_t* rw, int Lk, int h,
                               int prot, int i0, int i1, uint32_t* hist, uint32_t* red) {
  const int tid = threadIdx.x;
  uint32_t kmax = 0u;
  for (int j = i0 + tid; j < i1; j += NT) {
    const int u0 = max(j - h, 0) - k_begin, u1 = min(j + h, Lk - 1) - k_begin;
    float m = -INFINITY;
    for (int u = u0; u <= u1; ++u) m = fmaxf(m, sc[u]);
    prow[j] = m;
    const uint32_t key = float_key(m);
    kmax = max(kmax, key);
    if (j < prot) atomicAdd(&hist[key >> kShift1], 1u);
  }
  kmax = block_max_u32(kmax, red);
  if (tid == 0 && i0 < i1) atomicMax(&rw[kRowMax], kmax);
  for (int i = tid; i < kBins1; i += NT)
    if (hist[i]) atomicAdd(&rw[kRowHist1 + i], hist[i]);
}

}  // namespace dkv
