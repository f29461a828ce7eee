// Pool / protect / top-k / ascending sort of the DropKV scores on gfx950 (the
// selection half of DropKVCache._compute_keep_indices, dropkv_cache.py:464-475),
// optionally fused with the gather into the compressed cache
// (DropKVCache._gather_compressed, dropkv_cache.py:479-491).
//
//   pooled[j] = max(scores[j-h .. j+h]), h = ks/2, out-of-range = -inf
//   big = max_j pooled[j] + 1.0f ; pooled[Lk-window ..] = big
//   keep_idx = ascending indices of the `keep` largest pooled values; among
//              values equal to the threshold the lowest indices win.
//
// Floats are mapped to order-preserving uint32 keys and the keep-th largest
// key T is found by a radix select over 11 + 11 + 10 bits.  Every stage runs
// over (row, 1024-key chunk) workgroups, so all CUs take part:
//   pool   sliding max, row maximum (atomicMax on keys), histogram of the top
//          digit of the unprotected keys;
//   cand   every chunk finds the boundary bin of the top digit, counts its
//          keys above it and appends the keys inside it to a per-row
//          candidate list;
//   final  one workgroup per row resolves the two lower digits on the
//          candidates (a few percent of the row) and turns per-chunk counts
//          into output offsets;
//   emit   every chunk writes its kept indices at those offsets, in index
//          order (block prefix sums), and copies the kept K/V rows.
#include "dkv_common.h"
#include "dkv_internal.h"

#include <algorithm>

namespace dkv {

constexpr int kSelT = 256;            // threads per workgroup, all stages
constexpr int kChunk = 1024;          // keys per workgroup
constexpr int kPer = kChunk / kSelT;  // keys per thread
constexpr int kBins1 = 2048;          // key bits 31..21
constexpr int kBins2 = 2048;          // key bits 20..10
constexpr int kBins3 = 1024;          // key bits 9..0
constexpr int kMaxHalo = 64;          // kernel_size <= 2*kMaxHalo+1
constexpr int kMaxChunks = 4096;      // Lk <= kMaxChunks * kChunk
constexpr int kBatch = 8;             // independent loads in flight per thread
constexpr int kCandLds = 8192;        // candidates staged in LDS by the final stage

// Per-row words that must be zero on entry:
//   [0] max pooled key, [1 .. kBins1] top-digit histogram of the unprotected
//   keys, [kBins1+1] candidate count.
constexpr int kRowWords = kBins1 + 2;
constexpr int kCandCount = kBins1 + 1;

struct SelWs {
  uint32_t* rowws;     // [rows][kRowWords], zeroed per call
  float* pooled;       // [rows][Lk]
  uint32_t* cand_key;  // [rows][Lk]
  uint32_t* cand_idx;  // [rows][Lk]
  uint32_t* above;     // [rows][chunks] keys of a chunk above the boundary bin
  uint32_t* gt_off;    // [rows][chunks] kept keys > T in earlier chunks
  uint32_t* eq_off;    // [rows][chunks] keys == T in earlier chunks
  uint32_t* thr;       // [rows][2] T, number of keys == T kept
};

static inline size_t al256(size_t b) { return (b + 255) & ~size_t(255); }

static SelWs sel_layout(char* base, int64_t rows, int64_t Lk, size_t* total) {
  const int64_t chunks = (Lk + kChunk - 1) / kChunk;
  SelWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += al256(bytes);
    return p;
  };
  w.rowws = reinterpret_cast<uint32_t*>(take((size_t)rows * kRowWords * 4));
  w.pooled = reinterpret_cast<float*>(take((size_t)rows * Lk * 4));
  w.cand_key = reinterpret_cast<uint32_t*>(take((size_t)rows * Lk * 4));
  w.cand_idx = reinterpret_cast<uint32_t*>(take((size_t)rows * Lk * 4));
  w.above = reinterpret_cast<uint32_t*>(take((size_t)rows * chunks * 4));
  w.gt_off = reinterpret_cast<uint32_t*>(take((size_t)rows * chunks * 4));
  w.eq_off = reinterpret_cast<uint32_t*>(take((size_t)rows * chunks * 4));
  w.thr = reinterpret_cast<uint32_t*>(take((size_t)rows * 2 * 4));
  if (total) *total = off;
  return w;
}

// ---------------------------------------------------------------------------
// Block-level helpers for kSelT threads.
// ---------------------------------------------------------------------------
// Exclusive prefix sums of two counters over the threads of the block, and
// optionally their block totals.
__device__ __forceinline__ void block_excl_scan2(uint32_t a, uint32_t b, uint32_t* pa, uint32_t* pb,
                                                 uint32_t* ta, uint32_t* tb, uint32_t* wsum /*[8]*/) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t xa = a, xb = b;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t ya = __shfl_up((int)xa, o), yb = __shfl_up((int)xb, o);
    if (lane >= o) {
      xa += ya;
      xb += yb;
    }
  }
  __syncthreads();
  if (lane == 63) {
    wsum[w] = xa;
    wsum[4 + w] = xb;
  }
  __syncthreads();
  uint32_t oa = 0, ob = 0, sa = 0, sb = 0;
#pragma unroll
  for (int i = 0; i < kSelT / 64; ++i) {
    if (i < w) {
      oa += wsum[i];
      ob += wsum[4 + i];
    }
    sa += wsum[i];
    sb += wsum[4 + i];
  }
  *pa = oa + xa - a;
  *pb = ob + xb - b;
  if (ta) *ta = sa;
  if (tb) *tb = sb;
}

// For a histogram of NB bins in LDS and 1 <= k <= total: the bin b with
// (count of keys in bins > b) < k <= (count in bins >= b), and the count in
// bins > b.  Results land in *s_bin / *s_above (LDS); ends with a barrier.
template <int NB>
__device__ void find_bin(const uint32_t* hist, uint32_t k, int* s_bin, uint32_t* s_above, uint32_t* wsum) {
  constexpr int per = NB / kSelT;
  const int tid = threadIdx.x;
  uint32_t loc[per];
  uint32_t tsum = 0u;
#pragma unroll
  for (int i = 0; i < per; ++i) {
    loc[i] = hist[NB - 1 - (tid * per + i)];  // thread order = descending bins
    tsum += loc[i];
  }
  uint32_t run, dummy;
  block_excl_scan2(tsum, 0u, &run, &dummy, nullptr, nullptr, wsum);
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

__global__ void __launch_bounds__(kSelT)
sel_zero_kernel(uint32_t* __restrict__ p, int64_t n, uint64_t* __restrict__ prof) {
  prof_begin(prof, kStSelZero);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
  prof_end(prof, kStSelZero);
}

// ---------------------------------------------------------------------------
// Stage "pool": grid = rows * chunks.  The chunk and its halo are staged in
// LDS with all global loads in flight at once; the sliding max reads LDS.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kSelT)
sel_pool_kernel(const float* __restrict__ scores, int Lk, int ks, int window, int chunks, SelWs ws,
                uint64_t* __restrict__ prof) {
  prof_begin(prof, kStSelPool);
  __shared__ uint32_t hist[kBins1];
  __shared__ uint32_t wmax[kSelT / 64];
  __shared__ float xs[kChunk + 2 * kMaxHalo];
  const int tid = threadIdx.x;
  const int row = blockIdx.x / chunks;
  const int c0 = (blockIdx.x % chunks) * kChunk;
  const int h = ks / 2;
  const float* s = scores + (int64_t)row * Lk;

  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = c0 + tid + i * kSelT;
    v[i] = j < Lk ? s[j] : -INFINITY;
  }
  float hv = -INFINITY;
  int hslot = -1;
  if (tid < 2 * h) {
    const int j = tid < h ? c0 - h + tid : c0 + kChunk + (tid - h);
    hslot = tid < h ? kMaxHalo - h + tid : kMaxHalo + kChunk + (tid - h);
    hv = (j >= 0 && j < Lk) ? s[j] : -INFINITY;
  }
  for (int i = tid; i < kBins1; i += kSelT) hist[i] = 0u;
#pragma unroll
  for (int i = 0; i < kPer; ++i) xs[kMaxHalo + tid + i * kSelT] = v[i];
  if (hslot >= 0) xs[hslot] = hv;
  __syncthreads();

  uint32_t kmax = 0u;
  const int prot = Lk - window;
  float* pooled = ws.pooled + (int64_t)row * Lk;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int jl = tid + i * kSelT;
    const int j = c0 + jl;
    if (j < Lk) {
      const float* w = xs + kMaxHalo + jl - h;
      float m = -INFINITY;
#pragma unroll 11
      for (int t = 0; t <= 2 * h; ++t) m = fmaxf(m, w[t]);
      pooled[j] = m;
      const uint32_t key = float_key(m);
      kmax = max(kmax, key);
      if (j < prot) atomicAdd(&hist[key >> 21], 1u);
    }
  }
  for (int o = 32; o >= 1; o >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
  if ((tid & 63) == 0) wmax[tid >> 6] = kmax;
  __syncthreads();
  uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  if (tid == 0) {
    uint32_t m = 0u;
    for (int i = 0; i < kSelT / 64; ++i) m = max(m, wmax[i]);
    atomicMax(&rw[0], m);
  }
  for (int i = tid; i < kBins1; i += kSelT)
    if (hist[i]) atomicAdd(&rw[1 + i], hist[i]);
  prof_end(prof, kStSelPool);
}

// ---------------------------------------------------------------------------
// Stage "cand": grid = rows * chunks.  Each chunk finds the boundary bin of
// the top digit (all chunks compute the same one), counts its keys above it
// and appends the keys inside it to the row's candidate list.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kSelT)
sel_cand_kernel(int Lk, int window, int keep, int chunks, SelWs ws, uint64_t* __restrict__ prof) {
  prof_begin(prof, kStSelTopk);
  __shared__ uint32_t hist[kBins1];
  __shared__ uint32_t wsum[8];
  __shared__ int s_bin;
  __shared__ uint32_t s_above;
  const int tid = threadIdx.x;
  const int row = blockIdx.x / chunks;
  const int c = blockIdx.x % chunks;
  uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  const float* pooled = ws.pooled + (int64_t)row * Lk;
  uint32_t* ckey = ws.cand_key + (int64_t)row * Lk;
  uint32_t* cidx = ws.cand_idx + (int64_t)row * Lk;

  const float big = key_float(rw[0]) + 1.0f;
  const uint32_t kbig = float_key(big);
  const int prot = Lk - window;
  uint32_t keys[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = c * kChunk + tid + i * kSelT;
    keys[i] = j < Lk ? (j >= prot ? kbig : float_key(pooled[j])) : 0u;
  }
  for (int i = tid; i < kBins1; i += kSelT) hist[i] = rw[1 + i] + ((int)(kbig >> 21) == i ? (uint32_t)window : 0u);
  if (tid == 0) {
    s_bin = 0;
    s_above = 0u;
  }
  __syncthreads();
  find_bin<kBins1>(hist, (uint32_t)keep, &s_bin, &s_above, wsum);
  const uint32_t b1 = (uint32_t)s_bin;

  // Count this thread's keys above / inside the boundary bin, then reserve
  // the block's candidate slots with a single atomic.
  uint32_t above = 0u, ncand = 0u;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = c * kChunk + tid + i * kSelT;
    if (j < Lk) {
      above += (keys[i] >> 21) > b1 ? 1u : 0u;
      ncand += (keys[i] >> 21) == b1 ? 1u : 0u;
    }
  }
  uint32_t pa, pc, tot_above, tot_cand;
  block_excl_scan2(above, ncand, &pa, &pc, &tot_above, &tot_cand, wsum);
  __shared__ uint32_t s_base;
  if (tid == 0) {
    s_base = tot_cand ? atomicAdd(&rw[kCandCount], tot_cand) : 0u;
    ws.above[(int64_t)row * chunks + c] = tot_above;
    if (c == 0) {
      ws.thr[row * 2 + 0] = b1;  // boundary bin and what remains to take in it
      ws.thr[row * 2 + 1] = (uint32_t)keep - s_above;
    }
  }
  __syncthreads();
  uint32_t pos = s_base + pc;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = c * kChunk + tid + i * kSelT;
    if (j < Lk && (keys[i] >> 21) == b1) {
      ckey[pos] = keys[i];
      cidx[pos] = (uint32_t)j;
      ++pos;
    }
  }
  prof_end(prof, kStSelTopk);
}

// ---------------------------------------------------------------------------
// Stage "final": one workgroup per row.  Resolves the two lower digits on the
// candidates, giving the threshold key T and how many keys equal to T are
// kept, and turns per-chunk counts into output offsets.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kSelT)
sel_final_kernel(int chunks, SelWs ws, int64_t Lk, uint64_t* __restrict__ prof) {
  prof_begin(prof, kStSelZero);
  __shared__ uint32_t hist[kBins2];
  __shared__ uint32_t cgt[kMaxChunks], ceq[kMaxChunks];
  __shared__ uint32_t wsum[8];
  __shared__ int s_bin;
  __shared__ uint32_t s_above;
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  const uint32_t nc = rw[kCandCount];
  const uint32_t b1 = ws.thr[row * 2 + 0];
  const uint32_t k1 = ws.thr[row * 2 + 1];
  // The candidates (typically a few percent of the row) are read three
  // times: stage them in LDS when they fit.
  __shared__ uint32_t lkey[kCandLds], lidx[kCandLds];
  const uint32_t* ckey = ws.cand_key + (int64_t)row * Lk;
  const uint32_t* cidx = ws.cand_idx + (int64_t)row * Lk;
  if (nc <= (uint32_t)kCandLds) {
    for (uint32_t base = 0; base < nc; base += kSelT * kBatch) {
      uint32_t kv[kBatch], iv[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const uint32_t p = base + tid + i * kSelT;
        kv[i] = p < nc ? ckey[p] : 0u;
        iv[i] = p < nc ? cidx[p] : 0u;
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const uint32_t p = base + tid + i * kSelT;
        if (p < nc) {
          lkey[p] = kv[i];
          lidx[p] = iv[i];
        }
      }
    }
    ckey = lkey;
    cidx = lidx;
  }

  // Digit 2 over the candidates.
  for (int i = tid; i < kBins2; i += kSelT) hist[i] = 0u;
  if (tid == 0) {
    s_bin = 0;
    s_above = 0u;
  }
  __syncthreads();
  for (uint32_t base = 0; base < nc; base += kSelT * kBatch) {
    uint32_t kv[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const uint32_t p = base + tid + i * kSelT;
      kv[i] = p < nc ? ckey[p] : 0u;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (base + tid + i * kSelT < nc) atomicAdd(&hist[(kv[i] >> 10) & 2047u], 1u);
  }
  __syncthreads();
  find_bin<kBins2>(hist, k1, &s_bin, &s_above, wsum);
  const uint32_t b2 = (uint32_t)s_bin;
  const uint32_t k2 = k1 - s_above;
  // Digit 3 over the candidates that match the first two digits.
  for (int i = tid; i < kBins3; i += kSelT) hist[i] = 0u;
  __syncthreads();
  const uint32_t pre = (b1 << 11) | b2;
  for (uint32_t base = 0; base < nc; base += kSelT * kBatch) {
    uint32_t kv[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const uint32_t p = base + tid + i * kSelT;
      kv[i] = p < nc ? ckey[p] : 0u;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (base + tid + i * kSelT < nc && (kv[i] >> 10) == pre) atomicAdd(&hist[kv[i] & 1023u], 1u);
  }
  __syncthreads();
  find_bin<kBins3>(hist, k2, &s_bin, &s_above, wsum);
  const uint32_t T = (pre << 10) | (uint32_t)s_bin;
  const uint32_t take_eq = k2 - s_above;

  // Per-chunk counts of keys > T and == T, then exclusive offsets over chunks.
  for (int i = tid; i < chunks; i += kSelT) {
    cgt[i] = ws.above[(int64_t)row * chunks + i];
    ceq[i] = 0u;
  }
  __syncthreads();
  for (uint32_t base = 0; base < nc; base += kSelT * kBatch) {
    uint32_t kv[kBatch], iv[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const uint32_t p = base + tid + i * kSelT;
      kv[i] = p < nc ? ckey[p] : 0u;
      iv[i] = p < nc ? cidx[p] : 0u;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (base + tid + i * kSelT < nc) {
        if (kv[i] > T) atomicAdd(&cgt[iv[i] / kChunk], 1u);
        else if (kv[i] == T) atomicAdd(&ceq[iv[i] / kChunk], 1u);
      }
    }
  }
  __syncthreads();
  const int cpt = (chunks + kSelT - 1) / kSelT;  // chunks per thread, contiguous
  uint32_t sg = 0u, se = 0u;
  for (int i = 0; i < cpt; ++i) {
    const int cc = tid * cpt + i;
    if (cc < chunks) {
      sg += cgt[cc];
      se += ceq[cc];
    }
  }
  uint32_t og, oe;
  block_excl_scan2(sg, se, &og, &oe, nullptr, nullptr, wsum);
  for (int i = 0; i < cpt; ++i) {
    const int cc = tid * cpt + i;
    if (cc < chunks) {
      ws.gt_off[(int64_t)row * chunks + cc] = og;
      ws.eq_off[(int64_t)row * chunks + cc] = oe;
      og += cgt[cc];
      oe += ceq[cc];
    }
  }
  __syncthreads();
  if (tid == 0) {
    ws.thr[row * 2 + 0] = T;
    ws.thr[row * 2 + 1] = take_eq;
  }
  prof_end(prof, kStSelZero);
}

// ---------------------------------------------------------------------------
// Stage "emit": grid = rows * chunks.  Thread t owns the kPer consecutive keys
// c*kChunk + kPer*t ..; kept keys are written in index order, then (when
// ko is given) their K/V rows are copied.
// ---------------------------------------------------------------------------
struct CompactArgs {
  const uint8_t* k;
  const uint8_t* v;
  int64_t sb, sh, sl;  // source byte strides
  int H;
  int units;           // 16-byte units per row
  uint8_t* ko;
  uint8_t* vo;
};

__global__ void __launch_bounds__(kSelT)
sel_emit_kernel(int Lk, int window, int keep, int chunks, SelWs ws, int64_t* __restrict__ out_idx,
                float* __restrict__ pooled_out, CompactArgs ca, uint64_t* __restrict__ prof) {
  prof_begin(prof, kStCompact);
  __shared__ uint32_t wsum[8];
  __shared__ int s_src[kChunk];
  __shared__ int s_dst[kChunk];
  const int tid = threadIdx.x;
  const int row = blockIdx.x / chunks;
  const int c = blockIdx.x % chunks;
  const uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  const float* pooled = ws.pooled + (int64_t)row * Lk;
  const float big = key_float(rw[0]) + 1.0f;
  const uint32_t kbig = float_key(big);
  const int prot = Lk - window;
  const uint32_t T = ws.thr[row * 2 + 0], take_eq = ws.thr[row * 2 + 1];
  const uint32_t gt0 = ws.gt_off[(int64_t)row * chunks + c], eq0 = ws.eq_off[(int64_t)row * chunks + c];

  const int j0 = c * kChunk + kPer * tid;
  float pv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) pv[i] = (j0 + i < Lk) ? pooled[j0 + i] : 0.f;
  uint32_t keys[kPer];
  uint32_t ng = 0u, ne = 0u;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = j0 + i;
    keys[i] = j >= prot ? kbig : float_key(pv[i]);
    if (j < Lk) {
      ng += keys[i] > T ? 1u : 0u;
      ne += keys[i] == T ? 1u : 0u;
      if (pooled_out) pooled_out[(int64_t)row * Lk + j] = j >= prot ? big : pv[i];
    }
  }
  uint32_t pg, pe, tg, te;
  block_excl_scan2(ng, ne, &pg, &pe, &tg, &te, wsum);
  const uint32_t start = gt0 + min(eq0, take_eq);  // first output slot of this chunk
  uint32_t g_before = gt0 + pg, e_before = eq0 + pe;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = j0 + i;
    if (j < Lk) {
      const bool gt = keys[i] > T, eq = keys[i] == T;
      const bool kept = gt || (eq && e_before < take_eq);
      if (kept) {
        const uint32_t pos = g_before + min(e_before, take_eq);
        if (pos < (uint32_t)keep) {
          out_idx[(int64_t)row * keep + pos] = j;
          s_src[pos - start] = j;
          s_dst[pos - start] = (int)pos;
        }
      }
      g_before += gt ? 1u : 0u;
      e_before += eq ? 1u : 0u;
    }
  }
  if (ca.ko) {
    __syncthreads();
    const uint32_t last = min(gt0 + tg + min(eq0 + te, take_eq), (uint32_t)keep);
    const int nk = (int)min(last - start, (uint32_t)kChunk);
    const int b = row / ca.H, h = row % ca.H;
    const int total = nk * ca.units;
    const uint8_t* kb = ca.k + b * ca.sb + h * ca.sh;
    const uint8_t* vb = ca.v + b * ca.sb + h * ca.sh;
    for (int t0 = tid; t0 < total; t0 += 4 * kSelT) {
      u32x4 kv[4], vv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = t0 + q * kSelT;
        if (t < total) {
          const int64_t off = (int64_t)s_src[t / ca.units] * ca.sl + 16 * (t % ca.units);
          kv[q] = *reinterpret_cast<const u32x4*>(kb + off);
          vv[q] = *reinterpret_cast<const u32x4*>(vb + off);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = t0 + q * kSelT;
        if (t < total) {
          const int64_t o = ((int64_t)row * keep + s_dst[t / ca.units]) * ca.units * 16 + 16 * (t % ca.units);
          *reinterpret_cast<u32x4*>(ca.ko + o) = kv[q];
          *reinterpret_cast<u32x4*>(ca.vo + o) = vv[q];
        }
      }
    }
  }
  prof_end(prof, kStCompact);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
size_t select_workspace_bytes(int64_t rows, int64_t Lk) {
  size_t total = 0;
  sel_layout(nullptr, rows, Lk, &total);
  return total;
}

int64_t select_zero_words(int64_t rows) { return rows * kRowWords; }

int64_t select_max_len() { return (int64_t)kMaxChunks * kChunk; }

hipError_t launch_select(const float* scores, int rows, int Lk, int ks, int window, int keep, int64_t* out_idx,
                         float* pooled_out, char* ws_base, bool pre_zeroed, const SelectCompact* cp,
                         hipStream_t st) {
  const SelWs ws = sel_layout(ws_base, rows, Lk, nullptr);
  const int chunks = (Lk + kChunk - 1) / kChunk;
  uint64_t* prof = prof_slot();
  if (!pre_zeroed) {
    const int64_t zn = (int64_t)rows * kRowWords;
    hipLaunchKernelGGL(sel_zero_kernel, dim3((unsigned)std::min<int64_t>((zn + kSelT - 1) / kSelT, 1024)),
                       dim3(kSelT), 0, st, ws.rowws, zn, prof);
    timing_mark(st);
  }
  const dim3 grid((unsigned)(rows * chunks));
  hipLaunchKernelGGL(sel_pool_kernel, grid, dim3(kSelT), 0, st, scores, Lk, ks, window, chunks, ws, prof);
  timing_mark(st);
  hipLaunchKernelGGL(sel_cand_kernel, grid, dim3(kSelT), 0, st, Lk, window, keep, chunks, ws, prof);
  timing_mark(st);
  hipLaunchKernelGGL(sel_final_kernel, dim3((unsigned)rows), dim3(kSelT), 0, st, chunks, ws, (int64_t)Lk, prof);
  timing_mark(st);
  CompactArgs ca{};
  if (cp) {
    ca.k = static_cast<const uint8_t*>(cp->k);
    ca.v = static_cast<const uint8_t*>(cp->v);
    ca.sb = cp->s_b * cp->elem_bytes;
    ca.sh = cp->s_h * cp->elem_bytes;
    ca.sl = cp->s_l * cp->elem_bytes;
    ca.H = cp->H;
    ca.units = (int)(cp->D * cp->elem_bytes / 16);
    ca.ko = static_cast<uint8_t*>(cp->k_out);
    ca.vo = static_cast<uint8_t*>(cp->v_out);
  }
  hipLaunchKernelGGL(sel_emit_kernel, grid, dim3(kSelT), 0, st, Lk, window, keep, chunks, ws, out_idx, pooled_out,
                     ca, prof);
  timing_mark(st);
  return hipGetLastError();
}

}  // namespace dkv
