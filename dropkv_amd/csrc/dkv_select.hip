// Pool / protect / top-k / ascending sort of the DropKV scores on gfx950
// (the selection half of DropKVCache._compute_keep_indices,
// dropkv_cache.py:464-475).
//
//   pooled[j] = max(scores[j-h .. j+h]), h = ks/2, out-of-range = -inf
//   big = max_j pooled[j] + 1.0f ; pooled[Lk-window ..] = big
//   keep_idx = ascending indices of the `keep` largest pooled values; among
//              values equal to the threshold the lowest indices win.
//
// Floats are mapped to order-preserving uint32 keys.  The k-th largest key is
// found by a 3-digit radix select (11 + 11 + 10 bits).  Stage 1 runs over many
// workgroups: it pools, records the row maximum (atomicMax on keys, so the
// result does not depend on scheduling) and accumulates the histogram of the
// top digit.  Stage 2 runs one workgroup per row: it finishes the select on
// the LDS-resident keys and emits the indices in order with ballot prefix
// counts, so the output is sorted without a sort.
#include "dkv_common.h"
#include "dkv_internal.h"

#include <algorithm>

namespace dkv {

constexpr int kPoolChunk = 1024;   // pooled elements per stage-1 workgroup
constexpr int kPoolThreads = 256;
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kBins1 = 2048;        // key bits 31..21
constexpr int kBins2 = 2048;        // key bits 20..10
constexpr int kBins3 = 1024;        // key bits 9..0
constexpr int kLdsKeys = 32768;     // rows up to this length stay in LDS

struct SelectWs {
  // per row: [0] max key, [1..kBins1] top-digit histogram (non-protected keys)
  static constexpr int kRowWords = 1 + kBins1;
};

__global__ void __launch_bounds__(kPoolThreads)
sel_zero_kernel(uint32_t* __restrict__ p, int64_t n, uint64_t* __restrict__ prof) {
  prof_begin(prof, kStSelZero);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
  prof_end(prof, kStSelZero);
}

// Stage 1: grid = rows * ceil(Lk / kPoolChunk).
__global__ void __launch_bounds__(kPoolThreads)
sel_pool_kernel(const float* __restrict__ scores, int Lk, int ks, int window, int chunks,
                float* __restrict__ pooled, uint32_t* __restrict__ rowws, uint64_t* __restrict__ prof) {
  prof_begin(prof, kStSelPool);
  __shared__ uint32_t hist[kBins1];
  __shared__ uint32_t wmax[kPoolThreads / 64];
  const int row = blockIdx.x / chunks;
  const int c0 = (blockIdx.x % chunks) * kPoolChunk;
  const int h = ks / 2;
  const float* s = scores + (int64_t)row * Lk;
  for (int i = threadIdx.x; i < kBins1; i += kPoolThreads) hist[i] = 0u;
  __syncthreads();
  uint32_t kmax = 0u;
  const int prot = Lk - window;
  for (int j = c0 + threadIdx.x; j < min(c0 + kPoolChunk, Lk); j += kPoolThreads) {
    const int lo = max(j - h, 0), hi = min(j + h, Lk - 1);
    float m = -INFINITY;
    for (int t = lo; t <= hi; ++t) m = fmaxf(m, s[t]);
    pooled[(int64_t)row * Lk + j] = m;
    const uint32_t key = float_key(m);
    kmax = max(kmax, key);
    if (j < prot) atomicAdd(&hist[key >> 21], 1u);
  }
  // Block max of keys, then one atomicMax per block.
  for (int o = 32; o >= 1; o >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = kmax;
  __syncthreads();
  uint32_t* rw = rowws + (int64_t)row * SelectWs::kRowWords;
  if (threadIdx.x == 0) {
    uint32_t m = 0u;
    for (int i = 0; i < kPoolThreads / 64; ++i) m = max(m, wmax[i]);
    atomicMax(&rw[0], m);
  }
  for (int i = threadIdx.x; i < kBins1; i += kPoolThreads)
    if (hist[i]) atomicAdd(&rw[1 + i], hist[i]);
  prof_end(prof, kStSelPool);
}

// Inclusive suffix sums over `n` bins of `hist` (in place, n <= 2048) with
// 1024 threads; returns in `*sel_bin` the bin b with suffix(b) >= k and
// suffix(b+1) < k, and in `*above` = suffix(b+1).
__device__ void find_bin(uint32_t* hist, int n, uint32_t k, int* sel_bin, uint32_t* above, uint32_t* wsum) {
  const int tid = threadIdx.x;
  const int per = (n + kSelThreads - 1) / kSelThreads;  // 1 or 2 bins per thread
  // thread t owns bins n-1-(t*per) .. downward (so prefix in thread order = suffix in bin order)
  uint32_t local[2] = {0u, 0u};
  uint32_t tsum = 0u;
  for (int i = 0; i < per; ++i) {
    const int bidx = n - 1 - (tid * per + i);
    local[i] = bidx >= 0 ? hist[bidx] : 0u;
    tsum += local[i];
  }
  // wave inclusive scan of tsum
  const int lane = tid & 63, w = tid >> 6;
  uint32_t x = tsum;
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up((int)x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  uint32_t wpre = 0u;
  for (int i = 0; i < w; ++i) wpre += wsum[i];
  uint32_t run = wpre + x - tsum;  // exclusive prefix (count strictly above my bins)
  for (int i = 0; i < per; ++i) {
    const int bidx = n - 1 - (tid * per + i);
    if (bidx >= 0) {
      const uint32_t nxt = run + local[i];
      if (run < k && nxt >= k) {
        *sel_bin = bidx;
        *above = run;
      }
      run = nxt;
    }
  }
  __syncthreads();
}

// Stage 2: one workgroup of 1024 threads per row.
template <bool LDS_KEYS>
__global__ void __launch_bounds__(kSelThreads)
sel_topk_kernel(const float* __restrict__ pooled_in, int Lk, int window, int keep,
                const uint32_t* __restrict__ rowws, uint32_t* __restrict__ gkeys,
                int64_t* __restrict__ out_idx, float* __restrict__ pooled_out, uint64_t* __restrict__ prof) {
  prof_begin(prof, kStSelTopk);
  extern __shared__ uint32_t dyn[];
  __shared__ uint32_t hist[kBins2];
  __shared__ uint32_t wsum[kSelWaves];
  __shared__ int s_bin;
  __shared__ uint32_t s_above;
  __shared__ uint32_t cnt_gt[kSelWaves * 64], cnt_eq[kSelWaves * 64];  // per (chunk-group, wave)

  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const float* pin = pooled_in + (int64_t)row * Lk;
  const uint32_t* rw = rowws + (int64_t)row * SelectWs::kRowWords;
  uint32_t* keys = LDS_KEYS ? dyn : gkeys + (int64_t)row * Lk;

  const uint32_t kmax = rw[0];
  const float big = key_float(kmax) + 1.0f;
  const uint32_t kbig = float_key(big);
  const int prot = Lk - window;

  for (int j = tid; j < Lk; j += kSelThreads) {
    const uint32_t key = j >= prot ? kbig : float_key(pin[j]);
    keys[j] = key;
    if (pooled_out) pooled_out[(int64_t)row * Lk + j] = j >= prot ? big : pin[j];
  }
  // Digit 1 histogram from stage 1 plus the protected tail.
  for (int i = tid; i < kBins1; i += kSelThreads) hist[i] = rw[1 + i] + ((int)(kbig >> 21) == i ? (uint32_t)window : 0u);
  if (tid == 0) {
    s_bin = 0;
    s_above = 0u;
  }
  __syncthreads();

  uint32_t k = (uint32_t)keep;
  find_bin(hist, kBins1, k, &s_bin, &s_above, wsum);
  uint32_t prefix = (uint32_t)s_bin << 21;
  k -= s_above;
  __syncthreads();

  // Digit 2.
  for (int i = tid; i < kBins2; i += kSelThreads) hist[i] = 0u;
  __syncthreads();
  for (int j = tid; j < Lk; j += kSelThreads) {
    const uint32_t key = keys[j];
    if ((key >> 21) == (prefix >> 21)) atomicAdd(&hist[(key >> 10) & 2047u], 1u);
  }
  __syncthreads();
  find_bin(hist, kBins2, k, &s_bin, &s_above, wsum);
  prefix |= (uint32_t)s_bin << 10;
  k -= s_above;
  __syncthreads();

  // Digit 3.
  for (int i = tid; i < kBins3; i += kSelThreads) hist[i] = 0u;
  __syncthreads();
  for (int j = tid; j < Lk; j += kSelThreads) {
    const uint32_t key = keys[j];
    if ((key >> 10) == (prefix >> 10)) atomicAdd(&hist[key & 1023u], 1u);
  }
  __syncthreads();
  find_bin(hist, kBins3, k, &s_bin, &s_above, wsum);
  const uint32_t T = prefix | (uint32_t)s_bin;
  const uint32_t take_eq = k - s_above;  // how many keys equal to T are kept (lowest indices first)
  __syncthreads();

  // Ordered emission.  Indices are visited in rounds of kSelThreads
  // consecutive positions (round c: j = c*1024 + tid).  First count, per
  // (round, wave), keys > T and == T; then exclusive-scan those counts in
  // index order; then every thread knows its output slot.
  const int rounds = (Lk + kSelThreads - 1) / kSelThreads;
  for (int c0 = 0; c0 < rounds; c0 += 64) {
    const int cn = min(64, rounds - c0);
    for (int c = 0; c < cn; ++c) {
      const int j = (c0 + c) * kSelThreads + tid;
      const uint32_t key = j < Lk ? keys[j] : 0u;
      const unsigned long long bg = __ballot(j < Lk && key > T);
      const unsigned long long be = __ballot(j < Lk && key == T);
      if (lane == 0) {
        cnt_gt[c * kSelWaves + w] = (uint32_t)__popcll(bg);
        cnt_eq[c * kSelWaves + w] = (uint32_t)__popcll(be);
      }
    }
    __syncthreads();
    // Exclusive scan over cn*kSelWaves entries (index order = c-major, w-minor), by wave 0.
    __shared__ uint32_t carry_gt, carry_eq;
    if (c0 == 0 && tid == 0) {
      carry_gt = 0u;
      carry_eq = 0u;
    }
    __syncthreads();
    if (w == 0) {
      const int n = cn * kSelWaves;
      uint32_t cg = carry_gt, ce = carry_eq;
      for (int base = 0; base < n; base += 64) {
        const int i = base + lane;
        const uint32_t vg = i < n ? cnt_gt[i] : 0u, ve = i < n ? cnt_eq[i] : 0u;
        uint32_t xg = vg, xe = ve;
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t yg = __shfl_up((int)xg, o), ye = __shfl_up((int)xe, o);
          if (lane >= o) {
            xg += yg;
            xe += ye;
          }
        }
        if (i < n) {
          cnt_gt[i] = cg + xg - vg;
          cnt_eq[i] = ce + xe - ve;
        }
        cg += __shfl((int)xg, 63);
        ce += __shfl((int)xe, 63);
      }
      if (lane == 0) {
        carry_gt = cg;
        carry_eq = ce;
      }
    }
    __syncthreads();
    for (int c = 0; c < cn; ++c) {
      const int j = (c0 + c) * kSelThreads + tid;
      const uint32_t key = j < Lk ? keys[j] : 0u;
      const bool gt = j < Lk && key > T, eq = j < Lk && key == T;
      const unsigned long long bg = __ballot(gt);
      const unsigned long long be = __ballot(eq);
      const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      const uint32_t ngt = cnt_gt[c * kSelWaves + w] + (uint32_t)__popcll(bg & below);
      const uint32_t neq = cnt_eq[c * kSelWaves + w] + (uint32_t)__popcll(be & below);
      const bool kept = gt || (eq && neq < take_eq);
      const uint32_t pos = ngt + min(neq, take_eq);
      if (kept && pos < (uint32_t)keep) out_idx[(int64_t)row * keep + pos] = j;
    }
    __syncthreads();
  }
  prof_end(prof, kStSelTopk);
}

size_t select_workspace_bytes(int64_t rows, int64_t Lk) {
  size_t words = (size_t)rows * SelectWs::kRowWords;
  size_t b = (words * 4 + 255) & ~size_t(255);
  b += ((size_t)rows * Lk * 4 + 255) & ~size_t(255);  // pooled floats
  if (Lk > kLdsKeys) b += ((size_t)rows * Lk * 4 + 255) & ~size_t(255);  // global keys
  return b;
}

int64_t select_zero_words(int64_t rows) { return rows * SelectWs::kRowWords; }

hipError_t launch_select(const float* scores, int rows, int Lk, int ks, int window, int keep, int64_t* out_idx,
                         float* pooled_out, char* ws, bool pre_zeroed, hipStream_t st) {
  uint32_t* rowws = reinterpret_cast<uint32_t*>(ws);
  size_t off = ((size_t)rows * SelectWs::kRowWords * 4 + 255) & ~size_t(255);
  float* pooled = reinterpret_cast<float*>(ws + off);
  off += ((size_t)rows * Lk * 4 + 255) & ~size_t(255);
  uint32_t* gkeys = reinterpret_cast<uint32_t*>(ws + off);

  uint64_t* prof = prof_slot();
  if (!pre_zeroed) {
    const int64_t zn = (int64_t)rows * SelectWs::kRowWords;
    hipLaunchKernelGGL(sel_zero_kernel, dim3((unsigned)std::min<int64_t>((zn + 255) / 256, 1024)), dim3(256), 0, st,
                       rowws, zn, prof);
  }
  const int chunks = (Lk + kPoolChunk - 1) / kPoolChunk;
  hipLaunchKernelGGL(sel_pool_kernel, dim3(rows * chunks), dim3(kPoolThreads), 0, st, scores, Lk, ks, window,
                     chunks, pooled, rowws, prof);
  if (Lk <= kLdsKeys) {
    static bool attr_set = false;
    if (!attr_set) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&sel_topk_kernel<true>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, kLdsKeys * 4);
      if (e != hipSuccess) return e;
      attr_set = true;
    }
    hipLaunchKernelGGL((sel_topk_kernel<true>), dim3(rows), dim3(kSelThreads), (size_t)Lk * 4, st, pooled, Lk,
                       window, keep, rowws, gkeys, out_idx, pooled_out, prof);
  } else {
    hipLaunchKernelGGL((sel_topk_kernel<false>), dim3(rows), dim3(kSelThreads), 0, st, pooled, Lk, window, keep,
                       rowws, gkeys, out_idx, pooled_out, prof);
  }
  return hipGetLastError();
}

}  // namespace dkv
