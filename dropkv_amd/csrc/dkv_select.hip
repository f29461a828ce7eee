// Pool / protect / top-k / ascending sort of the DropKV scores on gfx950 (the
// selection half of DropKVCache._compute_keep_indices, dropkv_cache.py:464-475),
// optionally fused with the gather into the compressed cache
// (DropKVCache._gather_compressed, dropkv_cache.py:479-491).  The stages are
// described in dkv_select_dev.h.
//
// Standalone (dropkv_select): zero -> pool -> resolve -> emit.
// After a scoring pass that pooled its interiors (dropkv_evict): resolve -> emit.
#include "dkv_common.h"
#include "dkv_internal.h"
#include "dkv_select_dev.h"

#include <algorithm>

namespace dkv {

constexpr int kSelT = 1024;           // threads per workgroup: zero, pool
#ifndef DKV_EMIT_T
#define DKV_EMIT_T 256
#endif
constexpr int kEmitT = DKV_EMIT_T;    // threads per emit workgroup (one 1024-key chunk; 256: C5 emit 67 -> 41 us)
constexpr int kPer = kChunk / kEmitT;  // keys per emit thread

__global__ void __launch_bounds__(kSelT)
sel_zero_kernel(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// ---------------------------------------------------------------------------
// pool (standalone): grid = rows * chunks, every key of the chunk (the
// complete score row is readable, so windows may cross chunk edges).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kSelT)
sel_pool_kernel(const float* __restrict__ scores, int Lk, int ks, int window, int chunks, SelWs ws) {
  __shared__ uint32_t lds[kPoolLdsWords];
  const int row = blockIdx.x / chunks;
  const int c0 = (blockIdx.x % chunks) * kChunk;
  float* xs = reinterpret_cast<float*>(lds);
  uint32_t* hist = lds + kSub + 2 * kMaxHalo;
  uint32_t* red = hist + kBins1;
  pool_range<kSelT>(scores + (int64_t)row * Lk, ws.pooled + (int64_t)row * Lk, ws.rowws + (int64_t)row * kRowWords,
                    Lk, ks / 2, Lk - window, c0, min(c0 + kChunk, Lk), xs, hist, red);
}

// ---------------------------------------------------------------------------
// pool (standalone) for any kernel size, also those whose window exceeds the
// LDS halo of sel_pool_kernel (h > kMaxHalo).  The row is cut into blocks of
// w = 2h+1 keys (van Herk / Gil-Werman):
//   pre[j] = max x[block start .. j],  suf[j] = max x[j .. block end]
// (the last block ends at Lk-1).  A window [a, b] (a = max(j-h, 0),
// b = min(j+h, Lk-1), at most w keys) meets at most two blocks, so
//   max x[a..b] = max(suf[a], pre[b])  if a and b lie in different blocks,
//                 pre[b]               if a starts their common block,
//                 suf[a]               otherwise (then b = Lk-1 ends it).
// ---------------------------------------------------------------------------
constexpr int kWideScanT = 256;  // one wave per block of w keys

__device__ __forceinline__ float wave_incl_max_scan(float x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float t = __shfl_up(x, o);
    if (lane >= o) x = fmaxf(x, t);
  }
  return x;
}

// pre / suf: [rows][Lk] each (the tail's candidate regions, unused here).
__global__ void __launch_bounds__(kWideScanT)
sel_pool_wide_scan_kernel(const float* __restrict__ scores, int rows, int Lk, int w, int nblk,
                          float* __restrict__ pre, float* __restrict__ suf) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * (kWideScanT / 64) + (threadIdx.x >> 6);
  if (gw >= (int64_t)rows * nblk) return;
  const int row = (int)(gw / nblk), blk = (int)(gw % nblk);
  const int start = blk * w, end = min(start + w, Lk);  // keys [start, end)
  const float* x = scores + (int64_t)row * Lk;
  float* pr = pre + (int64_t)row * Lk;
  float* sf = suf + (int64_t)row * Lk;
  float carry = -INFINITY;
  for (int c = start; c < end; c += 64) {
    const int j = c + lane;
    const float v = fmaxf(wave_incl_max_scan(j < end ? x[j] : -INFINITY), carry);
    if (j < end) pr[j] = v;
    carry = __shfl(v, 63);
  }
  carry = -INFINITY;
  for (int c = end - 1; c >= start; c -= 64) {
    const int j = c - lane;  // lane 0 holds the block's last key of this round
    const float v = fmaxf(wave_incl_max_scan(j >= start ? x[j] : -INFINITY), carry);
    if (j >= start) sf[j] = v;
    carry = __shfl(v, 63);
  }
}

// grid = rows * chunks: the pooled values of the chunk's keys from pre / suf,
// into the pooled row, the row maximum and the top-digit histogram.
__global__ void __launch_bounds__(kSelT)
sel_pool_wide_kernel(const float* __restrict__ pre, const float* __restrict__ suf, int Lk, int h, int window,
                     int chunks, SelWs ws) {
  __shared__ uint32_t hist[kBins1];
  __shared__ uint32_t red[16];
  const int tid = threadIdx.x;
  const int row = blockIdx.x / chunks;
  const int c0 = (blockIdx.x % chunks) * kChunk, c1 = min(c0 + kChunk, Lk);
  const int w = 2 * h + 1, prot = Lk - window;
  const float* pr = pre + (int64_t)row * Lk;
  const float* sf = suf + (int64_t)row * Lk;
  float* prow = ws.pooled + (int64_t)row * Lk;
  uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  for (int i = tid; i < kBins1; i += kSelT) hist[i] = 0u;
  __syncthreads();
  uint32_t kmax = 0u;
  for (int j = c0 + tid; j < c1; j += kSelT) {
    const int a = max(j - h, 0), b = (int)min((int64_t)j + h, (int64_t)Lk - 1);
    const float m = a / w != b / w ? fmaxf(sf[a], pr[b]) : (a % w == 0 ? pr[b] : sf[a]);
    prow[j] = m;
    const uint32_t key = float_key(m);
    kmax = max(kmax, key);
    if (j < prot) atomicAdd(&hist[key >> kShift1], 1u);
  }
  kmax = block_max_u32(kmax, red);
  if (tid == 0 && c0 < c1) atomicMax(&rw[kRowMax], kmax);
  __syncthreads();
  for (int i = tid; i < kBins1; i += kSelT)
    if (hist[i]) atomicAdd(&rw[kRowHist1 + i], hist[i]);
}

// ---------------------------------------------------------------------------
// resolve: grid = rows * parts; part p of a row sweeps its chunks
// [p*cpp, (p+1)*cpp).
//   A. (every part) Pools the keys next to the scoring pass's split
//      boundaries (their windows straddle two workgroup ranges; the part
//      writes those in its chunks to the pooled row), which completes the
//      row's top-digit histogram and maximum in LDS; finds the top-digit bin
//      b1 of the keep-th largest key.
//   B. (every part) One sweep of its chunks: per chunk the keys above b1
//      (into cnt[].x), the keys inside b1 (the candidates) appended to the
//      row's list in the workspace; then its arrival on the row's counter.
//      What B and A publish is written with device-coherent stores, so an
//      arrival needs only the wait for them.
//   C. (the row's last part to arrive) Digits 2 and 3 over the candidates:
//      the threshold key T and how many keys equal to T are kept (the lowest
//      indices).
//   D. (the same) Per chunk, the kept keys above T and the keys equal to T
//      in the chunks before it (exclusive prefix sums), for emit.
// Past kResCandCap candidates (near-constant rows), C and D sweep the row
// instead of reading the list.  No part waits for another: the last one to
// arrive finishes the row, whenever the others ran.  A row of one part
// keeps its candidates and chunk counts in LDS (no publishing round trips).
// ---------------------------------------------------------------------------
constexpr int kResT = 1024;
constexpr int kResMaxParts = 8;
constexpr int kResPartMinChunks = 32;  // shorter rows are resolved by one workgroup (measured crossover)
constexpr int kRoundKeys = 4 * kResT;             // keys per sweep round: 4 per thread, 256 per wave
constexpr int kRoundsInFlight = 4;                // sweep rounds whose loads are issued together
constexpr int kResUnion = kBndLds > 2 * kResCandCap ? kBndLds : 2 * kResCandCap;
constexpr int kBndPer = kBndLds / kResT;          // boundary raw scores per thread (at most)
constexpr int kCntPer = kMaxChunks / kResT;       // chunk counters per thread (at most)
static_assert(kBins1 == 2 * kResT, "two top-digit histogram words per thread");
static_assert(kChunk % 256 == 0, "a wave's 256 keys of a round lie in one chunk");

__global__ void __launch_bounds__(kResT)
sel_resolve_kernel(const float* __restrict__ scores, int Lk, int ks, int window, int keep, int chunks, int parts,
                   int cpp, SplitGeom geom, SelWs ws) {
  __shared__ __attribute__((aligned(16))) uint32_t hist1[kBins1];
  __shared__ uint32_t hist2[kBins2];
  __shared__ uint32_t hist3[kBins3];
  __shared__ uint32_t gtc[kMaxChunks];  // per chunk: keys above b1, then kept keys above T
  __shared__ uint32_t eqc[kMaxChunks];  // per chunk: keys equal to T
  __shared__ __attribute__((aligned(16))) uint32_t un[kResUnion];  // boundary raw scores, then candidates
  __shared__ uint32_t small[128];  // scan partials [0, 32), bin / counts at 64.., max at 96.., flag at 112
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int row = blockIdx.x / parts, part = blockIdx.x % parts;
  const int c_begin = part * cpp, c_end = min(c_begin + cpp, chunks);
  const int kb = c_begin * kChunk, ke = min(c_end * kChunk, Lk);
  const int h = ks / 2;
  const int prot = Lk - window;
  uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  const float* srow = scores + (int64_t)row * Lk;
  float* prow = ws.pooled + (int64_t)row * Lk;

  // A. One round trip: the top-digit histogram and interior maximum, and the
  // raw scores [b-2h, b+2h) around each split boundary b = i*kps.
  const uint2 hv = reinterpret_cast<const uint2*>(rw + kRowHist1)[tid];
  const uint32_t rmax = rw[kRowMax];
  const int nb = geom.n_splits - 1;
  const int w4 = 4 * h, w2 = 2 * h;
  const int nbx = nb * w4;
  float bv[kBndPer];
#pragma unroll
  for (int i = 0; i < kBndPer; ++i) {
    if (i * kResT >= nbx) break;
    const int t = tid + i * kResT;
    bv[i] = -INFINITY;
    if (t < nbx) {
      const int u = (t / w4 + 1) * geom.kps - 2 * h + t % w4;
      if (u >= 0 && u < Lk) bv[i] = srow[u];
    }
  }
  const bool solo = parts == 1;
  for (int i = tid; i < cpp; i += kResT) gtc[i] = 0u;
  if (tid == 0) small[113] = 0u;  // candidates of a one-part row
  reinterpret_cast<uint2*>(hist1)[tid] = hv;
  float* bxs = reinterpret_cast<float*>(un);
#pragma unroll
  for (int i = 0; i < kBndPer; ++i) {
    if (i * kResT >= nbx) break;
    const int t = tid + i * kResT;
    if (t < nbx) bxs[t] = bv[i];
  }
  __syncthreads();
  uint32_t bmax = 0u;
  for (int t = tid; t < nb * w2; t += kResT) {
    const int bi = t / w2, k = t % w2;
    const int j = (bi + 1) * geom.kps - h + k;
    if (j < Lk) {
      const float* w = bxs + bi * w4 + k;
      float m = -INFINITY;
      for (int u = 0; u <= 2 * h; ++u) m = fmaxf(m, w[u]);
      const uint32_t key = float_key(m);
      bmax = max(bmax, key);
      if (j < prot) atomicAdd(&hist1[key >> kShift1], 1u);
      // read back by this part's sweep (after the barriers below), by the
      // last part's fallback sweep and by emit
      if (j >= kb && j < ke) st_dev(reinterpret_cast<uint32_t*>(prow + j), __float_as_uint(m));
    }
  }
  const uint32_t gmax = block_max_u32(max(bmax, rmax), small + 96);
  const uint32_t kbig = float_key(key_float(gmax) + 1.0f);
  if (tid == 0) hist1[kbig >> kShift1] += (uint32_t)window;
  __syncthreads();
  uint32_t* fb = small + 64;
  if (tid < 64) wave_find_bin<kBins1>(hist1, nullptr, (uint32_t)keep, fb);
  __syncthreads();
  const uint32_t b1 = fb[0];
  const uint32_t k1 = (uint32_t)keep - fb[1];

  // B. Sweep of [kb, ke): round r, wave w, lane l reads keys
  // r + 256w + 4l .. +3 (past Lk the loads return zeros, masked).  The
  // candidates of a batch of rounds take their slots with one atomic add per
  // wave on the row's counter.
  const rsrc_t prs = make_rsrc(prow, (uint32_t)Lk * 4u);
  uint2* gl = ws.cand + (int64_t)row * kResCandCap;
  uint2* cl = reinterpret_cast<uint2*>(un);  // the boundary raw scores are dead
  for (int r0 = kb; r0 < ke; r0 += kRoundsInFlight * kRoundKeys) {
    u32x4 x[kRoundsInFlight];
#pragma unroll
    for (int i = 0; i < kRoundsInFlight; ++i)
      x[i] = buf_load16(prs, (uint32_t)(r0 + i * kRoundKeys + 256 * wv + 4 * lane) * 4u);
    uint32_t nc = 0u;
#pragma unroll
    for (int i = 0; i < kRoundsInFlight; ++i) {
      const int base = r0 + i * kRoundKeys + 256 * wv;
      uint32_t na = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = base + 4 * lane + e;
        const uint32_t d = pooled_key(x[i][e], j, prot, kbig) >> kShift1;
        const bool valid = j < ke;
        na += (valid && d > b1) ? 1u : 0u;
        nc += (valid && d == b1) ? 1u : 0u;
      }
      const uint32_t s = wave_reduce_add(na);
      if (lane == 0 && base < ke && s) atomicAdd(&gtc[base / kChunk - c_begin], s);
    }
    const uint32_t incl = wave_incl_scan(nc);
    const uint32_t wtot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    uint32_t wbase = 0u;
    if (lane == 0 && wtot) wbase = solo ? atomicAdd(&small[113], wtot) : atomicAdd(rw + kRowNcand, wtot);
    wbase = (uint32_t)__builtin_amdgcn_readfirstlane((int)wbase);
    if (nc) {
      uint32_t pos = wbase + incl - nc;
#pragma unroll
      for (int i = 0; i < kRoundsInFlight; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = r0 + i * kRoundKeys + 256 * wv + 4 * lane + e;
          const uint32_t key = pooled_key(x[i][e], j, prot, kbig);
          if (j < ke && (key >> kShift1) == b1) {
            if (pos < (uint32_t)kResCandCap) {
              if (solo)
                cl[pos] = make_uint2(key, (uint32_t)j);
              else
                st_dev(reinterpret_cast<uint64_t*>(gl + pos), (uint64_t)key | ((uint64_t)(uint32_t)j << 32));
            }
            ++pos;
          }
        }
    }
  }
  __syncthreads();
  uint32_t ncand;
  if (solo) {
    ncand = small[113];
  } else {
    for (int c = c_begin + tid; c < c_end; c += kResT)
      st_dev(reinterpret_cast<uint32_t*>(ws.cnt + (int64_t)row * chunks + c), gtc[c - c_begin]);
    // Arrival: the stores above complete first; the last part continues.
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const bool last = atomicAdd(rw + kRowArrive, 1u) == (uint32_t)parts - 1u;
      if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      small[112] = last ? 1u : 0u;
    }
    __syncthreads();
    if (!small[112]) return;
    // The row's candidates and per-chunk counts, as the parts left them.
    ncand = __hip_atomic_load(rw + kRowNcand, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (ncand <= (uint32_t)kResCandCap)
      for (uint32_t p = tid; p < ncand; p += kResT) cl[p] = gl[p];
    for (int c = tid; c < chunks; c += kResT) gtc[c] = ws.cnt[(int64_t)row * chunks + c].x;
  }
  const bool in_lds = ncand <= (uint32_t)kResCandCap;
  for (int c = tid; c < chunks; c += kResT) eqc[c] = 0u;
  for (int i = tid; i < kBins2; i += kResT) hist2[i] = 0u;
  for (int i = tid; i < kBins3; i += kResT) hist3[i] = 0u;
  __syncthreads();

  // Every candidate (key, index): from the LDS list, or by sweeping the row.
  auto for_cands = [&](auto&& f) __attribute__((always_inline)) {
    if (in_lds) {
      for (uint32_t p = tid; p < ncand; p += kResT) {
        const uint2 cv = cl[p];
        f(cv.x, (int)cv.y);
      }
    } else {
      for (int j0 = 4 * tid; j0 < Lk; j0 += 4 * kResT) {
        const u32x4 xv = buf_load16(prs, (uint32_t)j0 * 4u);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = j0 + e;
          const uint32_t key = pooled_key(xv[e], j, prot, kbig);
          if (j < Lk && (key >> kShift1) == b1) f(key, j);
        }
      }
    }
  };

  // C. Digits 2 and 3.
  for_cands([&](uint32_t key, int) { atomicAdd(&hist2[(key >> kShift2) & (kBins2 - 1)], 1u); });
  __syncthreads();
  if (tid < 64) wave_find_bin<kBins2>(hist2, nullptr, k1, fb);
  __syncthreads();
  const uint32_t b2 = fb[0];
  const uint32_t k2 = k1 - fb[1];
  const uint32_t pre = (b1 << kBits2) | b2;
  for_cands([&](uint32_t key, int) {
    if ((key >> kShift2) == pre) atomicAdd(&hist3[key & (kBins3 - 1)], 1u);
  });
  __syncthreads();
  if (tid < 64) wave_find_bin<kBins3>(hist3, nullptr, k2, fb + 4);
  __syncthreads();
  const uint32_t T = (pre << kBits3) | fb[4];
  const uint32_t take_eq = k2 - fb[5];

  // D. Per-chunk counts, then their exclusive prefix sums for emit.
  for_cands([&](uint32_t key, int j) {
    if (key > T) atomicAdd(&gtc[j / kChunk], 1u);
    else if (key == T) atomicAdd(&eqc[j / kChunk], 1u);
  });
  __syncthreads();
  const int seg = (chunks + kResT - 1) / kResT;  // consecutive chunks per thread (<= kCntPer)
  uint32_t sg = 0u, se = 0u;
#pragma unroll
  for (int i = 0; i < kCntPer; ++i) {
    if (i >= seg) break;
    const int cc = tid * seg + i;
    if (cc < chunks) {
      sg += gtc[cc];
      se += eqc[cc];
    }
  }
  uint32_t pg, pe;
  block_excl_scan2<kResT>(sg, se, &pg, &pe, nullptr, nullptr, small);
  uint2* cnt = ws.cnt + (int64_t)row * chunks;
#pragma unroll
  for (int i = 0; i < kCntPer; ++i) {
    if (i >= seg) break;
    const int cc = tid * seg + i;
    if (cc < chunks) {
      cnt[cc] = make_uint2(pg, pe);
      pg += gtc[cc];
      pe += eqc[cc];
    }
  }
  if (tid == 0) {
    rw[kRowB1 + 0] = T;
    rw[kRowB1 + 1] = take_eq;
    rw[kRowB1 + 2] = gmax;
  }
}

// ---------------------------------------------------------------------------
// emit: grid = rows * chunks.  Thread t owns the kPer consecutive keys
// c*kChunk + kPer*t ..; the kept keys of the chunk are written in index
// order from the chunk's offsets (resolve), then (when ko is given) their
// K/V rows are copied.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kEmitT)
sel_emit_kernel(int Lk, int window, int keep, int chunks, SelWs ws, int64_t* __restrict__ out_idx,
                float* __restrict__ pooled_out, CompactArgs ca) {
  __shared__ uint32_t small[64];
  __shared__ int s_src[kChunk];
  __shared__ int s_dst[kChunk];
  const int tid = threadIdx.x;
  const int row = blockIdx.x / chunks;
  const int c = blockIdx.x % chunks;
  const uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  const float* pooled = ws.pooled + (int64_t)row * Lk;
  const int prot = Lk - window;

  // One round trip: this chunk's pooled values, its offsets and the row words.
  const int j0 = c * kChunk + kPer * tid;
  float pv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) pv[i] = (j0 + i < Lk) ? pooled[j0 + i] : 0.f;
  const uint2 off = ws.cnt[(int64_t)row * chunks + c];
  const uint32_t T = rw[kRowB1 + 0], take_eq = rw[kRowB1 + 1];
  const float big = key_float(rw[kRowB1 + 2]) + 1.0f;
  const uint32_t kbig = float_key(big);
  const uint32_t gt0 = off.x, eq0 = off.y;

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
  block_excl_scan2<kEmitT>(ng, ne, &pg, &pe, &tg, &te, small);
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
    constexpr int kG = 8;  // 16-byte units of K and of V in flight per thread
    for (int t0 = tid; t0 < total; t0 += kG * kEmitT) {
      u32x4 kv[kG], vv[kG];
#pragma unroll
      for (int q = 0; q < kG; ++q) {
        const int t = t0 + q * kEmitT;
        if (t < total) {
          const int64_t o = (int64_t)s_src[t / ca.units] * ca.sl + 16 * (t % ca.units);
          kv[q] = *reinterpret_cast<const u32x4*>(kb + o);
          vv[q] = *reinterpret_cast<const u32x4*>(vb + o);
        }
      }
#pragma unroll
      for (int q = 0; q < kG; ++q) {
        const int t = t0 + q * kEmitT;
        if (t < total) {
          const int64_t o = ((int64_t)row * ca.out_ld + s_dst[t / ca.units]) * ca.units * 16 + 16 * (t % ca.units);
          *reinterpret_cast<u32x4*>(ca.ko + o) = kv[q];
          *reinterpret_cast<u32x4*>(ca.vo + o) = vv[q];
        }
      }
    }
  }
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

CompactArgs compact_args(const SelectCompact* cp) {
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
    ca.out_ld = cp->out_ld;
  }
  return ca;
}

hipError_t launch_select_after_pool(const float* scores, int rows, int Lk, int ks, int window, int keep,
                                    int n_splits, int kps, int64_t* out_idx, float* pooled_out, char* ws_base,
                                    const SelectCompact* cp, hipStream_t st) {
  const SelWs ws = sel_layout(ws_base, rows, Lk, nullptr);
  const int chunks = (Lk + kChunk - 1) / kChunk;
  const dim3 grid((unsigned)(rows * chunks));
  // Rows of kResPartMinChunks chunks or more in up to kResMaxParts parts,
  // each a whole number of chunks; shorter rows in one.
  const int cpp = chunks < kResPartMinChunks ? chunks : (chunks + kResMaxParts - 1) / kResMaxParts;
  const int parts = (chunks + cpp - 1) / cpp;
  launch(sel_resolve_kernel, dim3((unsigned)(rows * parts)), dim3(kResT), 0, st, scores, Lk, ks, window, keep,
         chunks, parts, cpp, SplitGeom{n_splits, kps}, ws);
  launch(sel_emit_kernel, grid, dim3(kEmitT), 0, st, Lk, window, keep, chunks, ws, out_idx, pooled_out,
         compact_args(cp));
  return hipGetLastError();
}

hipError_t launch_select(const float* scores, int rows, int Lk, int ks, int window, int keep, int64_t* out_idx,
                         float* pooled_out, char* ws_base, bool pre_zeroed, const SelectCompact* cp,
                         hipStream_t st) {
  const SelWs ws = sel_layout(ws_base, rows, Lk, nullptr);
  const int chunks = (Lk + kChunk - 1) / kChunk;
  if (!pre_zeroed) {
    const int64_t zn = (int64_t)rows * kRowWords;
    launch(sel_zero_kernel, dim3((unsigned)std::min<int64_t>((zn + kSelT - 1) / kSelT, 1024)),
                       dim3(kSelT), 0, st, ws.rowws, zn);
  }
  const int h = ks / 2;
  if (h <= kMaxHalo) {
    launch(sel_pool_kernel, dim3((unsigned)(rows * chunks)), dim3(kSelT), 0, st, scores, Lk, ks, window, chunks, ws);
  } else {
    // Windows past the halo of sel_pool_kernel: block prefix / suffix maxima
    // first (in the tail's candidate regions, [rows][Lk + kScandPad] entries
    // of 8 bytes: room for both).  A window wider than the row pools like
    // one of 2*Lk+1 keys.
    const int hw = std::min(h, Lk);
    const int w = 2 * hw + 1;
    const int nblk = (Lk + w - 1) / w;
    float* pre = reinterpret_cast<float*>(ws.scand);
    float* suf = pre + (int64_t)rows * Lk;
    const int64_t waves = (int64_t)rows * nblk;
    launch(sel_pool_wide_scan_kernel, dim3((unsigned)((waves + kWideScanT / 64 - 1) / (kWideScanT / 64))),
           dim3(kWideScanT), 0, st, scores, rows, Lk, w, nblk, pre, suf);
    launch(sel_pool_wide_kernel, dim3((unsigned)(rows * chunks)), dim3(kSelT), 0, st, pre, suf, Lk, hw, window,
           chunks, ws);
  }
  return launch_select_after_pool(scores, rows, Lk, ks, window, keep, 1, Lk, out_idx, pooled_out, ws_base, cp, st);
}

bool select_after_pool_ok(int64_t n_splits, int64_t kps, int64_t Lk, int64_t ks) {
  const int64_t h = ks / 2;
  return h <= kMaxHalo && kps >= 2 * h && (Lk + kChunk - 1) / kChunk <= kMaxChunks && boundary_fits(n_splits, h);
}

}  // namespace dkv
