// Pool / protect / top-k / ascending sort of the DropKV scores on gfx950 (the
// selection half of DropKVCache._compute_keep_indices, dropkv_cache.py:464-475),
// optionally fused with the gather into the compressed cache
// (DropKVCache._gather_compressed, dropkv_cache.py:479-491).  The stages are
// described in dkv_select_dev.h.
//
// Standalone (dropkv_select): zero -> pool -> cand -> emit.
// After a scoring pass that pooled its interiors (dropkv_evict): cand -> emit.
#include "dkv_common.h"
#include "dkv_internal.h"
#include "dkv_select_dev.h"

#include <algorithm>

namespace dkv {

constexpr int kSelT = 1024;           // threads per workgroup, all stages
constexpr int kPer = kChunk / kSelT;  // keys per thread

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
// cand: grid = rows * chunks.
// ---------------------------------------------------------------------------
constexpr int kBndPer = kBndLds / kSelT;  // boundary raw scores per thread (at most)

__global__ void __launch_bounds__(kSelT)
sel_cand_kernel(const float* __restrict__ scores, int Lk, int ks, int window, int keep, int chunks, SplitGeom geom,
                SelWs ws) {
  __shared__ __attribute__((aligned(16))) uint32_t hist[kBins1];
  __shared__ float bxs[kBndLds];
  __shared__ float bpool[kBndPoolLds];
  __shared__ uint32_t small[128];  // scan partials [0, 32), bin / counts at 64.., max at 96..
  const int tid = threadIdx.x;
  const int row = blockIdx.x / chunks;
  const int c = blockIdx.x % chunks;
  const int h = ks / 2;
  const int prot = Lk - window;
  uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  const float* srow = scores + (int64_t)row * Lk;
  float* prow = ws.pooled + (int64_t)row * Lk;
  uint32_t* wsum = small;

  // One round trip: this chunk's pooled values (complete except the boundary
  // keys), the row's top-digit histogram and interior maximum, and the raw
  // scores [b-2h, b+2h) around each split boundary b = i*kps (1 <= i < n_splits).
  float cv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = c * kChunk + tid + i * kSelT;
    cv[i] = j < Lk ? prow[j] : 0.f;
  }
  static_assert(kBins1 == 2 * kSelT, "two histogram words per thread");
  const uint2 hv = reinterpret_cast<const uint2*>(rw + kRowHist1)[tid];
  const uint32_t rmax = rw[kRowMax];
  const int nb = geom.n_splits - 1;
  const int w4 = 4 * h, w2 = 2 * h;
  const int nbx = nb * w4;
  float bv[kBndPer];
#pragma unroll
  for (int i = 0; i < kBndPer; ++i) {
    if (i * kSelT >= nbx) break;
    const int t = tid + i * kSelT;
    bv[i] = -INFINITY;
    if (t < nbx) {
      const int u = (t / w4 + 1) * geom.kps - 2 * h + t % w4;
      if (u >= 0 && u < Lk) bv[i] = srow[u];
    }
  }
  reinterpret_cast<uint2*>(hist)[tid] = hv;
#pragma unroll
  for (int i = 0; i < kBndPer; ++i) {
    if (i * kSelT >= nbx) break;
    const int t = tid + i * kSelT;
    if (t < nbx) bxs[t] = bv[i];
  }
  __syncthreads();

  // The boundary keys' windows, read from LDS; they complete the histogram.
  uint32_t bmax = 0u;
  for (int t = tid; t < nb * w2; t += kSelT) {
    const int bi = t / w2, k = t % w2;
    const int j = (bi + 1) * geom.kps - h + k;
    float m = -INFINITY;
    if (j < Lk) {
      const float* w = bxs + bi * w4 + k;
      for (int u = 0; u <= 2 * h; ++u) m = fmaxf(m, w[u]);
      const uint32_t key = float_key(m);
      bmax = max(bmax, key);
      if (j < prot) atomicAdd(&hist[key >> kShift1], 1u);
    }
    bpool[t] = m;
  }
  const uint32_t gmax = block_max_u32(max(bmax, rmax), small + 96);
  const uint32_t kbig = float_key(key_float(gmax) + 1.0f);
  if (tid == 0) hist[kbig >> kShift1] += (uint32_t)window;
  __syncthreads();
  uint32_t* fb = small + 64;  // wave_find_bin result
  if (tid < 64) wave_find_bin<kBins1>(hist, nullptr, (uint32_t)keep, fb);
  __syncthreads();
  const uint32_t b1 = fb[0];
  const uint32_t k1 = (uint32_t)keep - fb[1];

  // This chunk: the count above b1 and the candidates (keys in b1), which go
  // to the chunk's own region of the candidate arrays.  Boundary keys take
  // their value from bpool and are written to the pooled row here.
  uint32_t keys[kPer];
  uint32_t nab = 0u, ncand = 0u;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = c * kChunk + tid + i * kSelT;
    keys[i] = 0u;
    if (j < Lk) {
      float v = cv[i];
      const int bi = (j + h) / geom.kps;
      const int off = j + h - bi * geom.kps;
      if (bi >= 1 && bi <= nb && off < w2) {
        v = bpool[(bi - 1) * w2 + off];
        prow[j] = v;
      }
      keys[i] = j >= prot ? kbig : float_key(v);
      const uint32_t d = keys[i] >> kShift1;
      nab += d > b1 ? 1u : 0u;
      ncand += d == b1 ? 1u : 0u;
    }
  }
  uint32_t pc, dummy, tot_c, tot_ab;
  block_excl_scan2<kSelT>(ncand, nab, &pc, &dummy, &tot_c, &tot_ab, wsum);
  uint32_t pos = (uint32_t)c * kChunk + pc;
  uint32_t* ckey = ws.cand_key + (int64_t)row * Lk;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int j = c * kChunk + tid + i * kSelT;
    if (j < Lk && (keys[i] >> kShift1) == b1) {
      ckey[pos] = keys[i];
      ++pos;
    }
  }
  if (tid == 0) {
    ws.cnt[(int64_t)row * chunks + c] = make_uint2(tot_ab, tot_c);
    if (c == 0) {
      rw[kRowB1 + 0] = b1;
      rw[kRowB1 + 1] = k1;
      rw[kRowB1 + 2] = gmax;
    }
  }
}

// ---------------------------------------------------------------------------
// emit: grid = rows * chunks.  Gathers the row's candidates into LDS and
// resolves T from them, then thread t owns the kPer consecutive keys
// c*kChunk + kPer*t ..; kept keys are written in index order, then (when ko
// is given) their K/V rows are copied.
// ---------------------------------------------------------------------------
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

constexpr int kEmitCandLds = 4096;                  // candidates held in LDS (more: read from global)
constexpr int kSpecPer = kEmitCandLds / (4 * kSelT);  // speculative 4-candidate groups per thread
constexpr int kCntPer = kMaxChunks / kSelT;           // chunk counts per thread (at most)
constexpr int kSpecMax = 128;                         // speculative candidates per chunk region (at most)

// Candidate p of the row's list (chunk-major) when it is not in LDS: chunk
// by binary search over the exclusive prefix counts s_pref[0..chunks].
__device__ __forceinline__ uint32_t cand_global(const uint32_t* s_pref, int chunks, const uint32_t* gkey,
                                                uint32_t p) {
  int lo = 0, hi = chunks - 1;  // last chunk with s_pref[cc] <= p
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= p) lo = mid;
    else hi = mid - 1;
  }
  const int64_t at = (int64_t)lo * kChunk + (p - s_pref[lo]);
  return gkey[at];
}

__global__ void __launch_bounds__(kSelT)
sel_emit_kernel(int Lk, int window, int keep, int chunks, int spec, SelWs ws, int64_t* __restrict__ out_idx,
                float* __restrict__ pooled_out, CompactArgs ca) {
  __shared__ uint32_t hist[kBins2 + kBins3];  // digit-2 and digit-3 histograms
  __shared__ uint32_t small[128];  // scan partials [0, 32), bin / counts at 64.., max at 96..
  __shared__ uint32_t lkey[kEmitCandLds];
  __shared__ uint32_t s_pref[kMaxChunks + 1];
  __shared__ int s_src[kChunk];
  __shared__ int s_dst[kChunk];
  const int tid = threadIdx.x;
  const int row = blockIdx.x / chunks;
  const int c = blockIdx.x % chunks;
  uint32_t* wsum = small;
  const uint32_t* rw = ws.rowws + (int64_t)row * kRowWords;
  const float* pooled = ws.pooled + (int64_t)row * Lk;
  const uint32_t* gkey = ws.cand_key + (int64_t)row * Lk;
  const uint2* cnt = ws.cnt + (int64_t)row * chunks;
  const int prot = Lk - window;

  // One round trip: the row words, this chunk's pooled values, every chunk's
  // counts and, speculatively, the first `spec` candidates (a multiple of 4)
  // of the first ncov = kEmitCandLds / spec chunk regions.
  const int j0 = c * kChunk + kPer * tid;
  float pv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) pv[i] = (j0 + i < Lk) ? pooled[j0 + i] : 0.f;
  const uint32_t b1 = rw[kRowB1 + 0], k1 = rw[kRowB1 + 1];
  const float big = key_float(rw[kRowB1 + 2]) + 1.0f;
  const uint32_t kbig = float_key(big);
  const int seg = (chunks + kSelT - 1) / kSelT;  // chunk counts owned by each thread (<= kCntPer)
  uint2 cv[kCntPer];
#pragma unroll
  for (int i = 0; i < kCntPer; ++i) {
    if (i >= seg) break;
    const int cc = tid * seg + i;
    cv[i] = cc < chunks ? cnt[cc] : make_uint2(0u, 0u);
  }
  uint4 sk[kSpecPer];
  const int nspec = min(chunks * spec, kEmitCandLds);
#pragma unroll
  for (int i = 0; i < kSpecPer; ++i) {
    if (4 * i * kSelT >= nspec) break;
    const int e = 4 * (tid + i * kSelT);
    const int cc = e / spec, off = e - cc * spec;
    const int64_t at = (int64_t)cc * kChunk + off;
    if (cc < chunks && at + 4 <= Lk) {
      sk[i] = *reinterpret_cast<const uint4*>(gkey + at);
    } else {
      sk[i] = make_uint4(0u, 0u, 0u, 0u);
    }
  }

  // Candidate counts -> exclusive prefix s_pref (chunk-major list order);
  // above-b1 keys of the chunks before this one.
  const int ncov = kEmitCandLds / spec;
  uint32_t tsum = 0u, g = 0u, e = 0u;
  bool overflow = false;
#pragma unroll
  for (int i = 0; i < kCntPer; ++i) {
    if (i >= seg) break;
    const int cc = tid * seg + i;
    if (cc < chunks) {
      tsum += cv[i].y;
      if (cc < c) g += cv[i].x;
      overflow |= cv[i].y > (cc < ncov ? (uint32_t)spec : 0u);
    }
  }
  uint32_t run, dummy, nc;
  block_excl_scan2<kSelT>(tsum, 0u, &run, &dummy, &nc, nullptr, wsum);
#pragma unroll
  for (int i = 0; i < kCntPer; ++i) {
    if (i >= seg) break;
    const int cc = tid * seg + i;
    if (cc < chunks) {
      s_pref[cc] = run;
      run += cv[i].y;
    }
  }
  if (tid == 0) s_pref[chunks] = nc;
  const bool any_overflow = __syncthreads_or(overflow);
  const bool in_lds = nc <= (uint32_t)kEmitCandLds;

  // Candidates into LDS: the speculative ones, then (rarely) the rest of any
  // region longer than spec.
  if (in_lds) {
#pragma unroll
    for (int i = 0; i < kSpecPer; ++i) {
      if (4 * i * kSelT >= nspec) break;
      const int e4 = 4 * (tid + i * kSelT);
      const int cc = e4 / spec, off = e4 - cc * spec;
      if (cc < chunks) {
        const uint32_t n = s_pref[cc + 1] - s_pref[cc];
        const uint32_t kk[4] = {sk[i].x, sk[i].y, sk[i].z, sk[i].w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if ((uint32_t)(off + q) < n) {
            lkey[s_pref[cc] + off + q] = kk[q];
          }
      }
    }
    if (any_overflow) {
      // Every list entry not covered by the speculative loads, 8 loads in
      // flight per thread.
      for (uint32_t p0 = tid; p0 < nc; p0 += 8 * kSelT) {
        uint32_t kv[8];
        int32_t dst[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t p = p0 + q * kSelT;
          dst[q] = -1;
          if (p < nc) {
            int lo = 0, hi = chunks - 1;  // chunk of entry p
            while (lo < hi) {
              const int mid = (lo + hi + 1) >> 1;
              if (s_pref[mid] <= p) lo = mid;
              else hi = mid - 1;
            }
            const uint32_t o = p - s_pref[lo];
            if (o >= (lo < ncov ? (uint32_t)spec : 0u)) {
              kv[q] = gkey[(int64_t)lo * kChunk + o];
              dst[q] = (int32_t)p;
            }
          }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (dst[q] >= 0) lkey[dst[q]] = kv[q];
      }
    }
  }
  uint32_t* hist2 = hist;
  uint32_t* hist3 = hist + kBins2;
  for (int i = tid; i < kBins2 + kBins3; i += kSelT) hist[i] = 0u;
  __syncthreads();

  // Digit 2 (every candidate is in bin b1); the bin searches run on one wave.
  uint32_t* fb = small + 64;
  for (uint32_t p = tid; p < nc; p += kSelT) {
    uint32_t kv;
    if (in_lds) kv = lkey[p];
    else kv = cand_global(s_pref, chunks, gkey, p);
    atomicAdd(&hist2[(kv >> kShift2) & (kBins2 - 1)], 1u);
  }
  __syncthreads();
  if (tid < 64) wave_find_bin<kBins2>(hist2, nullptr, k1, fb);
  __syncthreads();
  const uint32_t b2 = fb[0];
  const uint32_t k2 = k1 - fb[1];
  const uint32_t pre = (b1 << kBits2) | b2;
  // Digit 3 over the candidates matching the first two digits.
  for (uint32_t p = tid; p < nc; p += kSelT) {
    uint32_t kv;
    if (in_lds) kv = lkey[p];
    else kv = cand_global(s_pref, chunks, gkey, p);
    if ((kv >> kShift2) == pre) atomicAdd(&hist3[kv & (kBins3 - 1)], 1u);
  }
  __syncthreads();
  if (tid < 64) wave_find_bin<kBins3>(hist3, nullptr, k2, fb + 4);
  __syncthreads();
  const uint32_t T = (pre << kBits3) | fb[4];
  const uint32_t take_eq = k2 - fb[5];

  // Output offsets of this chunk: kept keys > T and keys == T in earlier
  // chunks (above-b1 keys per chunk, plus the candidates of those chunks,
  // which are list entries [0, s_pref[c])).
  const uint32_t lim = s_pref[c];
  for (uint32_t p = tid; p < lim; p += kSelT) {
    uint32_t kv;
    if (in_lds) kv = lkey[p];
    else kv = cand_global(s_pref, chunks, gkey, p);
    g += kv > T ? 1u : 0u;
    e += kv == T ? 1u : 0u;
  }
  uint32_t gt0, eq0;
  block_sum2<kSelT>(g, e, &gt0, &eq0, wsum);

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
  block_excl_scan2<kSelT>(ng, ne, &pg, &pe, &tg, &te, wsum);
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
    for (int t0 = tid; t0 < total; t0 += kG * kSelT) {
      u32x4 kv[kG], vv[kG];
#pragma unroll
      for (int q = 0; q < kG; ++q) {
        const int t = t0 + q * kSelT;
        if (t < total) {
          const int64_t off = (int64_t)s_src[t / ca.units] * ca.sl + 16 * (t % ca.units);
          kv[q] = *reinterpret_cast<const u32x4*>(kb + off);
          vv[q] = *reinterpret_cast<const u32x4*>(vb + off);
        }
      }
#pragma unroll
      for (int q = 0; q < kG; ++q) {
        const int t = t0 + q * kSelT;
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

static CompactArgs compact_args(const SelectCompact* cp) {
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
  launch(sel_cand_kernel, grid, dim3(kSelT), 0, st, scores, Lk, ks, window, keep, chunks,
                     SplitGeom{n_splits, kps}, ws);
  // Speculative candidates per chunk region: a multiple of 4, at least 4,
  // chunks * spec <= kEmitCandLds.
  const int spec = std::max(4, std::min(kSpecMax, kEmitCandLds / chunks) & ~3);
  launch(sel_emit_kernel, grid, dim3(kSelT), 0, st, Lk, window, keep, chunks, spec, ws, out_idx,
                     pooled_out, compact_args(cp));
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
  launch(sel_pool_kernel, dim3((unsigned)(rows * chunks)), dim3(kSelT), 0, st, scores, Lk, ks, window,
                     chunks, ws);
  return launch_select_after_pool(scores, rows, Lk, ks, window, keep, 1, Lk, out_idx, pooled_out, ws_base, cp, st);
}

bool select_after_pool_ok(int64_t n_splits, int64_t kps, int64_t Lk, int64_t ks) {
  const int64_t h = ks / 2;
  return h <= kMaxHalo && kps >= 2 * h && (Lk + kChunk - 1) / kChunk <= kMaxChunks && boundary_fits(n_splits, h);
}

}  // namespace dkv
