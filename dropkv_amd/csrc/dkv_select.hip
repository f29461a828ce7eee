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
// resolve: one workgroup per row.
//   A. Pools the keys next to the scoring pass's split boundaries (their
//      windows straddle two workgroup ranges), which completes the row's
//      top-digit histogram and maximum; finds the top-digit bin b1 of the
//      keep-th largest key.
//   B. One sweep over the pooled row: per chunk, the keys above b1; the keys
//      inside b1 (the candidates, a few percent of the row) into LDS.
//   C. Digits 2 and 3 over the candidates: the threshold key T and how many
//      keys equal to T are kept (the lowest indices).
//   D. Per chunk, the kept keys above T and the keys equal to T in the
//      chunks before it (exclusive prefix sums), for emit.
// Past kResCandCap candidates (near-constant rows), C and D sweep the row
// again instead of reading the list.
// ---------------------------------------------------------------------------
constexpr int kResT = 1024;
constexpr int kResWaves = kResT / 64;
constexpr int kWaveKeys = 2 * kChunk;              // keys per wave and sweep round: 8 x 4 per lane
constexpr int kRoundKeys = kResWaves * kWaveKeys;  // keys per sweep round
constexpr int kResCandCap = 4096;                  // candidates held in LDS as (key, index)
constexpr int kResUnion = kBndLds > 2 * kResCandCap ? kBndLds : 2 * kResCandCap;
constexpr int kBndPer = kBndLds / kResT;           // boundary raw scores per thread (at most)
constexpr int kCntPer = kMaxChunks / kResT;        // chunk counters per thread (at most)
static_assert(kBins1 == 2 * kResT, "two top-digit histogram words per thread");
static_assert(kWaveKeys == 2 * kChunk, "a wave's share of a round is two whole chunks");

// Sort key of a pooled value given as its bits (the buffer load's integer
// lanes), with the protected tail mapped to kbig.
__device__ __forceinline__ uint32_t pooled_key(uint32_t bits, int j, int prot, uint32_t kbig) {
  if (bits == 0x80000000u) bits = 0u;
  const uint32_t k = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return j >= prot ? kbig : k;
}

__global__ void __launch_bounds__(kResT)
sel_resolve_kernel(const float* __restrict__ scores, int Lk, int ks, int window, int keep, int chunks,
                   SplitGeom geom, SelWs ws) {
  __shared__ __attribute__((aligned(16))) uint32_t hist1[kBins1];
  __shared__ uint32_t hist2[kBins2];
  __shared__ uint32_t hist3[kBins3];
  __shared__ uint32_t gtc[kMaxChunks];  // per chunk: keys above b1, then kept keys above T
  __shared__ uint32_t eqc[kMaxChunks];  // per chunk: keys equal to T
  __shared__ float bpool[kBndPoolLds];
  __shared__ __attribute__((aligned(16))) uint32_t un[kResUnion];  // boundary raw scores, then candidates
  __shared__ uint32_t small[128];  // scan partials [0, 32), bin / counts at 64.., max at 96.., count at 112
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int row = blockIdx.x;
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
  for (int i = tid; i < chunks; i += kResT) eqc[i] = 0u;
  for (int i = tid; i < kBins2; i += kResT) hist2[i] = 0u;
  for (int i = tid; i < kBins3; i += kResT) hist3[i] = 0u;
  if (tid == 0) small[112] = 0u;
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
    float m = -INFINITY;
    if (j < Lk) {
      const float* w = bxs + bi * w4 + k;
      for (int u = 0; u <= 2 * h; ++u) m = fmaxf(m, w[u]);
      const uint32_t key = float_key(m);
      bmax = max(bmax, key);
      if (j < prot) atomicAdd(&hist1[key >> kShift1], 1u);
      prow[j] = m;  // read back by this workgroup's sweep (after the barriers below) and by emit
    }
    bpool[t] = m;
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

  // B. Sweep: wave w of round r reads keys r*kRoundKeys + w*kWaveKeys + ..,
  // lane l the 4-key groups l + 64 i; groups i < 4 lie in the wave's first
  // chunk, the rest in its second.  Past Lk the loads return zeros (masked).
  const rsrc_t prs = make_rsrc(prow, (uint32_t)Lk * 4u);
  uint2* cl = reinterpret_cast<uint2*>(un);
  for (int r0 = 0; r0 < Lk; r0 += kRoundKeys) {
    const int base = r0 + wv * kWaveKeys;
    if (base >= Lk) break;
    u32x4 x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = buf_load16(prs, (uint32_t)(base + 4 * (lane + 64 * i)) * 4u);
    uint32_t keys[8][4];
    uint32_t na0 = 0u, na1 = 0u, nc = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = base + 4 * (lane + 64 * i) + e;
        const uint32_t key = pooled_key(x[i][e], j, prot, kbig);
        keys[i][e] = key;
        const uint32_t d = key >> kShift1;
        const bool valid = j < Lk;
        const uint32_t above = (valid && d > b1) ? 1u : 0u;
        if (i < 4) na0 += above;
        else na1 += above;
        nc += (valid && d == b1) ? 1u : 0u;
      }
    const uint32_t s0 = wave_reduce_add(na0), s1 = wave_reduce_add(na1);
    const int c0 = base / kChunk;
    if (lane == 0) {
      gtc[c0] = s0;
      if (base + kChunk < Lk) gtc[c0 + 1] = s1;
    }
    // Candidate slots: a wave-wide exclusive scan of the lanes' counts and
    // one LDS atomic per wave.
    const uint32_t incl = wave_incl_scan(nc);
    const uint32_t wtot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    uint32_t wbase = 0u;
    if (lane == 0 && wtot) wbase = atomicAdd(&small[112], wtot);
    wbase = (uint32_t)__builtin_amdgcn_readfirstlane((int)wbase);
    if (nc) {
      uint32_t pos = wbase + incl - nc;
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = base + 4 * (lane + 64 * i) + e;
          if (j < Lk && (keys[i][e] >> kShift1) == b1) {
            if (pos < (uint32_t)kResCandCap) cl[pos] = make_uint2(keys[i][e], (uint32_t)j);
            ++pos;
          }
        }
    }
  }
  __syncthreads();
  const uint32_t ncand = small[112];
  const bool in_lds = ncand <= (uint32_t)kResCandCap;

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

__global__ void __launch_bounds__(kSelT)
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
  block_excl_scan2<kSelT>(ng, ne, &pg, &pe, &tg, &te, small);
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
          const int64_t o = (int64_t)s_src[t / ca.units] * ca.sl + 16 * (t % ca.units);
          kv[q] = *reinterpret_cast<const u32x4*>(kb + o);
          vv[q] = *reinterpret_cast<const u32x4*>(vb + o);
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
  launch(sel_resolve_kernel, dim3((unsigned)rows), dim3(kResT), 0, st, scores, Lk, ks, window, keep, chunks,
         SplitGeom{n_splits, kps}, ws);
  launch(sel_emit_kernel, grid, dim3(kSelT), 0, st, Lk, window, keep, chunks, ws, out_idx, pooled_out,
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
  launch(sel_pool_kernel, dim3((unsigned)(rows * chunks)), dim3(kSelT), 0, st, scores, Lk, ks, window,
                     chunks, ws);
  return launch_select_after_pool(scores, rows, Lk, ks, window, keep, 1, Lk, out_idx, pooled_out, ws_base, cp, st);
}

bool select_after_pool_ok(int64_t n_splits, int64_t kps, int64_t Lk, int64_t ks) {
  const int64_t h = ks / 2;
  return h <= kMaxHalo && kps >= 2 * h && (Lk + kChunk - 1) / kChunk <= kMaxChunks && boundary_fits(n_splits, h);
}

}  // namespace dkv
