// Decode step on the compressed cache: append the new token's K/V row and
// attend to every stored row (dropkv_cache.py:609-617 appends with torch.cat
// and the model then runs its attention over the concatenation).
//
// The cache lives in preallocated buffers [B, Hkv, C, D] whose first n rows
// are filled; n is read from device memory, so one captured launch serves
// every step of a decode loop (the caller advances n between steps).  The
// new row is not written before the attention: the workgroup that owns key n
// takes it from the k/v inputs and stores it, and no other workgroup reads
// row n in the same launch.
//
// Two kernels: split-key partials (online softmax per query head of the GQA
// group, one workgroup per (b, kv head, key split)) and a merge over the
// splits that writes the output in the [B, 1, Hq, D] layout of the
// attention's output.
#include "dkv_common.h"
#include "dkv_internal.h"

#include <algorithm>
#include <cmath>

namespace dkv {

constexpr int kDecMaxG = 16;      // query heads per KV head
constexpr int kDecKPL = 1;        // keys per lane per step (1: 64-key steps; 2 and 4 measured slower)
constexpr int kDecStep = 64 * kDecKPL;
constexpr int kDecMaxSplits = 64;

struct DecodeArgs {
  const void* q;  // [B, Hq, 1, D] element strides
  int64_t q_sb, q_sh, q_sd;
  const void* kn;  // new K/V rows [B, Hkv, 1, D] element strides
  const void* vn;
  int64_t n_sb, n_sh, n_sd;
  void* kbuf;  // [B, Hkv, C, D] contiguous
  void* vbuf;
  const int* n_rows;  // rows already stored (device)
  int B, Hq, Hkv, D, C, S;
  float scale_log2;
  float* part_m;  // [B*Hkv, S, g]
  float* part_l;
  float* part_o;  // [B*Hkv, S, g, D]
  void* out;      // [B, 1, Hq, D] element strides
  int64_t o_sb, o_sh, o_sd;
};

// One wave per (b, kv head, key split).  Each step covers 64 * kDecKPL keys:
// their K and V rows (contiguous in the cache buffer) are copied to LDS with 16-byte
// LDS-DMA loads (buffer view of the head's rows: rows past the buffer read as
// zeros), row n is then replaced by the new row, the lanes compute the G
// logits of kDecKPL keys each from LDS (q from LDS, G padded to a power of two
// with zero rows), one wave reduction per head gives the step maximum, p goes
// to LDS, and the lanes switch to head-dimension columns for P.V.
typedef __attribute__((address_space(3))) void lds_void_t;

template <typename T, int D, int G>
__global__ void __launch_bounds__(64) decode_partial_kernel(DecodeArgs a) {
  typedef typename Elem<T>::v8 v8;
  constexpr int DPL = D / 64;  // head-dim values per lane in the P.V phase
  constexpr int CPR = D / 8;   // 16-byte chunks per row
  constexpr int kRowBytes = D * (int)sizeof(T);
  constexpr int kStepBytes = kDecStep * kRowBytes;
  const int bh = blockIdx.x / a.S, split = blockIdx.x % a.S;
  const int b = bh / a.Hkv, hkv = bh % a.Hkv;
  const int g = a.Hq / a.Hkv;
  const int lane = threadIdx.x;

  __shared__ __attribute__((aligned(16))) float qs[D][G];  // q transposed: one float4 read serves 4 heads
  __shared__ __attribute__((aligned(16))) float pb[kDecStep][G];
  __shared__ __attribute__((aligned(16))) unsigned char ks_bytes[kStepBytes];
  __shared__ __attribute__((aligned(16))) unsigned char vs_bytes[kStepBytes];
  const T* ks = reinterpret_cast<const T*>(ks_bytes);
  T* vs = reinterpret_cast<T*>(vs_bytes);

  const T* q = static_cast<const T*>(a.q);
  for (int i = lane; i < G * D; i += 64) {
    const int h = i / D, d = i % D;
    qs[d][h] = h < g ? static_cast<float>(
                           q[(int64_t)b * a.q_sb + (int64_t)(hkv * g + h) * a.q_sh + (int64_t)d * a.q_sd])
                     : 0.f;
  }
  const T* kn = static_cast<const T*>(a.kn) + (int64_t)b * a.n_sb + (int64_t)hkv * a.n_sh;
  const T* vn = static_cast<const T*>(a.vn) + (int64_t)b * a.n_sb + (int64_t)hkv * a.n_sh;

  const int n = min(*a.n_rows, a.C - 1);  // the host keeps n < C; the clamp keeps every access in bounds
  const int nkeys = n + 1;
  const int kps = (nkeys + a.S - 1) / a.S;
  const int k0 = split * kps, k1 = min(k0 + kps, nkeys);

  T* kb = static_cast<T*>(a.kbuf) + (int64_t)bh * a.C * D;
  T* vb = static_cast<T*>(a.vbuf) + (int64_t)bh * a.C * D;
  const uint32_t head_bytes = (uint32_t)a.C * kRowBytes;
  const rsrc_t krs = make_rsrc(kb, head_bytes), vrs = make_rsrc(vb, head_bytes);
  if (k0 <= n && n < k1)  // this split owns key n: store the new row
    for (int d = lane; d < D; d += 64) {
      kb[(int64_t)n * D + d] = kn[(int64_t)d * a.n_sd];
      vb[(int64_t)n * D + d] = vn[(int64_t)d * a.n_sd];
    }

  float m[G], lp[G], o[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    lp[h] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[h][e] = 0.f;
  }

  for (int j0 = k0; j0 < k1; j0 += kDecStep) {
    // K and V rows j0 .. j0 + kDecStep - 1 to LDS (1 KB per instruction per wave).
    // The previous step's LDS reads must be done before the DMA writes land.
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const uint32_t src = (uint32_t)j0 * kRowBytes + 16u * lane;
#pragma unroll 8
    for (int it = 0; it < kStepBytes / 1024; ++it) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_t*)(ks_bytes + 1024 * it), 16, src + 1024u * it, 0, 0,
                                               0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_t*)(vs_bytes + 1024 * it), 16, src + 1024u * it, 0, 0,
                                               0);
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (n >= j0 && n < j0 + kDecStep)  // row n from the new row (its store above may not be visible yet)
      for (int d = lane; d < D; d += 64) {
        reinterpret_cast<T*>(ks_bytes)[(n - j0) * D + d] = kn[(int64_t)d * a.n_sd];
        vs[(n - j0) * D + d] = vn[(int64_t)d * a.n_sd];
      }
    __builtin_amdgcn_wave_barrier();
    // Logits of the lane's keys j0 + lane + 64u, scaled, to pb.
#pragma unroll 1
    for (int u = 0; u < kDecKPL; ++u) {
      const int r = lane + 64 * u;
      float x[G];
#pragma unroll
      for (int h = 0; h < G; ++h) x[h] = 0.f;
#pragma unroll
      for (int c = 0; c < CPR; ++c) {
        const v8 kv8 = bitcast_u4<v8>(*reinterpret_cast<const u32x4*>(ks + r * D + 8 * c));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 8 * c + e;
          const float kv = static_cast<float>(kv8[e]);
          if constexpr (G >= 4) {
#pragma unroll
            for (int h4 = 0; h4 < G; h4 += 4) {
              const float4 qv = *reinterpret_cast<const float4*>(&qs[d][h4]);
              x[h4 + 0] += qv.x * kv;
              x[h4 + 1] += qv.y * kv;
              x[h4 + 2] += qv.z * kv;
              x[h4 + 3] += qv.w * kv;
            }
          } else {
#pragma unroll
            for (int h = 0; h < G; ++h) x[h] += qs[d][h] * kv;
          }
        }
      }
      const bool valid = j0 + r < k1;
#pragma unroll
      for (int h = 0; h < G; ++h) pb[r][h] = valid ? x[h] * a.scale_log2 : -INFINITY;
    }
    __builtin_amdgcn_wave_barrier();
    // Online softmax per head over the step; p replaces the logits in pb.
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float xu[kDecKPL];
      float bm = -INFINITY;
#pragma unroll
      for (int u = 0; u < kDecKPL; ++u) {
        xu[u] = pb[lane + 64 * u][h];
        bm = fmaxf(bm, xu[u]);
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) bm = fmaxf(bm, __shfl_xor(bm, off));
      const float mn = fmaxf(m[h], bm);
      const float alpha = m[h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[h] - mn);
      float ps = 0.f;
#pragma unroll
      for (int u = 0; u < kDecKPL; ++u) {
        const float p = xu[u] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(xu[u] - mn);
        ps += p;
        pb[lane + 64 * u][h] = p;
      }
      lp[h] = lp[h] * alpha + ps;
#pragma unroll
      for (int e = 0; e < DPL; ++e) o[h][e] *= alpha;
      m[h] = mn;
    }
    __builtin_amdgcn_wave_barrier();
    // P.V with lanes over the head dimension.
    const int nb = min(kDecStep, k1 - j0);
    for (int jj = 0; jj < nb; ++jj) {
      float vv[DPL];
#pragma unroll
      for (int e = 0; e < DPL; ++e) vv[e] = static_cast<float>(vs[jj * D + lane * DPL + e]);
      if constexpr (G >= 4) {
#pragma unroll
        for (int h4 = 0; h4 < G; h4 += 4) {
          const float4 p4 = *reinterpret_cast<const float4*>(&pb[jj][h4]);
#pragma unroll
          for (int e = 0; e < DPL; ++e) {
            o[h4 + 0][e] += p4.x * vv[e];
            o[h4 + 1][e] += p4.y * vv[e];
            o[h4 + 2][e] += p4.z * vv[e];
            o[h4 + 3][e] += p4.w * vv[e];
          }
        }
      } else {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int e = 0; e < DPL; ++e) o[h][e] += pb[jj][h] * vv[e];
      }
    }
  }

  // The split's partials (heads h < g).
  const int64_t base = ((int64_t)bh * a.S + split) * g;
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float l = lp[h];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
    if (h < g) {
#pragma unroll
      for (int e = 0; e < DPL; ++e) a.part_o[(base + h) * D + lane * DPL + e] = o[h][e];
      if (lane == 0) {
        a.part_m[base + h] = m[h];
        a.part_l[base + h] = l;
      }
    }
  }
}

// One wave per query head: combine the splits and write the output row.
// Lane s holds split s's (m, l); the partial outputs are read in batches of
// 16 splits with every load of a batch in flight.
template <typename T, int D>
__global__ void __launch_bounds__(64) decode_merge_kernel(DecodeArgs a) {
  constexpr int DPL = D / 64;
  constexpr int kBatch = 16;
  const int g = a.Hq / a.Hkv;
  const int b = blockIdx.x / a.Hq, hq = blockIdx.x % a.Hq;
  const int hkv = hq / g, h = hq % g;
  const int lane = threadIdx.x;
  const int64_t base = ((int64_t)(b * a.Hkv + hkv) * a.S) * g + h;
  const float ml = lane < a.S ? a.part_m[base + (int64_t)lane * g] : -INFINITY;
  const float ll = lane < a.S ? a.part_l[base + (int64_t)lane * g] : 0.f;
  float mx = ml;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  const float f = ml == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml - mx);
  float l = ll * f;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off);
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < a.S; s0 += kBatch) {
    float ob[kBatch][DPL];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
#pragma unroll
      for (int e = 0; e < DPL; ++e)
        ob[u][e] = s0 + u < a.S ? a.part_o[(base + (int64_t)(s0 + u) * g) * D + lane * DPL + e] : 0.f;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float fs = __shfl(f, (s0 + u) & 63);
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[e] += s0 + u < a.S ? fs * ob[u][e] : 0.f;
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* out = static_cast<T*>(a.out);
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane * DPL + e;
    out[(int64_t)b * a.o_sb + (int64_t)hq * a.o_sh + (int64_t)d * a.o_sd] = static_cast<T>(acc[e] * inv);
  }
}

int decode_splits(int C) { return std::max(1, std::min(kDecMaxSplits, (C + kDecStep - 1) / kDecStep)); }

size_t decode_workspace_bytes(int B, int Hq, int Hkv, int D, int C) {
  const size_t S = (size_t)decode_splits(C);
  const size_t rows = (size_t)B * Hkv * S * (Hq / Hkv);
  return rows * sizeof(float) * (2 + (size_t)D) + 256;
}

template <typename T, int D>
static hipError_t launch_decode_t(DecodeArgs a, hipStream_t st) {
  const int g = a.Hq / a.Hkv;
  if (g < 1 || g > kDecMaxG) return hipErrorInvalidValue;
  const dim3 grid(a.B * a.Hkv * a.S);
  if (g <= 1)
    launch((decode_partial_kernel<T, D, 1>), grid, dim3(64), 0, st, a);
  else if (g <= 2)
    launch((decode_partial_kernel<T, D, 2>), grid, dim3(64), 0, st, a);
  else if (g <= 4)
    launch((decode_partial_kernel<T, D, 4>), grid, dim3(64), 0, st, a);
  else if (g <= 8)
    launch((decode_partial_kernel<T, D, 8>), grid, dim3(64), 0, st, a);
  else
    launch((decode_partial_kernel<T, D, 16>), grid, dim3(64), 0, st, a);
  launch((decode_merge_kernel<T, D>), dim3(a.B * a.Hq), dim3(64), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_decode_attention(const DecodeParams& p, hipStream_t st) {
  DecodeArgs a;
  a.q = p.q;
  a.q_sb = p.q_sb;
  a.q_sh = p.q_sh;
  a.q_sd = p.q_sd;
  a.kn = p.kn;
  a.vn = p.vn;
  a.n_sb = p.n_sb;
  a.n_sh = p.n_sh;
  a.n_sd = p.n_sd;
  a.kbuf = p.kbuf;
  a.vbuf = p.vbuf;
  a.n_rows = p.n_rows;
  a.B = p.B;
  a.Hq = p.Hq;
  a.Hkv = p.Hkv;
  a.D = p.D;
  a.C = p.C;
  a.S = decode_splits(p.C);
  a.scale_log2 = p.scale * 1.4426950408889634f;
  const size_t rows = (size_t)p.B * p.Hkv * a.S * (p.Hq / p.Hkv);
  char* ws = static_cast<char*>(p.workspace);
  a.part_m = reinterpret_cast<float*>(ws);
  a.part_l = a.part_m + rows;
  a.part_o = a.part_l + rows;
  a.out = p.out;
  a.o_sb = p.o_sb;
  a.o_sh = p.o_sh;
  a.o_sd = p.o_sd;
  if (p.dtype_bf16) {
    if (p.D == 64) return launch_decode_t<__bf16, 64>(a, st);
    return launch_decode_t<__bf16, 128>(a, st);
  }
  if (p.D == 64) return launch_decode_t<_Float16, 64>(a, st);
  return launch_decode_t<_Float16, 128>(a, st);
}

}  // namespace dkv
