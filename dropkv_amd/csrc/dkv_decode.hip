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

constexpr int kDecMaxG = 16;      // query heads per KV head: the 16 columns of the MFMA tiles
constexpr int kDecStep = 64;      // keys per step of a split
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
  int kps;  // rows of the buffer per split: ceil(C / S)
  float scale_log2;
  float* part_m;  // [B*Hkv, S, g]
  float* part_l;
  float* part_o;  // [B*Hkv, S, g, D]
  void* out;      // [B, 1, Hq, D] element strides
  int64_t o_sb, o_sh, o_sd;
};

// One wave per (b, kv head, key split).  Split s owns buffer rows
// [s * kps, (s + 1) * kps) whatever the row count, so its first step's loads
// are issued before the count has arrived; rows past the new row n are
// masked (splits past n write empty partials).  The new row is loaded into
// registers with the first step, put into LDS in place of row n, and stored
// into the buffer only after the attention, so that no wave waits on it.
// Each step covers 64 keys: their K and V rows (contiguous in the cache
// buffer) are copied to LDS with 16-byte LDS-DMA loads (buffer view of the
// head's rows: rows past the buffer read as zeros).  Both products run on
// the matrix cores with the group's query heads as the 16 columns (heads
// past the group are zero): S^T = K Q^T per 16-key block, and
// O^T += V^T P^T per 32 keys, V read transposed from LDS and P in two parts
// (hi and the rounded remainder, ~16 significant bits).  Lane (li, lg) holds
// head li's logits of keys 16 kb + 4 lg + r and its outputs at columns
// 16 dt + 4 lg + r; a head's maximum and sum combine its four lanes.
typedef __attribute__((address_space(3))) void lds_void_t;

template <typename T, int D>
__global__ void __launch_bounds__(64) decode_partial_kernel(DecodeArgs a) {
  typedef typename Elem<T>::v8 v8;
  constexpr int KK = D / 32;   // k-steps of the logits
  constexpr int DT = D / 16;   // 16-column blocks of the output
  constexpr int DPL = D / 64;  // elements of the new row per lane
  constexpr int kRowBytes = D * (int)sizeof(T);
  constexpr int kStepBytes = kDecStep * kRowBytes;
  static_assert(kDecStep == 64, "four 16-key blocks per step");
  const int bh = blockIdx.x / a.S, split = blockIdx.x % a.S;
  const int b = bh / a.Hkv, hkv = bh % a.Hkv;
  const int g = a.Hq / a.Hkv;
  const int lane = threadIdx.x;
  const int li = lane & 15, lg = lane >> 4;

  __shared__ __attribute__((aligned(16))) unsigned char ks_bytes[kStepBytes];
  __shared__ __attribute__((aligned(16))) unsigned char vs_bytes[kStepBytes];
  T* ks = reinterpret_cast<T*>(ks_bytes);
  T* vs = reinterpret_cast<T*>(vs_bytes);

  T* kb = static_cast<T*>(a.kbuf) + (int64_t)bh * a.C * D;
  T* vb = static_cast<T*>(a.vbuf) + (int64_t)bh * a.C * D;
  const uint32_t head_bytes = (uint32_t)a.C * kRowBytes;
  const rsrc_t krs = make_rsrc(kb, head_bytes), vrs = make_rsrc(vb, head_bytes);
  // K and V rows j0 .. j0 + kDecStep - 1 to LDS (1 KB per instruction per wave).
  auto issue_step = [&](int j0) __attribute__((always_inline)) {
    const uint32_t src = (uint32_t)j0 * kRowBytes + 16u * lane;
#pragma unroll 8
    for (int it = 0; it < kStepBytes / 1024; ++it) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void_t*)(ks_bytes + 1024 * it), 16, src + 1024u * it, 0, 0,
                                               0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void_t*)(vs_bytes + 1024 * it), 16, src + 1024u * it, 0, 0,
                                               0);
    }
  };
  const int k0 = split * a.kps;
  issue_step(k0);
  const int n_in = *a.n_rows;

  // Q as the B operand: lane (li, lg) holds head li's elements 32 kk + 8 lg .. +7.
  v8 qop[KK];
  {
    const bool hv = li < g;
    const T* qh = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)(hkv * g + (hv ? li : 0)) * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        qop[kk][e] = hv ? qh[(int64_t)(32 * kk + 8 * lg + e) * a.q_sd] : static_cast<T>(0.f);
  }
  // The new row (element lane + 64 e).
  const T* kn = static_cast<const T*>(a.kn) + (int64_t)b * a.n_sb + (int64_t)hkv * a.n_sh;
  const T* vn = static_cast<const T*>(a.vn) + (int64_t)b * a.n_sb + (int64_t)hkv * a.n_sh;
  T kn_r[DPL], vn_r[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    kn_r[e] = kn[(int64_t)(lane + 64 * e) * a.n_sd];
    vn_r[e] = vn[(int64_t)(lane + 64 * e) * a.n_sd];
  }

  const int n = min(n_in, a.C - 1);  // the host keeps n < C; the clamp keeps every access in bounds
  const int k1 = min(k0 + a.kps, n + 1);

  float m = -INFINITY, lsum = 0.f;  // head li, log2 units; lsum is this lane's share
  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int tr_row = 4 * lg + li / 4, tr_col = 4 * (li % 4);

  for (int j0 = k0; j0 < k1; j0 += kDecStep) {
    if (j0 != k0) {
      // The previous step's LDS reads must be done before the DMA writes land.
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue_step(j0);
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int nb = min(kDecStep, k1 - j0);
    if (n >= j0 && n < j0 + kDecStep)  // row n (not stored yet) from the new row
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        ks[(n - j0) * D + lane + 64 * e] = kn_r[e];
        vs[(n - j0) * D + lane + 64 * e] = vn_r[e];
      }
    // V rows past the split's last key to zero: their p is 0, but 0 * NaN
    // is not (the rows past n hold whatever the buffer held).
    for (int c = nb * (kRowBytes / 16) + lane; c < kStepBytes / 16; c += 64)
      reinterpret_cast<u32x4*>(vs_bytes)[c] = u32x4{0u, 0u, 0u, 0u};
    __builtin_amdgcn_wave_barrier();

    // S^T = K Q^T, 16 keys per block.
    f32x4 s[4];
#pragma unroll
    for (int kb4 = 0; kb4 < 4; ++kb4) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        acc = Elem<T>::mfma(
            bitcast_u4<v8>(*reinterpret_cast<const u32x4*>(ks + (16 * kb4 + li) * D + 32 * kk + 8 * lg)), qop[kk],
            acc);
      s[kb4] = acc;
    }
    // Keys past the split's last one masked; the head's step maximum over
    // its four lanes (IEEE maximum; scaling by a positive factor keeps the
    // order).
    float tmax = -INFINITY;
#pragma unroll
    for (int kb4 = 0; kb4 < 4; ++kb4)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = (16 * kb4 + 4 * lg + r) < nb ? s[kb4][r] : -INFINITY;
        s[kb4][r] = x;
        tmax = __builtin_elementwise_maximum(tmax, x);
      }
    tmax = max_xor32(max_xor16(tmax)) * a.scale_log2;
    const float mnew = fmaxf(m, tmax);  // finite: key j0 is valid
    const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
    float pv[16], psum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      pv[i] = __builtin_amdgcn_exp2f(fmaf(s[i / 4][i % 4], a.scale_log2, -mnew));
      psum += pv[i];
    }
    lsum = lsum * alpha + psum;
    m = mnew;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    // P^T operands of the two 32-key k-steps: element e of k-step ks is key
    // 32 ks + 4 lg + e (e < 4) or 32 ks + 16 + 4 lg + e - 4, which is
    // pv[8 ks + e]; the transposing V reads below give V^T in that key order.
    v8 phi[2], plo[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = pv[8 * k2 + e];
        phi[k2][e] = static_cast<T>(x);
        plo[k2][e] = static_cast<T>(x - static_cast<float>(phi[k2][e]));
      }
    // O^T += V^T P^T: lane (li, lg) of the A operand needs V[key][16 dt + li]
    // for the eight keys above; a transposing read gives output lane i of
    // each 16-lane group element e of input lane 4e + i/4's 8 bytes, element
    // i % 4, so input lane li reads key base + li/4, columns
    // 16 dt + 4 (li % 4) .. +3.
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      typedef short s4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) s4 lds_s4;
      const T* vrow = vs + 32 * k2 * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const s4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(vrow + tr_row * D + 16 * dt + tr_col));
        const s4 x1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(vrow + (16 + tr_row) * D + 16 * dt + tr_col));
        const v8 aop = __builtin_bit_cast(v8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dt] = Elem<T>::mfma(aop, phi[k2], o[dt]);
        o[dt] = Elem<T>::mfma(aop, plo[k2], o[dt]);
      }
    }
  }

  if (k0 <= n && n < k1)  // this split owns row n: store the new row
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      kb[(int64_t)n * D + lane + 64 * e] = kn_r[e];
      vb[(int64_t)n * D + lane + 64 * e] = vn_r[e];
    }
  // The split's partials (heads h < g).
  lsum = add_xor32(add_xor16(lsum));
  const int64_t base = ((int64_t)bh * a.S + split) * g;
  if (li < g) {
    float* po = a.part_o + (base + li) * D + 4 * lg;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) po[16 * dt + r] = o[dt][r];
    if (lg == 0) {
      a.part_m[base + li] = m;
      a.part_l[base + li] = lsum;
    }
  }
}

// One wave per query head: combine the splits and write the output row.
// Lane s holds split s's (m, l); the partial outputs of up to 32 splits are
// loaded together with the statistics, before the reductions.
template <typename T, int D>
__global__ void __launch_bounds__(64) decode_merge_kernel(DecodeArgs a) {
  constexpr int DPL = D / 64;
  constexpr int kBatch = 32;
  static_assert(kDecMaxSplits % kBatch == 0, "whole batches of splits");
  const int g = a.Hq / a.Hkv;
  const int b = blockIdx.x / a.Hq, hq = blockIdx.x % a.Hq;
  const int hkv = hq / g, h = hq % g;
  const int lane = threadIdx.x;
  const int64_t base = ((int64_t)(b * a.Hkv + hkv) * a.S) * g + h;
  float ob[kBatch][DPL];
  auto load_batch = [&](int s0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
#pragma unroll
      for (int e = 0; e < DPL; ++e)
        ob[u][e] = s0 + u < a.S ? a.part_o[(base + (int64_t)(s0 + u) * g) * D + lane * DPL + e] : 0.f;
  };
  const float ml = lane < a.S ? a.part_m[base + (int64_t)lane * g] : -INFINITY;
  const float ll = lane < a.S ? a.part_l[base + (int64_t)lane * g] : 0.f;
  load_batch(0);
  const float mx = wave_max_dpp(ml);
  // Lanes past S, and splits with no rows, weigh 0.
  const float f = ml == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml - mx);
  const float l = wave_sum_dpp(ll * f);
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < a.S; s0 += kBatch) {
    if (s0) load_batch(s0);
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float fs = read_lane_f(f, s0 + u);  // s0 + u < kDecMaxSplits <= 64
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[e] += fs * ob[u][e];
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
  launch((decode_partial_kernel<T, D>), grid, dim3(64), 0, st, a);
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
  a.kps = (p.C + a.S - 1) / a.S;
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
