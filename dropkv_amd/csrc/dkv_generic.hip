// DropKV scoring for the inputs the matrix-core kernels do not take: fp32
// Q/K/V (the reference's deployed path scores them in PyTorch fp32,
// dropkv_cache.py:399-460), or a head dimension outside the matrix-core set
// (dropkv_scores_triton accepts any power of two >= 32,
// dropkv_triton.py:707-713; the deployed path any D).
//
// Plain fp32 arithmetic on the vector ALUs, with the reference's semantics
// computed exactly rather than corrected afterwards:
//   stats kernel, one workgroup per (head, query row): a first sweep over the
//     row's keys for its maximum and sum (lse), a second for
//     y = sum_j p_j v_j with the final p (rounded to the input dtype first
//     when p_round, dropkv_triton.py:88-93; y itself rounded when y_round,
//     dropkv_cache.py:434);
//   score kernel, one workgroup per (head, 256 keys), one thread per key:
//     score_j = (1/g) sum_m w(p_mj) |v_j - y_m|^2 with the distance taken
//     directly (dropkv_triton.py:96-108 expands it; the direct form has no
//     cancellation).
// Each stage recomputes the logits it needs (one thread per key, the same
// sequential dot product in both kernels, so both see the same p) instead of
// storing a [rows, Lk] matrix: the workspace is the matrix-core plan's.
#include "dkv_common.h"
#include "dkv_internal.h"

namespace dkv {

constexpr int kGenThreads = 256;
constexpr int kGenMaxD = 4096;
constexpr int kGenCols = kGenMaxD / kGenThreads;  // y columns per thread of the stats kernel (at most)

// Query rows per pass of the score kernel: R rows of q and of y in 4096
// floats of LDS (16 KiB), at least one (2*D floats for D above 2048).
constexpr int gen_rows(int D) {
  return D <= 64 ? 32 : D <= 128 ? 16 : D <= 256 ? 8 : D <= 512 ? 4 : D <= 1024 ? 2 : 1;
}

template <typename T>
__device__ __forceinline__ float ld(const T* p) {
  return static_cast<float>(*p);
}

// Logit of query row qs (LDS, D floats) and key row k (D elements), scaled.
template <typename T>
__device__ __forceinline__ float gen_logit(const float* qs, const T* __restrict__ k, int D, float scale) {
  float acc = 0.f;
  for (int d = 0; d < D; ++d) acc = fmaf(qs[d], ld(k + d), acc);
  return acc * scale;
}

template <typename T>
__global__ void __launch_bounds__(kGenThreads)
gen_stats_kernel(const T* __restrict__ q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd,
                 const T* __restrict__ kp, const T* __restrict__ vp, int kv_ld, int Hkv, int Lq, int Lk, int D, int W,
                 int g, int M, int mpad, float scale, int p_round, int y_round, float* __restrict__ ystat,
                 float* __restrict__ yf32, uint32_t* __restrict__ zero_ptr, int64_t zero_words) {
  __shared__ float qs[kGenMaxD];
  __shared__ float ps[kGenThreads];
  __shared__ float red[2 * kGenThreads / 64];
  const int tid = threadIdx.x;
  if (zero_ptr)
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + tid; i < zero_words; i += (int64_t)gridDim.x * blockDim.x)
      zero_ptr[i] = 0u;
  const int head = blockIdx.x / M, m = blockIdx.x % M;
  const int b = head / Hkv, hkv = head % Hkv, gi = m / W, w = m % W;
  const T* qrow = q + (int64_t)b * q_sb + (int64_t)(hkv * g + gi) * q_sh + (int64_t)(Lq - W + w) * q_ss;
  for (int d = tid; d < D; d += kGenThreads) qs[d] = ld(qrow + (int64_t)d * q_sd);
  __syncthreads();
  const T* kh = kp + (int64_t)head * kv_ld * D;
  const T* vh = vp + (int64_t)head * kv_ld * D;
  const int bound = Lk - W + w;  // keys j <= bound are visible to this row

  // Sweep 1: maximum and sum of exp(l - max) per thread, then per row.
  float mt = -INFINITY, st = 0.f;
  for (int j = tid; j <= bound; j += kGenThreads) {
    const float l = gen_logit(qs, kh + (int64_t)j * D, D, scale);
    if (l > mt) {
      st = st * __expf(mt - l) + 1.f;
      mt = l;
    } else {
      st += __expf(l - mt);
    }
  }
  float mr = wave_max(mt);
  if ((tid & 63) == 0) red[tid >> 6] = mr;
  __syncthreads();
  mr = red[0];
  for (int i = 1; i < kGenThreads / 64; ++i) mr = fmaxf(mr, red[i]);
  const float sr = wave_sum(mt == -INFINITY ? 0.f : st * __expf(mt - mr));
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = sr;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < kGenThreads / 64; ++i) s += red[i];
  const float lse = mr + __logf(s);

  // Sweep 2: y = sum_j p_j v_j with the final p, 256 keys at a time.
  float y[kGenCols];  // columns tid + 256 c
#pragma unroll
  for (int c = 0; c < kGenCols; ++c) y[c] = 0.f;
  for (int j0 = 0; j0 <= bound; j0 += kGenThreads) {
    const int j = j0 + tid;
    float p = 0.f;
    if (j <= bound) {
      p = fminf(__expf(gen_logit(qs, kh + (int64_t)j * D, D, scale) - lse), 1.f);
      if (p_round) p = round_through<T>(p);
    }
    __syncthreads();
    ps[tid] = p;
    __syncthreads();
    const int n = min(kGenThreads, bound + 1 - j0);
    for (int u = 0; u < n; ++u) {
      const float pu = ps[u];
      const T* vr = vh + (int64_t)(j0 + u) * D;
#pragma unroll
      for (int c = 0; c < kGenCols; ++c)
        if (tid + c * kGenThreads < D) y[c] = fmaf(pu, ld(vr + tid + c * kGenThreads), y[c]);
    }
  }
  const int64_t rbase = (int64_t)head * mpad + m;
#pragma unroll
  for (int c = 0; c < kGenCols; ++c)
    if (tid + c * kGenThreads < D) yf32[rbase * D + tid + c * kGenThreads] = y_round ? round_through<T>(y[c]) : y[c];
  if (tid == 0) {
    ystat[rbase * 2 + 0] = lse * 1.4426950408889634f;  // log2 units, as the matrix-core merge stores it
    ystat[rbase * 2 + 1] = lse;                         // natural units, read by gen_score_kernel
  }
}

template <typename T, int R>
__global__ void __launch_bounds__(kGenThreads)
gen_score_kernel(const T* __restrict__ q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd,
                 const T* __restrict__ kp, const T* __restrict__ vp, int kv_ld, int Hkv, int Lq, int Lk, int D, int W,
                 int g, int M, int mpad, float scale, float eps, int p_round, const float* __restrict__ ystat,
                 const float* __restrict__ yf32, float* __restrict__ scores) {
  // R query rows of D, then R y rows of D (dynamic LDS).
  extern __shared__ float gen_lds[];
  float* qs = gen_lds;
  float* ys = gen_lds + R * D;
  __shared__ float ls[R];  // their lse
  const int tid = threadIdx.x;
  const int tiles = (Lk + kGenThreads - 1) / kGenThreads;
  const int head = blockIdx.x / tiles;
  const int j = (blockIdx.x % tiles) * kGenThreads + tid;
  const int b = head / Hkv, hkv = head % Hkv;
  const T* krow = kp + ((int64_t)head * kv_ld + min(j, Lk - 1)) * D;
  const T* vrow = vp + ((int64_t)head * kv_ld + min(j, Lk - 1)) * D;
  float score = 0.f;
  for (int r0 = 0; r0 < M; r0 += R) {
    const int nr = min(R, M - r0);
    __syncthreads();
    for (int i = tid; i < nr * D; i += kGenThreads) {
      const int r = i / D, d = i % D, m = r0 + r;
      const int gi = m / W, w = m % W;
      qs[i] = ld(q + (int64_t)b * q_sb + (int64_t)(hkv * g + gi) * q_sh + (int64_t)(Lq - W + w) * q_ss +
                 (int64_t)d * q_sd);
      ys[i] = yf32[((int64_t)head * mpad + m) * D + d];
    }
    if (tid < nr) ls[tid] = ystat[((int64_t)head * mpad + r0 + tid) * 2 + 1];
    __syncthreads();
    float dot[R], d2[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      dot[r] = 0.f;
      d2[r] = 0.f;
    }
    for (int d = 0; d < D; ++d) {
      const float kd = ld(krow + d), vd = ld(vrow + d);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (r < nr) {
          dot[r] = fmaf(qs[r * D + d], kd, dot[r]);
          const float df = vd - ys[r * D + d];
          d2[r] = fmaf(df, df, d2[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int m = r0 + r;
      if (r < nr && j <= Lk - W + (m % W)) {
        float p = fminf(__expf(dot[r] * scale - ls[r]), 1.f);
        if (p_round) p = round_through<T>(p);
        const float ratio = p / (1.f - p + eps);
        score = fmaf(ratio * ratio, d2[r], score);
      }
    }
  }
  if (j < Lk) scores[(int64_t)head * Lk + j] = score / static_cast<float>(g);
}

template <typename T>
static hipError_t launch_generic_t(const ScorePlan& p, int D, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                                   int64_t q_sd, const void* k, const void* v, int kv_ld, int Hkv, int Lq, int Lk,
                                   int W, float eps, int p_round, int y_round, float* scores, char* ws,
                                   uint32_t* zero_ptr, int64_t zero_words, hipStream_t st) {
  const float scale = 1.0f / sqrtf((float)D);
  float* ystat = reinterpret_cast<float*>(ws + p.off_stat);
  float* yf = reinterpret_cast<float*>(ws + p.off_yf);
  const T* qq = static_cast<const T*>(q);
  const T* kk = static_cast<const T*>(k);
  const T* vv = static_cast<const T*>(v);
  launch(gen_stats_kernel<T>, dim3(p.heads * p.M), dim3(kGenThreads), 0, st, qq, q_sb, q_sh, q_ss, q_sd, kk, vv,
         kv_ld, Hkv, Lq, Lk, D, W, p.g, p.M, p.mpad, scale, p_round, y_round, ystat, yf, zero_ptr, zero_words);
  const int tiles = (Lk + kGenThreads - 1) / kGenThreads;
  const size_t lds = (size_t)2 * gen_rows(D) * D * sizeof(float);
  auto score = [&](auto kern) {
    launch(kern, dim3(p.heads * tiles), dim3(kGenThreads), lds, st, qq, q_sb, q_sh, q_ss, q_sd, kk, vv, kv_ld, Hkv,
           Lq, Lk, D, W, p.g, p.M, p.mpad, scale, eps, p_round, ystat, yf, scores);
  };
  switch (gen_rows(D)) {
    case 32: score(gen_score_kernel<T, 32>); break;
    case 16: score(gen_score_kernel<T, 16>); break;
    case 8: score(gen_score_kernel<T, 8>); break;
    case 4: score(gen_score_kernel<T, 4>); break;
    case 2: score(gen_score_kernel<T, 2>); break;
    default: score(gen_score_kernel<T, 1>); break;
  }
  return hipGetLastError();
}

int64_t generic_max_head_dim() { return kGenMaxD; }

hipError_t launch_scores_generic(const ScorePlan& p, int dtype, int D, const void* q, int64_t q_sb, int64_t q_sh,
                                 int64_t q_ss, int64_t q_sd, const void* k, const void* v, int kv_ld, int Hkv, int Lq,
                                 int Lk, int W, float eps, int p_round, int y_round, float* scores, char* ws,
                                 uint32_t* zero_ptr, int64_t zero_words, hipStream_t st) {
  if (D < 1 || D > kGenMaxD) return hipErrorInvalidValue;
  switch (dtype) {
    case kDtypeBf16:
      return launch_generic_t<__bf16>(p, D, q, q_sb, q_sh, q_ss, q_sd, k, v, kv_ld, Hkv, Lq, Lk, W, eps, p_round,
                                      y_round, scores, ws, zero_ptr, zero_words, st);
    case kDtypeFp16:
      return launch_generic_t<_Float16>(p, D, q, q_sb, q_sh, q_ss, q_sd, k, v, kv_ld, Hkv, Lq, Lk, W, eps, p_round,
                                        y_round, scores, ws, zero_ptr, zero_words, st);
    case kDtypeFp32:
      return launch_generic_t<float>(p, D, q, q_sb, q_sh, q_ss, q_sd, k, v, kv_ld, Hkv, Lq, Lk, W, eps, p_round,
                                     y_round, scores, ws, zero_ptr, zero_words, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace dkv
