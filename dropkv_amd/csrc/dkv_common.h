// Shared device-side definitions for the DropKV gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dkv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Element traits: the bf16 / fp16 operand vector (8 elements = 16 bytes =
// one lane's share of a 16x16x32 MFMA operand) and the matching MFMA.
template <typename T>
struct Elem;

template <>
struct Elem<__bf16> {
  typedef __bf16 v8 __attribute__((__vector_size__(16)));
  static __device__ __forceinline__ f32x4 mfma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Elem<_Float16> {
  typedef _Float16 v8 __attribute__((__vector_size__(16)));
  static __device__ __forceinline__ f32x4 mfma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Round-to-nearest-even through the element type and back.
template <typename T>
__device__ __forceinline__ float round_through(float x) {
  return static_cast<float>(static_cast<T>(x));
}
// bf16: one packed conversion with x in the high half and +0 in the low half,
// whose 32 bits are then exactly the rounded value as a float (the plain
// conversion adds a shift).
template <>
__device__ __forceinline__ float round_through<__bf16>(float x) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(float, __builtin_convertvector((f2{0.f, x}), h2));
}

// Whether any lane of the wave has `pred`, as a scalar (SGPR) value, so that
// a branch on it is compiled as a uniform branch: the not-taken side then
// issues nothing.  (__any's result is not known to be uniform, and a branch
// on it is compiled as an exec-masked if/else whose both sides issue.)
__device__ __forceinline__ bool wave_any(bool pred) {
  return __builtin_amdgcn_readfirstlane((int)(__builtin_amdgcn_ballot_w64(pred) != 0)) != 0;
}

// min(p, 1) for p >= 0 or NaN (as unsigned integers: NaN gives 1, like fminf)
// and min(x, 0) for the sign of x (as signed integers): one integer op each,
// where fminf also canonicalises its operand.
__device__ __forceinline__ float min_one_nonneg(float p) {
  return __builtin_bit_cast(float, min(__builtin_bit_cast(uint32_t, p), 0x3f800000u));
}
__device__ __forceinline__ float min_zero(float x) {
  return __builtin_bit_cast(float, min(__builtin_bit_cast(int32_t, x), 0));
}

// Raw buffer view of `bytes` bytes at `base`.  Loads at byte offsets >= bytes
// return zeros and issue no memory request, so a tile loop can load past the
// end of its range without a branch.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // Word 3: 32-bit data format, no swizzle / stride / thread-id addressing.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

__device__ __forceinline__ uint16_t buf_load2(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0));
}

__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
}

// 8-byte loads come back as a float or an int vector, each converted from
// the load's result as a whole: this compiler turned a 64- or 128-bit buffer
// load whose uint32 elements were then bit-cast to float one by one into a
// 32-bit load (the other elements read undefined registers).  Elements of a
// uint32 vector used as integers are unaffected.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f32x2 buf_load8f(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0));
}
__device__ __forceinline__ i32x2 buf_load8i(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0));
}

template <typename V>
__device__ __forceinline__ V bitcast_u4(u32x4 x) {
  return __builtin_bit_cast(V, x);
}

// Stores that are coherent across the whole device when they complete
// (agent-scope relaxed atomic stores: write-through to the memory-side
// cache), for data that workgroups on other XCDs read within the same
// kernel after a counter handshake.  A release then needs only the wait for
// the stores, not a write-back of the XCD's L2.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The same write-through policy (sc1) for a 16-byte buffer store.
constexpr int kAuxSc1 = 16;
__device__ __forceinline__ void st_dev16(rsrc_t r, uint32_t voff, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff, 0, kAuxSc1);
}

// Order-preserving map float -> uint32 (larger float => larger key).
// -0.0 is folded onto +0.0 so that the two compare equal, as in torch.
__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t b = __float_as_uint(f);
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_float(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}

// Workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8).
// Remap so that consecutive logical ids land on the same XCD (and so share
// its L2) while keeping the dispatch order.  Bijective on [0, n).
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int q = n >> 3, r = n & 7;
  const int xcd = bid & 7, slot = bid >> 3;
  const int base = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
  return base + slot;
}

// Wave-wide reductions over DPP row operations: a max / min / sum within each
// row of 16 lanes (two quad permutes, the half-row mirror, the row mirror),
// then the four rows combined from lane reads.  The result is wave-uniform.
// Far shorter latency than lane shuffles through LDS (ds_bpermute).
template <int kCtrl>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_mov_dpp(x, kCtrl, 0xf, 0xf, false);
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, dpp_i<kCtrl>(__builtin_bit_cast(int, x)));
}
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror
__device__ __forceinline__ float read_lane_f(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

__device__ __forceinline__ float wave_max_dpp(float x) {
  x = fmaxf(x, dpp_f<kDppQuadSwap1>(x));
  x = fmaxf(x, dpp_f<kDppQuadSwap2>(x));
  x = fmaxf(x, dpp_f<kDppHalfMirror>(x));
  x = fmaxf(x, dpp_f<kDppMirror>(x));
  return fmaxf(fmaxf(read_lane_f(x, 0), read_lane_f(x, 16)), fmaxf(read_lane_f(x, 32), read_lane_f(x, 48)));
}

__device__ __forceinline__ float wave_sum_dpp(float x) {
  x += dpp_f<kDppQuadSwap1>(x);
  x += dpp_f<kDppQuadSwap2>(x);
  x += dpp_f<kDppHalfMirror>(x);
  x += dpp_f<kDppMirror>(x);
  return (read_lane_f(x, 0) + read_lane_f(x, 16)) + (read_lane_f(x, 32) + read_lane_f(x, 48));
}

__device__ __forceinline__ int wave_min_dpp(int x) {
  x = min(x, dpp_i<kDppQuadSwap1>(x));
  x = min(x, dpp_i<kDppQuadSwap2>(x));
  x = min(x, dpp_i<kDppHalfMirror>(x));
  x = min(x, dpp_i<kDppMirror>(x));
  return min(min(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
             min(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// Lane i combined with lane i ^ 16 or i ^ 32 through v_permlane16_swap /
// v_permlane32_swap (one VALU operation instead of an LDS-routed shuffle):
// with both operands x, the swap leaves each lane holding {x[i], x[i ^ 16]}
// (resp. 32) in its two results, in an order that depends on the lane, so
// only commutative combinations are formed here.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The value of lane i ^ 16 (resp. i ^ 32): the swap's two results are the
// values of the lane with that bit clear and of the lane with it set.
__device__ __forceinline__ uint32_t from_xor16(uint32_t x, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  return (lane & 16) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t from_xor32(uint32_t x, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return (lane & 32) ? r[0] : r[1];
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

}  // namespace dkv
