// Gather-compaction of the retained keys/values (DropKVCache._gather_compressed,
// dropkv_cache.py:479-491) and its two-segment form for the chunked-prefill
// continuation (dropkv_cache.py:581-607).  Bit copies in 16-byte pieces when
// the row allows it, element copies otherwise.  Indices outside [0, L) are
// not dereferenced; their output rows are zero-filled.  Outputs are written
// with non-temporal stores: a short copy kernel that leaves its output dirty
// in the L2 waits at its end for the write-back (a 16 MB append took 20 us
// with plain stores against 5 us).
#include "dkv_common.h"
#include "dkv_internal.h"

namespace dkv {

constexpr int kCopyThreads = 256;
constexpr int kRowsPerBlock = 64;

struct Seg {
  const uint8_t* k;
  const uint8_t* v;
  int64_t sb, sh, sl;  // byte strides
  int64_t len;
};

// Each thread copies up to kItems (row, unit) pieces per round with every
// index load, then every data load, in flight before the stores.
constexpr int kItems = 4;

template <typename U>
__global__ void __launch_bounds__(kCopyThreads)
compact_kernel(Seg s0, Seg s1, int H, int units_per_row, const int64_t* __restrict__ idx, int keep,
               int blocks_per_head, uint8_t* __restrict__ ko, uint8_t* __restrict__ vo) {
  const int bh = blockIdx.x / blocks_per_head;
  const int r0 = (blockIdx.x % blocks_per_head) * kRowsPerBlock;
  const int b = bh / H, h = bh % H;
  const int64_t out_row_bytes = (int64_t)units_per_row * sizeof(U);
  const int total = min(kRowsPerBlock, keep - r0) * units_per_row;
  for (int t0 = threadIdx.x; t0 < total; t0 += kItems * kCopyThreads) {
    int64_t src[kItems];
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
      const int t = t0 + q * kCopyThreads;
      src[q] = t < total ? idx[(int64_t)bh * keep + r0 + t / units_per_row] : -1;
    }
    U kval[kItems], vval[kItems];
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
      const int u = (t0 + q * kCopyThreads) % units_per_row;
      kval[q] = U{};
      vval[q] = U{};
      if (src[q] >= 0 && src[q] < s0.len) {
        const int64_t off = b * s0.sb + h * s0.sh + src[q] * s0.sl;
        kval[q] = reinterpret_cast<const U*>(s0.k + off)[u];
        vval[q] = reinterpret_cast<const U*>(s0.v + off)[u];
      } else if (src[q] >= s0.len && src[q] < s0.len + s1.len) {
        const int64_t off = b * s1.sb + h * s1.sh + (src[q] - s0.len) * s1.sl;
        kval[q] = reinterpret_cast<const U*>(s1.k + off)[u];
        vval[q] = reinterpret_cast<const U*>(s1.v + off)[u];
      }
    }
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
      const int t = t0 + q * kCopyThreads;
      if (t < total) {
        const int64_t o = ((int64_t)bh * keep + r0 + t / units_per_row) * out_row_bytes;
        __builtin_nontemporal_store(kval[q], reinterpret_cast<U*>(ko + o) + t % units_per_row);
        __builtin_nontemporal_store(vval[q], reinterpret_cast<U*>(vo + o) + t % units_per_row);
      }
    }
  }
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Append: rows 0 .. L-1 of each head of src to rows row0 .. of the head in a
// [B*H, dst_ld, D] buffer.  kRowsPerBlock rows per workgroup, kItems pieces
// per thread with every load in flight before the stores.
template <typename U>
__global__ void __launch_bounds__(kCopyThreads)
append_kernel(Seg s, int H, int units_per_row, int L, int blocks_per_head, uint8_t* __restrict__ dk,
              uint8_t* __restrict__ dv, int64_t dst_ld, int64_t row0) {
  const int bh = blockIdx.x / blocks_per_head;
  const int r0 = (blockIdx.x % blocks_per_head) * kRowsPerBlock;
  const int b = bh / H, h = bh % H;
  const int64_t row_bytes = (int64_t)units_per_row * sizeof(U);
  const int total = min(kRowsPerBlock, L - r0) * units_per_row;
  for (int t0 = threadIdx.x; t0 < total; t0 += kItems * kCopyThreads) {
    U kval[kItems], vval[kItems];
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
      const int t = t0 + q * kCopyThreads;
      if (t < total) {
        const int64_t off = b * s.sb + h * s.sh + (int64_t)(r0 + t / units_per_row) * s.sl;
        kval[q] = reinterpret_cast<const U*>(s.k + off)[t % units_per_row];
        vval[q] = reinterpret_cast<const U*>(s.v + off)[t % units_per_row];
      }
    }
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
      const int t = t0 + q * kCopyThreads;
      if (t < total) {
        const int64_t o = ((int64_t)bh * dst_ld + row0 + r0 + t / units_per_row) * row_bytes;
        __builtin_nontemporal_store(kval[q], reinterpret_cast<U*>(dk + o) + t % units_per_row);
        __builtin_nontemporal_store(vval[q], reinterpret_cast<U*>(dv + o) + t % units_per_row);
      }
    }
  }
}

hipError_t launch_append(const void* k, const void* v, int64_t s_b, int64_t s_h, int64_t s_l, int64_t eb, int64_t B,
                         int64_t H, int64_t L, int64_t D, void* dk, void* dv, int64_t dst_ld, int64_t row0,
                         hipStream_t st) {
  if (L <= 0 || B * H == 0) return hipSuccess;
  const Seg a{static_cast<const uint8_t*>(k), static_cast<const uint8_t*>(v), s_b * eb, s_h * eb, s_l * eb, L};
  const int64_t row_bytes = D * eb;
  const bool vec = (row_bytes % 16) == 0 && aligned16(dk) && aligned16(dv) && aligned16(k) && aligned16(v) &&
                   (a.sb % 16) == 0 && (a.sh % 16) == 0 && (a.sl % 16) == 0;
  const int bph = (int)((L + kRowsPerBlock - 1) / kRowsPerBlock);
  const dim3 grid((unsigned)(B * H * bph));
  uint8_t* k8 = static_cast<uint8_t*>(dk);
  uint8_t* v8 = static_cast<uint8_t*>(dv);
  if (vec)
    launch(append_kernel<u32x4>, grid, dim3(kCopyThreads), 0, st, a, (int)H, (int)(row_bytes / 16), (int)L, bph, k8,
           v8, dst_ld, row0);
  else if (eb == 2)
    launch(append_kernel<uint16_t>, grid, dim3(kCopyThreads), 0, st, a, (int)H, (int)D, (int)L, bph, k8, v8, dst_ld,
           row0);
  else if (eb == 4)
    launch(append_kernel<uint32_t>, grid, dim3(kCopyThreads), 0, st, a, (int)H, (int)D, (int)L, bph, k8, v8, dst_ld,
           row0);
  else
    launch(append_kernel<uint8_t>, grid, dim3(kCopyThreads), 0, st, a, (int)H, (int)row_bytes, (int)L, bph, k8, v8,
           dst_ld, row0);
  return hipGetLastError();
}

hipError_t launch_compact(const void* k0, const void* v0, int64_t s0b, int64_t s0h, int64_t s0l, int64_t L0,
                          const void* k1, const void* v1, int64_t s1b, int64_t s1h, int64_t s1l, int64_t L1,
                          int64_t eb, int64_t B, int64_t H, int64_t D, const int64_t* idx, int64_t keep, void* ko,
                          void* vo, hipStream_t st) {
  if (keep <= 0 || B * H == 0) return hipSuccess;
  Seg a{static_cast<const uint8_t*>(k0), static_cast<const uint8_t*>(v0), s0b * eb, s0h * eb, s0l * eb, L0};
  Seg c{static_cast<const uint8_t*>(k1), static_cast<const uint8_t*>(v1), s1b * eb, s1h * eb, s1l * eb, L1};
  const int64_t row_bytes = D * eb;
  bool vec = (row_bytes % 16) == 0 && aligned16(ko) && aligned16(vo);
  auto seg_ok = [&](const Seg& s, const void* kp, const void* vp) {
    if (s.len == 0) return true;
    return aligned16(kp) && aligned16(vp) && (s.sb % 16) == 0 && (s.sh % 16) == 0 && (s.sl % 16) == 0;
  };
  vec = vec && seg_ok(a, k0, v0) && seg_ok(c, k1, v1);
  const int bph = (int)((keep + kRowsPerBlock - 1) / kRowsPerBlock);
  const dim3 grid((unsigned)(B * H * bph));
  if (vec) {
    launch(compact_kernel<u32x4>, grid, dim3(kCopyThreads), 0, st, a, c, (int)H, (int)(row_bytes / 16),
                       idx, (int)keep, bph, static_cast<uint8_t*>(ko), static_cast<uint8_t*>(vo));
  } else if (eb == 2) {
    launch(compact_kernel<uint16_t>, grid, dim3(kCopyThreads), 0, st, a, c, (int)H, (int)D, idx,
                       (int)keep, bph, static_cast<uint8_t*>(ko), static_cast<uint8_t*>(vo));
  } else if (eb == 4) {
    launch(compact_kernel<uint32_t>, grid, dim3(kCopyThreads), 0, st, a, c, (int)H, (int)D, idx,
                       (int)keep, bph, static_cast<uint8_t*>(ko), static_cast<uint8_t*>(vo));
  } else {
    launch(compact_kernel<uint8_t>, grid, dim3(kCopyThreads), 0, st, a, c, (int)H, (int)row_bytes, idx,
                       (int)keep, bph, static_cast<uint8_t*>(ko), static_cast<uint8_t*>(vo));
  }
  return hipGetLastError();
}

}  // namespace dkv
