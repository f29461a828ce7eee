// Host-side interfaces between the kernel translation units and the C ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dkv {

// Kernel timing (dropkv_timing_*): when enabled on the calling thread,
// timing_pair hands out the (start, stop) events of the current call's next
// kernel and returns true.  hipExtLaunchKernel sets them to that dispatch's
// own begin and end time stamps, so the elapsed time is the kernel's
// execution alone, without the dispatch gap before it.
bool timing_pair(hipEvent_t* start, hipEvent_t* stop);

// Every kernel of the API calls is launched through here.
template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t st,
                   Args... args) {
  hipEvent_t a, b;
  if (timing_pair(&a, &b))
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, st, a, b, 0u, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, shmem, st, args...);
}

// Element types (the DROPKV_BF16 / _FP16 / _FP32 codes of the C ABI).
constexpr int kDtypeBf16 = 1, kDtypeFp16 = 2, kDtypeFp32 = 3;

// Head dimensions of the matrix-core scoring kernels; every other one (and
// fp32 inputs) takes the generic kernels (dkv_generic.hip).
constexpr int64_t kMfmaHeadDims[] = {32, 64, 128};
inline bool mfma_head_dim(int64_t D) {
  for (int64_t d : kMfmaHeadDims)
    if (d == D) return true;
  return false;
}
// Query rows per KV head (g * W) the matrix-core kernels take; more go to the
// generic kernels too.
constexpr int64_t kMfmaMaxRows = 4096;
inline bool scores_generic(int dtype, int64_t D, int64_t M) {
  return dtype == kDtypeFp32 || !mfma_head_dim(D) || M > kMfmaMaxRows;
}

// Launch geometry and workspace layout of one scoring call.
struct ScorePlan {
  int heads, g, M, n_mc, mpad;
  int s1, kps1;  // pass 1: splits per (head, row-chunk), keys per split
  int s2, kps2;  // pass 2: splits per head, keys per split
  int p1_waves, p2_waves;  // launch shapes
  int p1_wide;                     // pass 1 with all row-chunks of a head in one workgroup
  size_t off_sync, off_ml, off_y, off_cand, off_op, off_stb, off_stat, off_yf, total;
};

ScorePlan make_score_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t Lk, int64_t D, int64_t W, int64_t splits);
struct SelectCompact;
// Pooling fused into the scoring pass: the selection workspace (its per-row
// words are cleared by the merge kernel through zero_ptr) and the pooling
// parameters.  The selection then continues with launch_select_after_pool
// using the pass-2 split geometry (ScorePlan::s2, ::kps2).
struct FuseSelect {
  char* ws;
  int ks, window;
  // The whole selection in the scoring pass's tail (threshold, ordered emit
  // and the gather through `cp`), when the plan and the GPU allow it: the
  // scoring launch then sets *tail_done and the caller skips
  // launch_select_after_pool.  keep_idx null: never.
  int keep;
  int64_t* keep_idx;
  const SelectCompact* cp;
  int* tail_done;
};
// K/V: [B*Hkv, kv_ld, D] with rows 0 .. Lk-1 of each head used (kv_ld = Lk: contiguous).
hipError_t launch_scores(const ScorePlan& p, int dtype, int D, const void* q, int64_t q_sb, int64_t q_sh,
                         int64_t q_ss, int64_t q_sd, const void* k, const void* v, int kv_ld, int Hkv, int Lq,
                         int Lk, int W, float eps, int p_round, int y_round, float* scores, char* ws,
                         uint32_t* zero_ptr, int64_t zero_words, const FuseSelect* fuse, hipStream_t st);
// Counters at the start of every score / evict workspace
// (ScorePlan::off_sync): zero when a workspace is first used, and zero again
// after every call (the DROPKV_SYNC_BYTES contract of the C ABI).
constexpr size_t kSyncBytes = 4096;
hipError_t launch_debug_state(const ScorePlan& p, const char* ws, int D, float* lse_out, float* y_out,
                              hipStream_t st);
// The generic scoring kernels (fp32 arithmetic on the vector ALUs) on the
// same plan's workspace; no fused pooling.
hipError_t launch_scores_generic(const ScorePlan& p, int dtype, int D, const void* q, int64_t q_sb, int64_t q_sh,
                                 int64_t q_ss, int64_t q_sd, const void* k, const void* v, int kv_ld, int Hkv, int Lq,
                                 int Lk, int W, float eps, int p_round, int y_round, float* scores, char* ws,
                                 uint32_t* zero_ptr, int64_t zero_words, hipStream_t st);
int64_t generic_max_head_dim();
hipError_t launch_mfma_selftest(float* out, hipStream_t st);

// Decode step on the compressed cache (dkv_decode.hip).
struct DecodeParams {
  const void* q;  // [B, Hq, 1, D] element strides
  int64_t q_sb, q_sh, q_sd;
  const void* kn;  // the new token's K and V rows [B, Hkv, 1, D] (same strides)
  const void* vn;
  int64_t n_sb, n_sh, n_sd;
  void* kbuf;  // [B, Hkv, C, D] contiguous cache buffers
  void* vbuf;
  const int* n_rows;  // device int: rows already stored
  int B, Hq, Hkv, D, C;
  int dtype_bf16;
  float scale;
  void* out;  // [B, 1, Hq, D] element strides
  int64_t o_sb, o_sh, o_sd;
  void* workspace;
};
int decode_splits(int C);
size_t decode_workspace_bytes(int B, int Hq, int Hkv, int D, int C);
hipError_t launch_decode_attention(const DecodeParams& p, hipStream_t st);

size_t select_workspace_bytes(int64_t rows, int64_t Lk);
// Words at the start of the selection workspace that must be zero on entry
// (cleared by launch_select itself unless the caller already did it).
int64_t select_zero_words(int64_t rows);
// Longest row the selection kernels take.
int64_t select_max_len();
// Optional K/V gather fused into the selection's emit stage: rows of
// [B, H, L, D] sources (element strides s_b, s_h, s_l; D contiguous; 16-byte
// aligned rows) go to contiguous [B, H, keep, D] outputs.
struct SelectCompact {
  const void* k;
  const void* v;
  int64_t s_b, s_h, s_l, elem_bytes, D;
  int H;
  void* k_out;
  void* v_out;
  int64_t out_ld;  // rows per head in k_out / v_out ([B, H, out_ld, D]; keep: contiguous)
};
struct CompactArgs;
CompactArgs compact_args(const SelectCompact* cp);
// mode 0: the selection always runs as its own kernels after the scoring
// pass; 1: in the scoring pass's tail whenever the call allows it.  spin >= 0
// sets the polls a workgroup waits at the tail's first barrier before it
// leaves the row to the last one to arrive, spin_b >= 0 the polls at the
// second barrier before it finishes the row alone (tests use 0 to force
// those paths).
void set_tail_select(int mode, int spin, int spin_b);
hipError_t launch_select(const float* scores, int rows, int Lk, int ks, int window, int keep, int64_t* out_idx,
                         float* pooled_out, char* ws, bool pre_zeroed, const SelectCompact* cp, hipStream_t st);
// The resolve and emit stages after a pooling stage that pooled every key
// except those within kernel_size/2 of j = i*kps (1 <= i < n_splits).
hipError_t launch_select_after_pool(const float* scores, int rows, int Lk, int ks, int window, int keep,
                                    int n_splits, int kps, int64_t* out_idx, float* pooled_out, char* ws,
                                    const SelectCompact* cp, hipStream_t st);
// Whether launch_select_after_pool accepts that geometry.
bool select_after_pool_ok(int64_t n_splits, int64_t kps, int64_t Lk, int64_t ks);

// Rows 0 .. L-1 of src ([B, H, L, D], element strides s_b, s_h, s_l, D
// contiguous) to rows row0 .. row0+L-1 of dst ([B, H, dst_ld, D] contiguous).
hipError_t launch_append(const void* k, const void* v, int64_t s_b, int64_t s_h, int64_t s_l, int64_t eb, int64_t B,
                         int64_t H, int64_t L, int64_t D, void* dk, void* dv, int64_t dst_ld, int64_t row0,
                         hipStream_t st);

hipError_t launch_compact(const void* k0, const void* v0, int64_t s0b, int64_t s0h, int64_t s0l, int64_t L0,
                          const void* k1, const void* v1, int64_t s1b, int64_t s1h, int64_t s1l, int64_t L1,
                          int64_t eb, int64_t B, int64_t H, int64_t D, const int64_t* idx, int64_t keep, void* ko,
                          void* vo, hipStream_t st);

}  // namespace dkv
