// extern "C" entry points of libdropkv_amd.so (declared in include/dropkv_amd.h).
// Argument validation happens here, before anything is enqueued.
#include <cstdarg>
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/dropkv_amd.h"
#include "dkv_internal.h"



namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return DROPKV_OK;
  return fail(DROPKV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int64_t kMaxLk = (int64_t)1 << 30;

// Head dimensions of the decode kernels.
bool decode_head_dim_supported(int64_t D) { return D == 64 || D == 128; }

int64_t elem_size(int dtype) { return dtype == DROPKV_FP32 ? 4 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Whether the plan's 32-bit counts hold: query rows B*Hq*W (the generic
// grid, g*W as the plan's M) and keys B*Hkv*Lk (grids and row offsets of the
// selection).  Larger shapes (K/V of 512 GB and more, or billions of window
// rows) are refused, not wrapped around.
bool shape_counts_fit(int64_t B, int64_t Hq, int64_t Hkv, int64_t Lk, int64_t W) {
  const double rows = (double)B * (double)Hq * (double)W, keys = (double)B * (double)Hkv * (double)Lk;
  return rows <= (double)INT32_MAX && keys <= (double)INT32_MAX;
}

int check_score_args(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t Hq, int64_t Hkv,
                     int64_t Lq, int64_t Lk, int64_t D, int64_t W) {
  if (!q || !k || !v) return fail(DROPKV_E_ARG, "null q/k/v pointer");
  if (dtype != DROPKV_BF16 && dtype != DROPKV_FP16 && dtype != DROPKV_FP32)
    return fail(DROPKV_E_ARG, "dtype must be bf16, fp16 or fp32");
  if (B < 1 || Hq < 1 || Hkv < 1) return fail(DROPKV_E_ARG, "B, Hq, Hkv must be positive");
  if (Hq % Hkv != 0) return fail(DROPKV_E_ARG, "Hq (%lld) must be divisible by Hkv (%lld)", (long long)Hq,
                                 (long long)Hkv);
  if (W < 1) return fail(DROPKV_E_ARG, "window must be positive");
  if (Lq < W) return fail(DROPKV_E_ARG, "Lq (%lld) must be >= window_size (%lld)", (long long)Lq, (long long)W);
  if (Lk < W) return fail(DROPKV_E_ARG, "Lk (%lld) must be >= window_size (%lld)", (long long)Lk, (long long)W);
  if (Lq > Lk) return fail(DROPKV_E_ARG, "Lq (%lld) must be <= Lk (%lld)", (long long)Lq, (long long)Lk);
  if (Lk > kMaxLk) return fail(DROPKV_E_UNSUPPORTED, "Lk (%lld) too large", (long long)Lk);
  if (!shape_counts_fit(B, Hq, Hkv, Lk, W))
    return fail(DROPKV_E_UNSUPPORTED, "B*Hq*W or B*Hkv*Lk above %d", INT32_MAX);
  if (D < 1) return fail(DROPKV_E_ARG, "head dim must be positive");
  if (dkv::scores_generic(dtype, D, (Hq / Hkv) * W) && D > dkv::generic_max_head_dim())
    return fail(DROPKV_E_UNSUPPORTED, "head dim %lld above %lld", (long long)D, (long long)dkv::generic_max_head_dim());
  if (!aligned16(k) || !aligned16(v)) return fail(DROPKV_E_ARG, "k and v must be 16-byte aligned");
  return DROPKV_OK;
}

// Kernel timing (dropkv_timing_*), per calling thread: the i-th kernel of
// the most recent timed call gets events ev[2i] (start) and ev[2i+1] (stop),
// filled by hipExtLaunchKernel with the dispatch's begin and end time stamps.
constexpr int kMaxTimedKernels = 16;
struct Timing {
  bool on = false, created = false;
  int n = 0;  // kernels of the most recent call that got an event pair
  hipEvent_t ev[2 * kMaxTimedKernels];
};
thread_local Timing t_timing;

// Called at the start of every API entry that launches kernels.
void timing_start(hipStream_t) { t_timing.n = 0; }

}  // namespace

namespace dkv {
bool timing_pair(hipEvent_t* start, hipEvent_t* stop) {
  Timing& t = t_timing;
  if (!t.on || t.n >= kMaxTimedKernels) return false;
  *start = t.ev[2 * t.n];
  *stop = t.ev[2 * t.n + 1];
  ++t.n;
  return true;
}
}  // namespace dkv

extern "C" {

int dropkv_version(void) { return 100; }

const char* dropkv_last_error(void) { return g_err.c_str(); }

int dropkv_supported_head_dims(int64_t* out, int cap) {
  const int n = (int)(sizeof(dkv::kMfmaHeadDims) / sizeof(dkv::kMfmaHeadDims[0]));
  for (int i = 0; i < n && i < cap; ++i) out[i] = dkv::kMfmaHeadDims[i];
  return n;
}

size_t dropkv_scores_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Lk, int64_t D, int64_t W,
                                     int64_t splits) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || W < 1 || Lk < 1 || D < 1) return 0;
  if (Lk > kMaxLk || !shape_counts_fit(B, Hq, Hkv, Lk, W)) return 0;
  return dkv::make_score_plan(B, Hq, Hkv, Lk, D, W, splits).total;
}

int dropkv_scores(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, const void* k,
                  const void* v, int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D,
                  int64_t W, float eps, int p_round, int y_round, int64_t splits, float* scores, void* workspace,
                  size_t workspace_bytes, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  int rc = check_score_args(q, k, v, dtype, B, Hq, Hkv, Lq, Lk, D, W);
  if (rc) return rc;
  if (!scores) return fail(DROPKV_E_ARG, "null scores pointer");
  const dkv::ScorePlan p = dkv::make_score_plan(B, Hq, Hkv, Lk, D, W, splits);
  if (!workspace || workspace_bytes < p.total)
    return fail(DROPKV_E_WORKSPACE, "workspace too small: need %zu bytes, got %zu", p.total, workspace_bytes);
  timing_start(static_cast<hipStream_t>(stream));
  return hip_status(dkv::launch_scores(p, dtype, (int)D, q, q_sb, q_sh, q_ss, q_sd, k, v, (int)Lk,
                                       (int)Hkv, (int)Lq, (int)Lk, (int)W, eps, p_round ? 1 : 0, y_round ? 1 : 0, scores,
                                       static_cast<char*>(workspace), nullptr, 0, nullptr,
                                       static_cast<hipStream_t>(stream)),
                    "dropkv_scores launch");
}

int dropkv_scores_debug_state(const void* workspace, int64_t B, int64_t Hq, int64_t Hkv, int64_t Lk, int64_t D,
                              int64_t W, int64_t splits, float* lse_out, float* y_out, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  if (!workspace || !lse_out || !y_out) return fail(DROPKV_E_ARG, "null pointer");
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || W < 1 || Lk < W || D < 1 || D > dkv::generic_max_head_dim())
    return fail(DROPKV_E_ARG, "invalid shape");
  const dkv::ScorePlan p = dkv::make_score_plan(B, Hq, Hkv, Lk, D, W, splits);
  return hip_status(dkv::launch_debug_state(p, static_cast<const char*>(workspace), (int)D, lse_out, y_out,
                                            static_cast<hipStream_t>(stream)),
                    "dropkv_scores_debug_state launch");
}

size_t dropkv_select_workspace_bytes(int64_t rows, int64_t Lk) {
  if (rows < 1 || Lk < 1 || Lk > kMaxLk || (double)rows * (double)Lk > (double)INT32_MAX) return 0;
  return dkv::select_workspace_bytes(rows, Lk);
}

static int check_select_args(const float* scores, int64_t rows, int64_t Lk, int64_t ks, int64_t window,
                             int64_t keep, const int64_t* keep_idx) {
  if (!scores || !keep_idx) return fail(DROPKV_E_ARG, "null scores/keep_idx pointer");
  if (rows < 1 || Lk < 1) return fail(DROPKV_E_ARG, "rows and Lk must be positive");
  if (rows > 65535 * 64) return fail(DROPKV_E_UNSUPPORTED, "too many rows");
  if ((double)rows * (double)Lk > (double)INT32_MAX) return fail(DROPKV_E_UNSUPPORTED, "rows*Lk above %d", INT32_MAX);
  if (Lk > dkv::select_max_len()) return fail(DROPKV_E_UNSUPPORTED, "Lk (%lld) too large", (long long)Lk);
  if (ks < 1 || ks % 2 == 0) return fail(DROPKV_E_ARG, "kernel_size must be a positive odd integer");
  if (ks > INT32_MAX) return fail(DROPKV_E_UNSUPPORTED, "kernel_size too large");
  if (window < 0 || window > Lk) return fail(DROPKV_E_ARG, "window must be in [0, Lk]");
  if (keep < 1 || keep > Lk) return fail(DROPKV_E_ARG, "keep (%lld) must be in [1, Lk=%lld]", (long long)keep,
                                         (long long)Lk);
  return DROPKV_OK;
}

int dropkv_select(const float* scores, int64_t rows, int64_t Lk, int64_t kernel_size, int64_t window, int64_t keep,
                  int64_t* keep_idx, float* pooled, void* workspace, size_t workspace_bytes, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  int rc = check_select_args(scores, rows, Lk, kernel_size, window, keep, keep_idx);
  if (rc) return rc;
  const size_t need = dkv::select_workspace_bytes(rows, Lk);
  if (!workspace || workspace_bytes < need)
    return fail(DROPKV_E_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  timing_start(static_cast<hipStream_t>(stream));
  return hip_status(dkv::launch_select(scores, (int)rows, (int)Lk, (int)kernel_size, (int)window, (int)keep, keep_idx,
                                       pooled, static_cast<char*>(workspace), false, nullptr,
                                       static_cast<hipStream_t>(stream)),
                    "dropkv_select launch");
}

static int check_compact_common(const int64_t* idx, int64_t eb, int64_t B, int64_t H, int64_t D, int64_t keep,
                                const void* ko, const void* vo) {
  if (!idx || !ko || !vo) return fail(DROPKV_E_ARG, "null idx/output pointer");
  if (eb != 1 && eb != 2 && eb != 4 && eb != 8) return fail(DROPKV_E_ARG, "elem_bytes must be 1, 2, 4 or 8");
  if (B < 0 || H < 0 || D < 1 || keep < 0) return fail(DROPKV_E_ARG, "invalid shape");
  if (keep > kMaxLk) return fail(DROPKV_E_UNSUPPORTED, "keep too large");
  return DROPKV_OK;
}

int dropkv_compact(const void* k, const void* v, int64_t s_b, int64_t s_h, int64_t s_l, int64_t elem_bytes,
                   int64_t B, int64_t H, int64_t L, int64_t D, const int64_t* idx, int64_t keep, void* k_out,
                   void* v_out, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  int rc = check_compact_common(idx, elem_bytes, B, H, D, keep, k_out, v_out);
  if (rc) return rc;
  if (!k || !v) return fail(DROPKV_E_ARG, "null k/v pointer");
  timing_start(static_cast<hipStream_t>(stream));
  return hip_status(dkv::launch_compact(k, v, s_b, s_h, s_l, L, nullptr, nullptr, 0, 0, 0, 0, elem_bytes, B, H, D,
                                        idx, keep, k_out, v_out, static_cast<hipStream_t>(stream)),
                    "dropkv_compact launch");
}

int dropkv_compact2(const void* k0, const void* v0, int64_t s0_b, int64_t s0_h, int64_t s0_l, int64_t L0,
                    const void* k1, const void* v1, int64_t s1_b, int64_t s1_h, int64_t s1_l, int64_t L1,
                    int64_t elem_bytes, int64_t B, int64_t H, int64_t D, const int64_t* idx, int64_t keep,
                    void* k_out, void* v_out, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  int rc = check_compact_common(idx, elem_bytes, B, H, D, keep, k_out, v_out);
  if (rc) return rc;
  if ((L0 > 0 && (!k0 || !v0)) || (L1 > 0 && (!k1 || !v1))) return fail(DROPKV_E_ARG, "null segment pointer");
  if (L0 < 0 || L1 < 0) return fail(DROPKV_E_ARG, "segment lengths must be >= 0");
  timing_start(static_cast<hipStream_t>(stream));
  return hip_status(dkv::launch_compact(k0, v0, s0_b, s0_h, s0_l, L0, k1, v1, s1_b, s1_h, s1_l, L1, elem_bytes, B, H,
                                        D, idx, keep, k_out, v_out, static_cast<hipStream_t>(stream)),
                    "dropkv_compact2 launch");
}

size_t dropkv_evict_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Lk, int64_t D, int64_t W,
                                    int64_t splits) {
  const size_t a = dropkv_scores_workspace_bytes(B, Hq, Hkv, Lk, D, W, splits);
  if (!a) return 0;
  const size_t s = ((size_t)B * Hkv * Lk * 4 + 255) & ~size_t(255);
  return a + s + dkv::select_workspace_bytes(B * Hkv, Lk);
}


// One layer-call on K/V of [B*Hkv, kv_ld, D] (rows 0 .. Lk-1 used) into
// outputs of [B*Hkv, out_ld, D] (rows 0 .. keep-1 written).
static int evict_impl(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, const void* k, const void* v,
               int64_t kv_ld, int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D,
               int64_t W, float eps, int p_round, int y_round, int64_t splits, int64_t kernel_size,
               int64_t protect_window, int64_t keep, float* scores, int64_t* keep_idx, void* k_out, void* v_out,
               int64_t out_ld, void* workspace, size_t workspace_bytes, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  int rc = check_score_args(q, k, v, dtype, B, Hq, Hkv, Lq, Lk, D, W);
  if (rc) return rc;
  rc = check_select_args(reinterpret_cast<const float*>(1), B * Hkv, Lk, kernel_size, protect_window, keep, keep_idx);
  if (rc) return rc;
  if (!k_out || !v_out) return fail(DROPKV_E_ARG, "null k_out/v_out pointer");
  if (kv_ld < Lk || out_ld < keep) return fail(DROPKV_E_ARG, "row capacity below the rows used");
  if (kv_ld > INT32_MAX) return fail(DROPKV_E_UNSUPPORTED, "row capacity too large");
  const dkv::ScorePlan p = dkv::make_score_plan(B, Hq, Hkv, Lk, D, W, splits);
  const size_t s_bytes = ((size_t)B * Hkv * Lk * 4 + 255) & ~size_t(255);
  const size_t need = p.total + s_bytes + dkv::select_workspace_bytes(B * Hkv, Lk);
  if (!workspace || workspace_bytes < need)
    return fail(DROPKV_E_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  float* sc = scores ? scores : reinterpret_cast<float*>(ws + p.total);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* sel_ws = ws + p.total + s_bytes;
  // The gather runs inside the selection's emit stage when the rows allow
  // 16-byte copies; otherwise as its own kernel (contiguous outputs only).
  const int64_t eb = elem_size(dtype);
  const bool vec = (D * eb) % 16 == 0 && aligned16(k_out) && aligned16(v_out);
  if (!vec && out_ld != keep)
    return fail(DROPKV_E_UNSUPPORTED, "outputs with a row capacity need 16-byte aligned rows");
  timing_start(st);
  const dkv::SelectCompact cp{k, v, Hkv * kv_ld * D, kv_ld * D, D, eb, D, (int)Hkv, k_out, v_out, out_ld};
  // Pooling runs in the tail of the scoring pass when the plan allows it
  // (the matrix-core kernels only); otherwise as the standalone selection's
  // pool kernel.  Where pass 2 cannot run the whole selection in its tail,
  // the selection continues in its own kernels after the scores.
  const bool mfma = !dkv::scores_generic(dtype, D, p.M);
  const bool fused = mfma && dkv::select_after_pool_ok(p.s2, p.kps2, Lk, kernel_size);
  int tail_done = 0;
  const dkv::FuseSelect fs{sel_ws,   (int)kernel_size,        (int)protect_window, (int)keep,
                           keep_idx, vec ? &cp : nullptr, &tail_done};
  hipError_t e = dkv::launch_scores(p, dtype, (int)D, q, q_sb, q_sh, q_ss, q_sd, k, v, (int)kv_ld, (int)Hkv, (int)Lq,
                                    (int)Lk, (int)W, eps, p_round ? 1 : 0, y_round ? 1 : 0, sc, ws,
                                    reinterpret_cast<uint32_t*>(sel_ws), dkv::select_zero_words(B * Hkv),
                                    fused ? &fs : nullptr, st);
  if (e != hipSuccess) return hip_status(e, "dropkv_evict scores");
  if (tail_done)
    e = hipSuccess;
  else if (fused)
    e = dkv::launch_select_after_pool(sc, (int)(B * Hkv), (int)Lk, (int)kernel_size, (int)protect_window, (int)keep,
                                      p.s2, p.kps2, keep_idx, nullptr, sel_ws, vec ? &cp : nullptr, st);
  else
    e = dkv::launch_select(sc, (int)(B * Hkv), (int)Lk, (int)kernel_size, (int)protect_window, (int)keep, keep_idx,
                           nullptr, sel_ws, true, vec ? &cp : nullptr, st);
  if (e != hipSuccess) return hip_status(e, "dropkv_evict select");
  if (vec) return DROPKV_OK;
  e = dkv::launch_compact(k, v, Hkv * kv_ld * D, kv_ld * D, D, Lk, nullptr, nullptr, 0, 0, 0, 0, eb, B, Hkv, D,
                          keep_idx, keep, k_out, v_out, st);
  return hip_status(e, "dropkv_evict compact");
}

int dropkv_evict(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, const void* k, const void* v,
                 int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D, int64_t W,
                 float eps, int p_round, int y_round, int64_t splits, int64_t kernel_size, int64_t protect_window,
                 int64_t keep, float* scores, int64_t* keep_idx, void* k_out, void* v_out, void* workspace,
                 size_t workspace_bytes, void* stream) {
  return evict_impl(q, q_sb, q_sh, q_ss, q_sd, k, v, Lk, dtype, B, Hq, Hkv, Lq, Lk, D, W, eps, p_round, y_round,
                    splits, kernel_size, protect_window, keep, scores, keep_idx, k_out, v_out, keep, workspace,
                    workspace_bytes, stream);
}

}  // extern "C"

// Scratch of dropkv_evict_noalloc: one copy per GPU, for the life of the
// process.  In host code `scratch` names a host-side stand-in, not device
// memory: every host use goes through the per-device address that
// hipGetSymbolAddress returns (noalloc_scratch).
static __device__ __align__(256) unsigned char scratch[DROPKV_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch` per device ordinal

// The current device's copy of `scratch`, looked up once per device (with
// that device current); the stream must belong to the current device.
int noalloc_scratch(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxScratchDevices) return fail(DROPKV_E_UNSUPPORTED, "device ordinal %d too large", dev);
  if (st) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess) return hip_status(e, "hipStreamGetDevice");
    if (sdev != dev)
      return fail(DROPKV_E_ARG, "stream belongs to device %d, the current device is %d", (int)sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(DROPKV_E_HIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DROPKV_OK;
}
}  // namespace

extern "C" {

int dropkv_evict_noalloc(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, const void* k,
                         const void* v, int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk,
                         int64_t D, int64_t W, float eps, int p_round, int y_round, int64_t splits,
                         int64_t kernel_size, int64_t protect_window, int64_t keep, float* scores,
                         int64_t* keep_idx, void* k_out, void* v_out, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  int rc = check_score_args(q, k, v, dtype, B, Hq, Hkv, Lq, Lk, D, W);
  if (rc) return rc;
  const size_t need = dropkv_evict_workspace_bytes(B, Hq, Hkv, Lk, D, W, splits);
  if (need > DROPKV_NOALLOC_SCRATCH_BYTES)
    return fail(DROPKV_E_UNSUPPORTED,
                "dropkv_evict_noalloc: this shape needs %zu bytes of scratch, above the maximum of %zu; "
                "use dropkv_evict with a workspace",
                need, (size_t)DROPKV_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = noalloc_scratch(static_cast<hipStream_t>(stream), &ws);
  if (rc) return rc;
  return evict_impl(q, q_sb, q_sh, q_ss, q_sd, k, v, Lk, dtype, B, Hq, Hkv, Lq, Lk, D, W, eps, p_round, y_round,
                    splits, kernel_size, protect_window, keep, scores, keep_idx, k_out, v_out, keep, ws,
                    DROPKV_NOALLOC_SCRATCH_BYTES, stream);
}

int dropkv_evict_ld(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd, const void* k,
                    const void* v, int64_t kv_ld, int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq,
                    int64_t Lk, int64_t D, int64_t W, float eps, int p_round, int y_round, int64_t splits,
                    int64_t kernel_size, int64_t protect_window, int64_t keep, float* scores, int64_t* keep_idx,
                    void* k_out, void* v_out, int64_t out_ld, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return evict_impl(q, q_sb, q_sh, q_ss, q_sd, k, v, kv_ld, dtype, B, Hq, Hkv, Lq, Lk, D, W, eps, p_round, y_round,
                    splits, kernel_size, protect_window, keep, scores, keep_idx, k_out, v_out, out_ld, workspace,
                    workspace_bytes, stream);
}

int dropkv_append(const void* k, const void* v, int64_t s_b, int64_t s_h, int64_t s_l, int64_t elem_bytes,
                  int64_t B, int64_t H, int64_t L, int64_t D, void* k_dst, void* v_dst, int64_t dst_ld, int64_t row0,
                  void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    return fail(DROPKV_E_ARG, "elem_bytes must be 1, 2, 4 or 8");
  if (B < 0 || H < 0 || L < 0 || D < 1 || row0 < 0) return fail(DROPKV_E_ARG, "invalid shape");
  if (row0 + L > dst_ld) return fail(DROPKV_E_ARG, "rows %lld..%lld do not fit a capacity of %lld", (long long)row0,
                                     (long long)(row0 + L), (long long)dst_ld);
  if (L > 0 && B * H > 0 && (!k || !v || !k_dst || !v_dst)) return fail(DROPKV_E_ARG, "null pointer");
  timing_start(static_cast<hipStream_t>(stream));
  return hip_status(dkv::launch_append(k, v, s_b, s_h, s_l, elem_bytes, B, H, L, D, k_dst, v_dst, dst_ld, row0,
                                       static_cast<hipStream_t>(stream)),
                    "dropkv_append launch");
}

static_assert(DROPKV_SYNC_BYTES == dkv::kSyncBytes, "the header's sync area is the plan's");

int dropkv_set_tail_select(int mode, int64_t spin_polls, int64_t spin_polls_b) {
  if (mode != 0 && mode != 1) return fail(DROPKV_E_ARG, "mode must be 0 or 1");
  if (spin_polls > INT32_MAX || spin_polls_b > INT32_MAX) return fail(DROPKV_E_ARG, "spin_polls too large");
  dkv::set_tail_select(mode, spin_polls < 0 ? -1 : (int)spin_polls, spin_polls_b < 0 ? -1 : (int)spin_polls_b);
  return DROPKV_OK;
}

int dropkv_timing_enable(int on) {
  Timing& t = t_timing;
  (void)hipGetLastError();
  if (on && !t.created) {
    for (int i = 0; i < 2 * kMaxTimedKernels; ++i) {
      hipError_t e = hipEventCreate(&t.ev[i]);
      if (e != hipSuccess) {
        for (int j = 0; j < i; ++j) (void)hipEventDestroy(t.ev[j]);
        return hip_status(e, "hipEventCreate");
      }
    }
    t.created = true;
  }
  t.on = on != 0;
  t.n = 0;
  return DROPKV_OK;
}

int dropkv_timing_read(double* stage_ms, int cap) {
  Timing& t = t_timing;
  if (!stage_ms || cap < 0) return -fail(DROPKV_E_ARG, "null stage_ms");
  if (t.n < 1) return 0;
  hipError_t e = hipEventSynchronize(t.ev[2 * t.n - 1]);
  if (e != hipSuccess) return -hip_status(e, "hipEventSynchronize");
  for (int i = 0; i < t.n && i < cap; ++i) {
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, t.ev[2 * i], t.ev[2 * i + 1]);
    if (e != hipSuccess) return -hip_status(e, "hipEventElapsedTime");
    stage_ms[i] = ms;
  }
  return t.n;
}

size_t dropkv_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t capacity) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || capacity < 1 || !decode_head_dim_supported(D)) return 0;
  return dkv::decode_workspace_bytes((int)B, (int)Hq, (int)Hkv, (int)D, (int)capacity);
}

int dropkv_decode_attention(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sd, const void* k_new,
                            const void* v_new, int64_t n_sb, int64_t n_sh, int64_t n_sd, void* k_cache,
                            void* v_cache, const int32_t* n_rows, int dtype, int64_t B, int64_t Hq, int64_t Hkv,
                            int64_t D, int64_t capacity, float scale, void* out, int64_t o_sb, int64_t o_sh,
                            int64_t o_sd, void* workspace, size_t workspace_bytes, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !n_rows || !out || !workspace)
    return fail(DROPKV_E_ARG, "null pointer argument");
  if (dtype != DROPKV_BF16 && dtype != DROPKV_FP16) return fail(DROPKV_E_ARG, "dtype must be bf16 or fp16");
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv) return fail(DROPKV_E_ARG, "B, Hq, Hkv must be positive, Hkv | Hq");
  if (Hq / Hkv > 16) return fail(DROPKV_E_UNSUPPORTED, "more than 16 query heads per KV head");
  if (!decode_head_dim_supported(D)) return fail(DROPKV_E_UNSUPPORTED, "head dim %lld not supported", (long long)D);
  if (capacity < 1 || capacity * D * 2 > ((int64_t)1 << 31)) return fail(DROPKV_E_ARG, "capacity out of range");
  if (!aligned16(k_cache) || !aligned16(v_cache)) return fail(DROPKV_E_ARG, "cache buffers must be 16-byte aligned");
  if (workspace_bytes < dkv::decode_workspace_bytes((int)B, (int)Hq, (int)Hkv, (int)D, (int)capacity))
    return fail(DROPKV_E_ARG, "workspace too small");
  dkv::DecodeParams p{};
  p.q = q;
  p.q_sb = q_sb;
  p.q_sh = q_sh;
  p.q_sd = q_sd;
  p.kn = k_new;
  p.vn = v_new;
  p.n_sb = n_sb;
  p.n_sh = n_sh;
  p.n_sd = n_sd;
  p.kbuf = k_cache;
  p.vbuf = v_cache;
  p.n_rows = n_rows;
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.D = (int)D;
  p.C = (int)capacity;
  p.dtype_bf16 = dtype == DROPKV_BF16;
  p.scale = scale;
  p.out = out;
  p.o_sb = o_sb;
  p.o_sh = o_sh;
  p.o_sd = o_sd;
  p.workspace = workspace;
  timing_start(static_cast<hipStream_t>(stream));
  return hip_status(dkv::launch_decode_attention(p, static_cast<hipStream_t>(stream)), "decode launch");
}

int dropkv_selftest_mfma(float* out, void* stream) {
  (void)hipGetLastError();  // a failure left by an unrelated earlier call is not ours
  if (!out) return fail(DROPKV_E_ARG, "null out");
  return hip_status(dkv::launch_mfma_selftest(out, static_cast<hipStream_t>(stream)), "selftest launch");
}

}  // extern "C"
