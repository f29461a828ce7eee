/*
 * dropkv_amd.h -- C ABI of the MI355X (gfx950) DropKV prefill KV-eviction path.
 *
 * Plain pointers, element strides and sizes; no framework types.  All device
 * pointers are HIP device memory; `stream` is a hipStream_t passed as void*
 * (NULL = the legacy default stream).  Every call only enqueues work on
 * `stream` and returns without synchronising.  Inputs are never written.
 *
 * Return value: 0 on success, otherwise a nonzero DROPKV_E_* code; the
 * message of the last failure on the calling thread is available from
 * dropkv_last_error().  Argument checks happen before anything is enqueued.
 *
 * Citations refer to the reference checkout (AozhongZhang/DropKV).
 */
#ifndef DROPKV_AMD_H
#define DROPKV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element type codes */
#define DROPKV_BF16 1
#define DROPKV_FP16 2
#define DROPKV_FP32 3  /* scoring and eviction only (not decode) */

/* status codes */
#define DROPKV_OK 0
#define DROPKV_E_ARG 1         /* invalid shape / argument */
#define DROPKV_E_UNSUPPORTED 2 /* valid but not implemented here (e.g. D) */
#define DROPKV_E_WORKSPACE 3   /* workspace too small */
#define DROPKV_E_HIP 4         /* HIP runtime error */

/* Library version (major*10000 + minor*100 + patch). */
int dropkv_version(void);

/* Message describing the last failure on this thread ("" if none). */
const char* dropkv_last_error(void);

/* Head dimensions of the matrix-core scoring kernels (bf16 / fp16 inputs);
 * writes up to `cap` values into `out` and returns how many exist.  Every
 * other head dimension up to 4096, fp32 inputs, and GQA groups of more than
 * 4096 query rows (g * W) are scored by generic fp32 kernels on the vector
 * ALUs with the same arguments and results. */
int dropkv_supported_head_dims(int64_t* out, int cap);

/* ------------------------------------------------------------------------
 * Scoring.  Replaces dropkv_scores_triton (dropkv_triton.py:643-828) and its
 * kernels _compute_logits_block / _dropkv_attn_fwd_kernel /
 * _dropkv_attn_fwd_split_kernel / _dropkv_reduce_kernel /
 * _dropkv_score_kernel (dropkv_triton.py:117-610); with y_round=1 and
 * W=min(window,Lq) it also serves the deployed scoring path of
 * DropKVCache._compute_keep_indices (dropkv_cache.py:401-460).
 *
 *   q      [B,Hq,Lq,D], arbitrary element strides q_s* (only the last W rows
 *          along Lq are read; query row w sits at key position Lk-W+w)
 *   k, v   [B,Hkv,Lk,D] contiguous, 16-byte aligned, same dtype as q
 *          (bf16, fp16 or fp32)
 *   scores [B,Hkv,Lk] fp32 contiguous (output)
 *   p_round 0: keep softmax probabilities in fp32; 1: round them to the input
 *          dtype before w = (p/(1-p+eps))^2 (match_pytorch_precision=True,
 *          dropkv_triton.py:584-587)
 *   y_round 0: attention output y in fp32; 1: y rounded to the input dtype
 *          (deployed path, dropkv_cache.py:434)
 *   splits 0 = automatic split-K depth over keys, otherwise that many splits
 *          per (b, hkv, row-chunk)
 * Requires Hq % Hkv == 0, 1 <= W <= Lq <= Lk, 1 <= D <= 4096, and
 * B*Hq*W and B*Hkv*Lk at most 2^31-1 (the workspace functions return 0
 * otherwise).
 * The first DROPKV_SYNC_BYTES of the workspace must be zero when a workspace
 * is first used; every call leaves them zero (see dropkv_evict).
 * ------------------------------------------------------------------------ */
size_t dropkv_scores_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Lk,
                                     int64_t D, int64_t W, int64_t splits);

int dropkv_scores(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd,
                  const void* k, const void* v, int dtype,
                  int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D,
                  int64_t W, float eps, int p_round, int y_round, int64_t splits,
                  float* scores, void* workspace, size_t workspace_bytes, void* stream);

/* Debug view of the scoring intermediates written by the last dropkv_scores
 * call into `workspace`: lse [B*Hkv, M] (natural log) and y [B*Hkv, M, D] fp32
 * (normalised attention output), M = (Hq/Hkv)*W.  Lets tests check the
 * A<->B contract sum_j exp(l_j - lse) == 1 (reference tests:170-236). */
int dropkv_scores_debug_state(const void* workspace, int64_t B, int64_t Hq, int64_t Hkv,
                              int64_t Lk, int64_t D, int64_t W, int64_t splits,
                              float* lse_out, float* y_out, void* stream);

/* ------------------------------------------------------------------------
 * Selection.  Replaces the pool / protect / top-k / sort sequence of
 * DropKVCache._compute_keep_indices (dropkv_cache.py:464-475):
 *   pooled = max_pool1d(scores, kernel_size, pad=kernel_size//2, stride 1)
 *   pooled[..., Lk-window:] = max(pooled) + 1.0f
 *   keep_idx = ascending indices of the `keep` largest pooled values, the
 *              lowest indices first among values equal to the threshold.
 *   scores   [rows, Lk] fp32 contiguous
 *   keep_idx [rows, keep] int64 (output)
 *   pooled   [rows, Lk] fp32 (optional output, may be NULL)
 * ------------------------------------------------------------------------ */
size_t dropkv_select_workspace_bytes(int64_t rows, int64_t Lk);

int dropkv_select(const float* scores, int64_t rows, int64_t Lk, int64_t kernel_size,
                  int64_t window, int64_t keep, int64_t* keep_idx, float* pooled,
                  void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Compaction.  Replaces DropKVCache._gather_compressed (dropkv_cache.py:479-491):
 *   k_out[b,h,i,:] = k[b,h,idx[b,h,i],:]   (same for v), bit-exact copies.
 * Sources have element strides (s_b, s_h, s_l) with the D axis contiguous;
 * outputs are contiguous [B,H,keep,D].  elem_bytes is 2 for bf16/fp16.
 * ------------------------------------------------------------------------ */
int dropkv_compact(const void* k, const void* v, int64_t s_b, int64_t s_h, int64_t s_l,
                   int64_t elem_bytes, int64_t B, int64_t H, int64_t L, int64_t D,
                   const int64_t* idx, int64_t keep, void* k_out, void* v_out, void* stream);

/* Two-segment compaction for the chunked-prefill continuation
 * (dropkv_cache.py:581-607): the logical sequence is seg0 (length L0, the
 * stored cache) followed by seg1 (length L1, the new chunk); index i < L0
 * reads seg0[i], otherwise seg1[i-L0].  Same output layout as dropkv_compact. */
int dropkv_compact2(const void* k0, const void* v0, int64_t s0_b, int64_t s0_h, int64_t s0_l,
                    int64_t L0,
                    const void* k1, const void* v1, int64_t s1_b, int64_t s1_h, int64_t s1_l,
                    int64_t L1,
                    int64_t elem_bytes, int64_t B, int64_t H, int64_t D,
                    const int64_t* idx, int64_t keep, void* k_out, void* v_out, void* stream);

/* ------------------------------------------------------------------------
 * One layer-call of prefill eviction: scores -> select -> compact, all
 * enqueued on `stream` by one call.  Equivalent to
 * DropKVCache._compute_keep_indices followed by _gather_compressed
 * (dropkv_cache.py:355-491) on the fast path.  `protect_window` is the
 * cache's window_size (the last protect_window keys are always kept, as
 * dropkv_cache.py:466-467), `W` the scoring window (min(window, Lq) on the
 * deployed path).  `scores` may be NULL (then it lives in the workspace).
 * Pooling and the top-k threshold run in the tail of the scoring kernel
 * whenever the plan allows it (three kernels per call), otherwise as the
 * standalone selection kernels.  kernel_size may be any positive odd number
 * (windows past 129 keys pool in two extra kernels).
 *
 * The first DROPKV_SYNC_BYTES of the workspace are reserved for call
 * counters: they must be zero when a workspace is first used (fill a new
 * workspace with zeros), and every call leaves them zero.  The rest of the
 * workspace needs no initialisation.  Calls that share a workspace must be
 * serialised (one stream), as for every workspace here.
 * ------------------------------------------------------------------------ */
#define DROPKV_SYNC_BYTES 4096
size_t dropkv_evict_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Lk,
                                    int64_t D, int64_t W, int64_t splits);

int dropkv_evict(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd,
                 const void* k, const void* v, int dtype,
                 int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D,
                 int64_t W, float eps, int p_round, int y_round, int64_t splits,
                 int64_t kernel_size, int64_t protect_window, int64_t keep,
                 float* scores, int64_t* keep_idx, void* k_out, void* v_out,
                 void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * dropkv_evict without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops with a
 * fixed memory budget, harnesses that forbid hipMalloc).  No counterpart in
 * the reference, which allocates per call.
 *
 * The scratch the kernels need lives in a static device array of
 * DROPKV_NOALLOC_SCRATCH_BYTES (32 MiB), one per GPU, held until the process
 * ends.  The first call on a device looks up its address there (make that
 * first call outside graph capture); no call allocates or frees anything.
 * Calls whose dropkv_evict_workspace_bytes exceeds the maximum return
 * DROPKV_E_UNSUPPORTED: 32 MiB covers a Llama-3.1-8B layer (B 1, Hq 32,
 * Hkv 8, D 128, W 8) up to 231544 keys and a Qwen2-0.5B layer (B 1, Hq 14,
 * Hkv 2, D 64, W 8) up to 992160 keys; the B4 Hq64 Hkv8 D128 W32 128K-key
 * stress shape needs 111.5 MiB and is refused.
 * Every call on one GPU uses the same scratch and leaves its contents
 * behind: calls that overlap on one GPU (two streams, or two threads) race
 * and must be serialised by the caller.  The caller initialises nothing (the
 * counters at the start of the scratch are zero when the library is loaded
 * and every call leaves them zero).  Arguments and results are those of
 * dropkv_evict.
 * ------------------------------------------------------------------------ */
#define DROPKV_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

int dropkv_evict_noalloc(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd,
                         const void* k, const void* v, int dtype,
                         int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D,
                         int64_t W, float eps, int p_round, int y_round, int64_t splits,
                         int64_t kernel_size, int64_t protect_window, int64_t keep,
                         float* scores, int64_t* keep_idx, void* k_out, void* v_out, void* stream);

/* ------------------------------------------------------------------------
 * Chunked prefill on preallocated capacity.  Replaces the torch.cat of the
 * stored K/V and the chunk and the gather that follows it in the
 * evict_accumulated branch of DropKVCache.update (dropkv_cache.py:581-607),
 * and the torch.cat of the accumulate branches (dropkv_cache.py:571-579,
 * :618-620), for a cache that keeps each layer's K/V in buffers of a fixed
 * row capacity.
 *
 * dropkv_append: rows 0 .. L-1 of each head of k / v ([B,H,L,D], element
 * strides s_b, s_h, s_l, D contiguous) are copied, bit for bit, to rows
 * row0 .. row0+L-1 of k_dst / v_dst ([B,H,dst_ld,D] contiguous).
 * Requires row0 + L <= dst_ld.
 *
 * dropkv_evict_ld: dropkv_evict on K/V held in [B,Hkv,kv_ld,D] buffers (rows
 * 0 .. Lk-1 of each head are the sequence) that writes the compressed rows
 * to rows 0 .. keep-1 of [B,Hkv,out_ld,D] buffers.  Requires kv_ld >= Lk,
 * out_ld >= keep and, when out_ld > keep, 16-byte aligned rows.  The output
 * buffers must not overlap the inputs.  With kv_ld = Lk and out_ld = keep it
 * is dropkv_evict.
 * ------------------------------------------------------------------------ */
int dropkv_append(const void* k, const void* v, int64_t s_b, int64_t s_h, int64_t s_l, int64_t elem_bytes,
                  int64_t B, int64_t H, int64_t L, int64_t D, void* k_dst, void* v_dst, int64_t dst_ld,
                  int64_t row0, void* stream);

int dropkv_evict_ld(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_sd,
                    const void* k, const void* v, int64_t kv_ld, int dtype,
                    int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D,
                    int64_t W, float eps, int p_round, int y_round, int64_t splits,
                    int64_t kernel_size, int64_t protect_window, int64_t keep,
                    float* scores, int64_t* keep_idx, void* k_out, void* v_out, int64_t out_ld,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Where the layer-calls' selection runs (no counterpart in the reference,
 * whose pooling, top-k and gather are separate torch ops).  mode 1 (the
 * default): dropkv_evict / dropkv_evict_ld / dropkv_evict_noalloc finish the
 * selection (threshold, ordered emit of keep_idx, K/V gather) in the tail of
 * the scoring kernel whenever the call allows it (matrix-core scoring with at
 * most two 32-row query chunks per KV head, each split's scores in LDS, and
 * every workgroup of the scoring grid running at once on the GPU); its
 * workgroups then wait for one another twice per call.  mode 0: the
 * selection always runs as two further kernels.  Both give the same
 * results.  A workgroup that has waited spin_polls polls at the first wait
 * (default 65536, a few tens of milliseconds) leaves its row to the row's
 * last workgroup to arrive, which finishes the row alone; one that has
 * waited spin_polls_b polls at the second wait (default 4194304, seconds)
 * finishes the whole row alone itself.  Either way the outputs are the same
 * bits.  A limit < 0 leaves it unchanged; 0 forces that path (tests).
 * Process-wide: a call reads the settings once when it is enqueued. */
int dropkv_set_tail_select(int mode, int64_t spin_polls, int64_t spin_polls_b);

/* Kernel timing with HIP events (no counterpart in the reference, which has
 * no timers).  dropkv_timing_enable(1) makes every later dropkv_scores /
 * dropkv_select / dropkv_compact / dropkv_compact2 / dropkv_evict /
 * dropkv_evict_ld / dropkv_append / dropkv_decode_attention call on the calling thread launch its kernels with
 * hipExtLaunchKernel and a (start, stop) event pair each, which the runtime
 * sets to that dispatch's own begin and end time stamps.  dropkv_timing_read
 * waits for the last kernel of the most recent such call, writes the
 * execution time in milliseconds of each of its kernels, in launch order,
 * into stage_ms (at most cap values) and returns the number of kernels (0 if
 * none were timed, a negative status code on error).  The times exclude the
 * dispatch gaps between kernels.  At most 16 kernels per call are timed;
 * only the most recent call is kept; not for use while a stream is being
 * captured into a graph. */
int dropkv_timing_enable(int on);
int dropkv_timing_read(double* stage_ms, int cap);

/* Self-test of the matrix-core operand layout the kernels assume: computes a
 * 16x16 fp32 product of fixed bf16 patterns with one MFMA and writes it to
 * `out` (256 floats, device memory), row-major. */
int dropkv_selftest_mfma(float* out, void* stream);

/* ------------------------------------------------------------------------
 * Decode on the compressed cache.  Replaces the decode branch of
 * DropKVCache.update (dropkv_cache.py:609-617: torch.cat of the new row onto
 * the stored K/V) together with the attention the model then runs over the
 * concatenation (torch SDPA in the reference's Transformers integration,
 * patches/dropkv_transformers.patch:206-213).
 *
 * k_cache / v_cache: [B, Hkv, capacity, D] contiguous buffers whose first
 * *n_rows rows (device int32) are filled.  One call stores the new token's
 * rows k_new / v_new ([B, Hkv, 1, D], element strides n_*) at row *n_rows
 * and writes softmax(q K^T * scale) V over rows 0 .. *n_rows into out
 * ([B, 1, Hq, D], element strides o_*) for the query q ([B, Hq, 1, D],
 * element strides q_*), the GQA group of query head h being KV head
 * h / (Hq / Hkv).  *n_rows is read on the device and not advanced: the
 * caller adds 1 after the step (so a captured graph replays every step).
 * Requires *n_rows < capacity; larger values are clamped to capacity - 1 and
 * overwrite the last row.  Hq / Hkv <= 16, D in dropkv_supported_head_dims.
 * The workspace (dropkv_decode_workspace_bytes) holds the split partials.
 * ------------------------------------------------------------------------ */
size_t dropkv_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t capacity);
int dropkv_decode_attention(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_sd, const void* k_new,
                            const void* v_new, int64_t n_sb, int64_t n_sh, int64_t n_sd, void* k_cache,
                            void* v_cache, const int32_t* n_rows, int dtype, int64_t B, int64_t Hq, int64_t Hkv,
                            int64_t D, int64_t capacity, float scale, void* out, int64_t o_sb, int64_t o_sh,
                            int64_t o_sd, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DROPKV_AMD_H */
