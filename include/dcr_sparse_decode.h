/*
 * dcr_sparse_decode.h -- C ABI of libdcr_sparse_decode.so, the MI355X (gfx950)
 * implementation of DCR-Attention's sparse decode path.
 *
 * Every entry point replaces one function of the reference's Triton path
 * (Seqev/dcr-attention_v3, dcr_attention/kernel/triton/) or of its M1 oracle
 * (dcr_attention/kernel/qaxis_topk_reference.py), cited per function below.
 *
 * Conventions
 *   - All tensors are device pointers to row-major arrays:
 *       Q [B, H, D], u [B, H, D] fp32, scores [B, H, N] bf16 bit patterns,
 *       idx [B, H, k] int32, O [B, H, D] in the dtype of Q/K/V, contiguous;
 *       K/V [B, Hkv, N, D] with rows of D contiguous elements, row n of KV
 *       head (b, g) at element ((b*Hkv + g)*ldn + n)*D.  ldn >= N is the
 *       number of rows between consecutive KV heads: N for a contiguous
 *       cache, the capacity of a preallocated cache [B, Hkv, N_max, D], or
 *       n_rep*N for every n_rep-th head of a GQA-repeated [B, H, N, D]
 *       tensor (the un-repeat view K[:, ::n_rep], read without a copy).
 *   - dtype codes: DCR_F32, DCR_F16, DCR_BF16.  Q, K and V share one dtype.
 *   - Supported shapes: D in {64, 128}; n_rep = H / Hkv in {1, 2, 4, 8};
 *     top-k needs 0 < k < N <= 16777216 (rows longer than 131072 take the chunked select).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream);
 *     nothing synchronises.  Scratch memory comes from the caller's
 *     `workspace` (size from the matching *_workspace_bytes function, 256-byte
 *     alignment); the library allocates nothing per call.  Calls that share a
 *     workspace must not overlap in time.
 *   - Return value: DCR_OK or a negative dcr_status; dcr_last_error() gives a
 *     message for the calling thread's last failure.
 */
#ifndef DCR_SPARSE_DECODE_H
#define DCR_SPARSE_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* dcr_stream_t; /* hipStream_t */

enum dcr_dtype { DCR_F32 = 0, DCR_F16 = 1, DCR_BF16 = 2 };

enum dcr_status {
    DCR_OK = 0,
    DCR_ERR_INVALID_ARG = -1, /* null pointer, bad shape, dtype or k */
    DCR_ERR_UNSUPPORTED = -2, /* valid but outside the built kernels (D, n_rep, N) */
    DCR_ERR_WORKSPACE = -3,   /* workspace missing or smaller than required */
    DCR_ERR_HIP = -4          /* a kernel launch failed */
};

/* Library ABI version (bumped on any signature change). */
int dcr_abi_version(void);
/* Static text for a status code. */
const char* dcr_status_string(int status);
/* Message describing the calling thread's last failed call ("" if none). */
const char* dcr_last_error(void);

/* u = Q / max(||Q||_2, eps), fp32, per row of D elements.
 * Replaces _compute_u_Q (qaxis_topk_reference.py:42-55), which the Triton
 * path calls from topk_axis.py:47. */
int dcr_compute_uq(const void* Q, int dtype, float* uQ, int rows, int D, float eps,
                   dcr_stream_t stream);

/* scores[b, g*n_rep + r, n] = bf16(sum_d K[b,g,n,d] * u[b, g*n_rep + r, d]).
 * Replaces topk_pass1_projection (topk_axis_pass1.py:104-153). */
int dcr_score_pass(const void* K, int dtype, const float* uQ, uint16_t* scores, int B, int Hkv,
                   int n_rep, int N, int ldn, int D, dcr_stream_t stream);

/* Ascending int32 indices of the k largest scores of each of `rows` rows
 * (stable: ties go to the lower index).
 * Replaces topk_pass2_select (topk_axis_pass2.py:16-43). */
size_t dcr_topk_select_workspace_bytes(int rows, int N);
int dcr_topk_select(const uint16_t* scores, int32_t* idx, int rows, int N, int k, void* workspace,
                    size_t workspace_bytes, dcr_stream_t stream);

/* Softmax attention of each query head over its k gathered K/V rows
 * (indices must lie in [0, N); rows outside are skipped).
 * Replaces fused_topk_attention (fused_attn.py:158-211). */
size_t dcr_gather_attn_workspace_bytes(int B, int H, int Hkv, int D, int k);
int dcr_gather_attn(const void* Q, const void* K, const void* V, int dtype, const int32_t* idx,
                    void* O, int B, int H, int Hkv, int N, int ldn, int D, int k,
                    void* workspace, size_t workspace_bytes, dcr_stream_t stream);

/* u_Q + score pass + top-k select (u_Q is computed inside the score kernel).
 * Replaces topk_qaxis_select (topk_axis.py:20-55). */
size_t dcr_qaxis_select_workspace_bytes(int B, int H, int Hkv, int N, int D, int dtype);
int dcr_qaxis_select(const void* Q, const void* K, int dtype, int32_t* idx, int B, int H, int Hkv,
                     int N, int ldn, int D, int k, float eps, void* workspace,
                     size_t workspace_bytes, dcr_stream_t stream);

/* The whole sparse decode op: score pass (with u_Q and the level-1
 * histogram fused in), top-k select, gather + attention, combine -- in one
 * launch or three (dcr_set_sparse_path).  idx_out may be NULL (the indices
 * are then not written out).
 * Replaces topk_qaxis_attention (topk_axis.py:58-90). */
size_t dcr_sparse_decode_workspace_bytes(int B, int H, int Hkv, int N, int D, int k, int dtype);
int dcr_sparse_decode(const void* Q, const void* K, const void* V, int dtype, void* O,
                      int32_t* idx_out, int B, int H, int Hkv, int N, int ldn, int D, int k,
                      float eps, void* workspace, size_t workspace_bytes, dcr_stream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): dcr_sparse_decode with its workspace taken from a static
 * device array of DCR_STATIC_SCRATCH_BYTES inside the library instead of a
 * caller buffer.  Each GPU holds its own copy of the array from the first call
 * on that device until the process ends; the call itself allocates nothing.
 * Shapes whose dcr_sparse_decode_workspace_bytes exceeds the maximum are
 * rejected with DCR_ERR_WORKSPACE.  Every call on a GPU shares that GPU's
 * array: calls that overlap in time on one GPU (other streams, other host
 * threads) race and must be serialised by the caller.  Nothing in the array
 * needs to be zero on entry.  Same arguments, results and errors as
 * dcr_sparse_decode otherwise. */
#define DCR_STATIC_SCRATCH_BYTES (32u * 1024u * 1024u)
int dcr_sparse_decode_static(const void* Q, const void* K, const void* V, int dtype, void* O,
                             int32_t* idx_out, int B, int H, int Hkv, int N, int ldn, int D, int k,
                             float eps, dcr_stream_t stream);

/* No counterpart in the reference (a control of this implementation).  Which
 * launch sequence dcr_sparse_decode / dcr_sparse_decode_static run,
 * process-wide:
 *   DCR_PATH_AUTO     the library's choice; currently DCR_PATH_CLASSIC, the
 *                     fastest measured on MI355X for every benchmark shape
 *                     (default);
 *   DCR_PATH_CLASSIC  three launches: score pass, top-k select writing each
 *                     query head's index list, attention over the lists;
 *   DCR_PATH_FUSED    one launch for the whole step where the shape allows it
 *                     (fp16/bf16, D in {64, 128}, n_rep in {1, 2, 4}, B*Hkv a
 *                     multiple of 8 with B*Hkv/8 dividing 32) on a 256-CU
 *                     device with nothing else running, DCR_PATH_CLASSIC
 *                     otherwise;
 *   DCR_PATH_UNION    three launches; for fp16 and bf16 the select kernel
 *                     passes each row's selection to the attention in closed
 *                     form and the attention reads every V row a GQA group
 *                     selected once (DCR_PATH_CLASSIC for fp32).
 * All give bit-identical indices and outputs within fp32 rounding of each
 * other.  Returns the previous setting, or a negative status. */
enum dcr_sparse_path { DCR_PATH_AUTO = 0, DCR_PATH_CLASSIC = 1, DCR_PATH_FUSED = 2, DCR_PATH_UNION = 3 };
int dcr_set_sparse_path(int path);

/* No counterpart in the reference (a control of this implementation, for
 * measuring the two forms of the score pass against each other).  Which form
 * the score pass of dcr_sparse_decode / dcr_qaxis_select runs, process-wide:
 *   DCR_SCORE_AUTO  a v_mfma_f32_4x4x1f32 chain where the group's heads fit
 *                   its operands (ceil(n_rep/4) * D <= 128), VALU FMAs
 *                   otherwise (default);
 *   DCR_SCORE_VALU  always the VALU form (u_Q by a separate launch, then a
 *                   per-lane FMA chain).
 * Both give bit-identical scores.  Returns the previous setting, or a
 * negative status. */
enum dcr_score_form { DCR_SCORE_AUTO = 0, DCR_SCORE_VALU = 1 };
int dcr_set_score_form(int form);

/* No counterpart in the reference.  How many kernel launches
 * dcr_sparse_decode makes for this shape on the current device under the
 * current dcr_set_sparse_path setting: 1 or 3, or a negative status for
 * arguments it would reject. */
int dcr_sparse_decode_launches(int B, int H, int Hkv, int N, int D, int k, int dtype);

/* No counterpart in the reference.  The library's sticky error word on the
 * current device: bit 0, a phase barrier of a one-launch (DCR_PATH_FUSED)
 * launch gave up waiting, after about 2 s; bit 1, a dcr_dense_decode launch
 * could not set up a merge ticket (a bounded retry loop ran out; not expected
 * in any correct use).  Either bit means that some launch's output is not
 * valid; 0 when every launch completed normally.  Synchronous (copies one
 * word); clear != 0 also resets it. */
int dcr_fused_errors(int clear, unsigned* errors);

/* Dense GQA decode attention over all N rows (fp32 softmax).  The caller's
 * comparator and its k >= N fallback: the decode case of _sdpa_forward
 * (attention.py:673-739) without materialising repeat_kv.  One launch (each
 * group's last workgroup merges the splits); nothing in the workspace needs
 * to be zero on entry, and calls that share a workspace must not overlap. */
size_t dcr_dense_decode_workspace_bytes(int B, int H, int Hkv, int N, int D);
int dcr_dense_decode(const void* Q, const void* K, const void* V, int dtype, void* O, int B, int H,
                     int Hkv, int N, int ldn, int D, void* workspace, size_t workspace_bytes,
                     dcr_stream_t stream);

/* Rank-local (sorted-window) attention forward: replaces rank_local_fwd_triton
 * (dcr_attention/kernel/rank_local_fwd_triton.py:216-334, kernel :50-213;
 * CPU twin rank_local_fwd_torch, rank_local_fwd_torch.py:21-113).
 * Q [BH, Nq, D], K_sorted / V_sorted [BH, Nkv, D] contiguous in one dtype,
 * r_center [BH, Nq] int32, outputs O [BH, Nq, D] in the dtype and lse [BH, Nq]
 * fp32 (natural log).  Query i of head bh attends to sorted positions
 * 0 <= j < Nkv with |j - r_center[bh, i]| <= k_window / 2, r_center used as
 * given (the reference's mask, rank_local_fwd_triton.py:138-153); a window
 * that holds no position gives O = 0 and lse = -inf (:194-202).
 * D in {32, 64, 128}; scale is the logit factor (1/sqrt(D) by default). */
int dcr_rank_local_fwd(const void* Q, const void* K_sorted, const void* V_sorted, int dtype,
                       const int32_t* r_center, void* O, float* lse, int BH, int Nq, int Nkv,
                       int D, int k_window, float scale, dcr_stream_t stream);

/* The same forward reading K and V in place through the sort permutation
 * instead of from sorted copies: row j of query head bh = b * H + h is row
 * perm[bh, j] of KV head (b, h / (H / Hkv)) of the cache, K/V [B, Hkv, ldn, D]
 * (rows 16-byte aligned, Nkv <= ldn), perm [B*H, Nkv] int32 (entries clamped to
 * [0, Nkv) on the device).  Replaces the gather-then-call sequence of
 * RankLocalAttentionFn.forward (dcr_attention/kernel/rank_local_attention.py:84-101:
 * gather_by_sort_idx of K and V, then rank_local_fwd_triton); the result is
 * bit-identical to running dcr_rank_local_fwd on the gathered copies.  Q, r_center,
 * O and lse as in dcr_rank_local_fwd (B*H heads). */
int dcr_rank_local_fwd_gather(const void* Q, const void* K, const void* V, int dtype,
                              const int32_t* perm, const int32_t* r_center, void* O, float* lse, int B,
                              int H, int Hkv, int Nq, int Nkv, int ldn, int D, int k_window, float scale,
                              dcr_stream_t stream);

/* Kernel timing for benchmarks (no counterpart in the reference, whose
 * harness times whole calls with torch.cuda.Event, test_m3_fused_attn.py:215-224).
 * While enabled, every kernel an entry point launches carries a pair of
 * hipEvents (hipExtLaunchKernelGGL start/stop events: the dispatch packet's
 * own begin and end times on its stream); nothing is recorded when disabled.
 * Not thread-safe: one profiling session per process at a time.  Measured on
 * ROCm 7: the first session after the process has freed and allocated device
 * memory again can include a one-time stall of a few milliseconds inside its
 * first launches (the kernels do run longer); repeated sessions over the same
 * buffers agree with rocprofv3.  Time a warm-up session first in that case. */
int dcr_profile_begin(void);
/* Waits for the recorded events, disables profiling and writes up to `max`
 * per-kernel aggregates (static name, summed microseconds, launch count).
 * Returns the number of entries, or a negative dcr_status. */
int dcr_profile_end(const char** names, double* total_us, int* launches, int max);

#ifdef __cplusplus
}
#endif
#endif /* DCR_SPARSE_DECODE_H */
