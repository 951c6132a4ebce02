/*
 * dcr_oracle.h -- CPU restatement of the reference's M1 sparse decode oracle
 * (dcr_attention/kernel/qaxis_topk_reference.py:42-259).
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; never linked into the product.
 *
 * Layouts (row-major, contiguous):
 *   Q [B, H, D], K/V [B, Hkv, N, D], u [B, H, D] fp32,
 *   scores [B, H, N] bf16 bits, idx [B, H, k] int32 ascending, O [B, H, D].
 * dtype codes: 0 = fp32, 1 = fp16, 2 = bf16 (same codes as the C-ABI).
 * D <= 512.
 */
#ifndef DCR_ORACLE_H
#define DCR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_BF16 = 2 };

float oracle_load_elem(const void* p, int dtype, size_t i);
uint16_t oracle_f32_to_bf16(float f);

/* _compute_u_Q, qaxis_topk_reference.py:42-55 */
void oracle_compute_uq(const void* Q, int dtype, int rows, int D, float eps, float* u);

/* _compute_projection_scores, qaxis_topk_reference.py:58-88 */
void oracle_scores(const void* K, int dtype, const float* u, int B, int Hkv, int n_rep, int N,
                   int D, uint16_t* scores);

/* _select_topk_indices, qaxis_topk_reference.py:91-108 (int32 like
 * topk_axis_pass2.py:43).  Returns -1 if k is out of (0, N]. */
int oracle_topk(const uint16_t* scores, int rows, int N, int k, int32_t* idx);

/* _gather_kv + _fused_softmax_attention, qaxis_topk_reference.py:111-193 */
void oracle_attention(const void* Q, const void* K, const void* V, int dtype, const int32_t* idx,
                      int B, int H, int Hkv, int N, int D, int k, float* O);

/* Exact (float64) softmax attention over the selected rows. */
void oracle_attention_f64(const void* Q, const void* K, const void* V, int dtype, const int32_t* idx,
                          int B, int H, int Hkv, int N, int D, int k, double* O);

/* Exact (float64) dense decode attention over all N rows. */
void oracle_dense_f64(const void* Q, const void* K, const void* V, int dtype, int B, int H, int Hkv,
                      int N, int D, double* O);

/* Exact (float64) rank-local window attention over sorted K/V [BH, Nkv, D]:
 * rank_local_fwd_torch, rank_local_fwd_torch.py:21-113.  O [BH, Nq, D],
 * lse [BH, Nq] (natural log). */
void oracle_rank_local_f64(const void* Q, const void* K, const void* V, int dtype,
                           const int32_t* r_center, int BH, int Nq, int Nkv, int D, int k_window,
                           double scale, double* O, double* lse);

/* topk_qaxis_attention_reference, qaxis_topk_reference.py:200-259.
 * Returns -1 for invalid shapes (the reference raises). */
int oracle_sparse_decode(const void* Q, const void* K, const void* V, int dtype, int B, int H,
                         int Hkv, int N, int D, int k, float eps, float* u, uint16_t* scores,
                         int32_t* idx, float* O);

#ifdef __cplusplus
}
#endif
#endif
