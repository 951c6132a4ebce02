/*
 * dcr_oracle.c -- CPU restatement of DCR-Attention's sparse decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels in
 * dcr-attention_v3_amd/csrc; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product path never calls it.
 *
 * It restates the reference's M1 oracle,
 *   dcr_attention/kernel/qaxis_topk_reference.py:42-259,
 * step by step, with every floating-point order written out so that a GPU
 * kernel following the same order can be compared bit for bit:
 *
 *   oracle_compute_uq       _compute_u_Q                  (:42-55)
 *   oracle_scores           _compute_projection_scores    (:58-88)
 *   oracle_topk             _select_topk_indices          (:91-108)
 *                           + topk_axis_pass2.py:16-43 (int32 output)
 *   oracle_attention        _gather_kv + _fused_softmax_attention (:111-193)
 *   oracle_attention_f64    exact softmax attention over a selected set,
 *                           float64 (closed form, pins oracle_attention)
 *   oracle_dense_f64        exact dense decode attention over all N rows
 *                           (comparator, attention.py:673-739 semantics)
 *   oracle_rank_local_f64   exact rank-local (sorted-window) attention and
 *                           its log-sum-exp, float64: the mathematics of
 *                           rank_local_fwd_torch (rank_local_fwd_torch.py:
 *                           21-113) and _rank_local_fwd_kernel
 *                           (rank_local_fwd_triton.py:50-213)
 *
 * Floating-point orders (all fp32, round-to-nearest-even, no contraction
 * except where fmaf is written):
 *   norm   : 8 strided accumulators acc[j] = fmaf(x[8i+j], x[8i+j], acc[j]),
 *            then acc[0]+acc[1]+...+acc[7] left to right, then a scalar tail
 *            s = s + x*x for D % 8 != 0; norm = sqrtf(s); clamp at eps;
 *            u = x / norm (IEEE division).  This is the order torch's CPU
 *            vector-norm kernel uses on AVX2/AVX-512 hosts.
 *   score  : acc = +0; acc = fmaf(K[d], u[d], acc) for d = 0..D-1; the
 *            order an MKL sgemm micro-kernel uses for einsum('bnd,bhd->bnh').
 *            Rounded to bf16 with round-to-nearest-even (NaN -> 0x7FC0).
 *   attn   : 64-row tiles in ascending index order; logit = (sum_d fmaf) *
 *            scale; m/l/o carried in fp32 exactly as M1 step 4 does.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "dcr_oracle.h"

/* ---------------------------------------------------------------- dtypes */

static float f32_from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static uint32_t bits_from_f32(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* IEEE binary16 -> binary32, exact (normals, subnormals, inf, NaN). */
static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    if (exp == 0x1f) return f32_from_bits(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return f32_from_bits(sign);
        /* subnormal: man * 2^-24, exact in fp32 */
        float v = (float)man * 0x1p-24f;
        return sign ? -v : v;
    }
    return f32_from_bits(sign | ((exp + 112u) << 23) | (man << 13));
}

static float bf16_to_float(uint16_t b) { return f32_from_bits((uint32_t)b << 16); }

float oracle_load_elem(const void* p, int dtype, size_t i) {
    switch (dtype) {
        case ORACLE_F32: return ((const float*)p)[i];
        case ORACLE_F16: return half_to_float(((const uint16_t*)p)[i]);
        default: return bf16_to_float(((const uint16_t*)p)[i]);
    }
}

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = bits_from_f32(f);
    if (isnan(f)) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* ------------------------------------------------------------------ u_Q */

void oracle_compute_uq(const void* Q, int dtype, int rows, int D, float eps, float* u) {
    for (int r = 0; r < rows; ++r) {
        const size_t base = (size_t)r * D;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int d = 0;
        for (; d + 8 <= D; d += 8)
            for (int j = 0; j < 8; ++j) {
                float x = oracle_load_elem(Q, dtype, base + d + j);
                acc[j] = fmaf(x, x, acc[j]);
            }
        float s = acc[0];
        for (int j = 1; j < 8; ++j) s = s + acc[j];
        for (; d < D; ++d) {
            float x = oracle_load_elem(Q, dtype, base + d);
            float sq = x * x;
            s = s + sq;
        }
        float n = sqrtf(s);
        if (n < eps) n = eps; /* torch clamp(min=eps) */
        for (int e = 0; e < D; ++e) u[base + e] = oracle_load_elem(Q, dtype, base + e) / n;
    }
}

/* --------------------------------------------------------------- scores */

void oracle_scores(const void* K, int dtype, const float* u, int B, int Hkv, int n_rep, int N,
                   int D, uint16_t* scores) {
    const int H = Hkv * n_rep;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int g = 0; g < Hkv; ++g) {
            float row[512];
            for (int n = 0; n < N; ++n) {
                const size_t kb = (((size_t)b * Hkv + g) * N + n) * D;
                for (int d = 0; d < D; ++d) row[d] = oracle_load_elem(K, dtype, kb + d);
                for (int r = 0; r < n_rep; ++r) {
                    const int h = g * n_rep + r;
                    const float* uh = u + ((size_t)b * H + h) * D;
                    float acc = 0.0f;
                    for (int d = 0; d < D; ++d) acc = fmaf(row[d], uh[d], acc);
                    scores[((size_t)b * H + h) * N + n] = oracle_f32_to_bf16(acc);
                }
            }
        }
}

/* ---------------------------------------------------------------- top-K */

/* Ordering used by torch.argsort(descending=True, stable=True) on the
 * fp32-promoted bf16 scores: larger value first, NaN above everything,
 * -0 == +0, equal values keep ascending index order. */
typedef struct {
    float v;
    int32_t i;
} scored_t;

static int desc_stable_cmp(const void* a, const void* b) {
    const scored_t* x = (const scored_t*)a;
    const scored_t* y = (const scored_t*)b;
    int xn = isnan(x->v), yn = isnan(y->v);
    if (xn != yn) return xn ? -1 : 1;
    if (!xn) {
        if (x->v > y->v) return -1;
        if (x->v < y->v) return 1;
    }
    return (x->i < y->i) ? -1 : (x->i > y->i);
}

static int int_cmp(const void* a, const void* b) {
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

int oracle_topk(const uint16_t* scores, int rows, int N, int k, int32_t* idx) {
    if (k <= 0 || k > N) return -1;
#pragma omp parallel
    {
        scored_t* buf = (scored_t*)malloc(sizeof(scored_t) * (size_t)N);
#pragma omp for schedule(static)
        for (int r = 0; r < rows; ++r) {
            for (int n = 0; n < N; ++n) {
                buf[n].v = bf16_to_float(scores[(size_t)r * N + n]);
                buf[n].i = n;
            }
            /* (value desc, index asc) is a total order, so any sort is the
             * stable descending argsort of the reference. */
            qsort(buf, (size_t)N, sizeof(scored_t), desc_stable_cmp);
            int32_t* out = idx + (size_t)r * k;
            for (int j = 0; j < k; ++j) out[j] = buf[j].i;
            qsort(out, (size_t)k, sizeof(int32_t), int_cmp);
        }
        free(buf);
    }
    return 0;
}

/* ------------------------------------------------------------ attention */

void oracle_attention(const void* Q, const void* K, const void* V, int dtype, const int32_t* idx,
                      int B, int H, int Hkv, int N, int D, int k, float* O) {
    const int n_rep = H / Hkv;
    const float scale = 1.0f / sqrtf((float)D);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int g = h / n_rep;
            float q[512], o[512], s[64];
            for (int d = 0; d < D; ++d) {
                q[d] = oracle_load_elem(Q, dtype, ((size_t)b * H + h) * D + d);
                o[d] = 0.0f;
            }
            float m = -INFINITY, l = 0.0f;
            const int32_t* ix = idx + ((size_t)b * H + h) * k;
            const size_t kvb = ((size_t)b * Hkv + g) * N;
            for (int t0 = 0; t0 < k; t0 += 64) {
                const int tn = (k - t0 < 64) ? (k - t0) : 64;
                float tmax = -INFINITY;
                for (int j = 0; j < tn; ++j) {
                    const size_t row = (kvb + (size_t)ix[t0 + j]) * D;
                    float acc = 0.0f;
                    for (int d = 0; d < D; ++d)
                        acc = fmaf(q[d], oracle_load_elem(K, dtype, row + d), acc);
                    s[j] = acc * scale;
                    if (s[j] > tmax) tmax = s[j];
                }
                const float m_new = fmaxf(m, tmax);
                const float alpha = expf(m - m_new);
                float bsum = 0.0f;
                for (int j = 0; j < tn; ++j) {
                    s[j] = expf(s[j] - m_new);
                    bsum = bsum + s[j];
                }
                l = alpha * l + bsum;
                for (int d = 0; d < D; ++d) {
                    float acc = 0.0f;
                    for (int j = 0; j < tn; ++j) {
                        const size_t row = (kvb + (size_t)ix[t0 + j]) * D;
                        acc = fmaf(s[j], oracle_load_elem(V, dtype, row + d), acc);
                    }
                    o[d] = alpha * o[d] + acc;
                }
                m = m_new;
            }
            for (int d = 0; d < D; ++d) O[((size_t)b * H + h) * D + d] = o[d] / l;
        }
}

static void attention_f64_rows(const void* Q, const void* K, const void* V, int dtype,
                               const int32_t* idx, int B, int H, int Hkv, int N, int D, int k,
                               double* O) {
    const int n_rep = H / Hkv;
    const double scale = 1.0 / sqrt((double)D);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int g = h / n_rep;
            const size_t kvb = ((size_t)b * Hkv + g) * N;
            double* s = (double*)malloc(sizeof(double) * (size_t)k);
            double mx = -INFINITY;
            for (int j = 0; j < k; ++j) {
                const int n = idx ? idx[((size_t)b * H + h) * k + j] : j;
                double acc = 0.0;
                for (int d = 0; d < D; ++d)
                    acc += (double)oracle_load_elem(Q, dtype, ((size_t)b * H + h) * D + d) *
                           (double)oracle_load_elem(K, dtype, (kvb + n) * D + d);
                s[j] = acc * scale;
                if (s[j] > mx) mx = s[j];
            }
            double l = 0.0;
            for (int j = 0; j < k; ++j) {
                s[j] = exp(s[j] - mx);
                l += s[j];
            }
            for (int d = 0; d < D; ++d) {
                double acc = 0.0;
                for (int j = 0; j < k; ++j) {
                    const int n = idx ? idx[((size_t)b * H + h) * k + j] : j;
                    acc += s[j] * (double)oracle_load_elem(V, dtype, (kvb + n) * D + d);
                }
                O[((size_t)b * H + h) * D + d] = acc / l;
            }
            free(s);
        }
}

void oracle_attention_f64(const void* Q, const void* K, const void* V, int dtype, const int32_t* idx,
                          int B, int H, int Hkv, int N, int D, int k, double* O) {
    attention_f64_rows(Q, K, V, dtype, idx, B, H, Hkv, N, D, k, O);
}

void oracle_dense_f64(const void* Q, const void* K, const void* V, int dtype, int B, int H, int Hkv,
                      int N, int D, double* O) {
    attention_f64_rows(Q, K, V, dtype, NULL, B, H, Hkv, N, D, N, O);
}

/* ------------------------------------------------------------- pipeline */

int oracle_sparse_decode(const void* Q, const void* K, const void* V, int dtype, int B, int H,
                         int Hkv, int N, int D, int k, float eps, float* u, uint16_t* scores,
                         int32_t* idx, float* O) {
    if (H % Hkv != 0 || k <= 0 || k >= N || D > 512) return -1;
    oracle_compute_uq(Q, dtype, B * H, D, eps, u);
    oracle_scores(K, dtype, u, B, Hkv, H / Hkv, N, D, scores);
    if (oracle_topk(scores, B * H, N, k, idx) != 0) return -1;
    oracle_attention(Q, K, V, dtype, idx, B, H, Hkv, N, D, k, O);
    return 0;
}

/* --------------------------------------------------------- rank-local */

/* For each head bh and query i: rows 0 <= j < Nkv with |j - r| <= k_window / 2
 * (r = r_center[bh, i] as given: the reference's mask, rank_local_fwd_torch.py:
 * 84-87, rank_local_fwd_triton.py:138-153), logits (Q_i . K_j) * scale in
 * float64, softmax, O = sum p_j V_j, LSE = log sum exp(logit_j).  Two passes
 * over the window: the maximum, then the exponentials.  A window holding no
 * row gives O = 0 and LSE = -inf (the reference's empty rows:
 * rank_local_fwd_torch.py:104-108 nan_to_num, rank_local_fwd_triton.py:194-202). */
void oracle_rank_local_f64(const void* Q, const void* K, const void* V, int dtype,
                           const int32_t* r_center, int BH, int Nq, int Nkv, int D, int k_window,
                           double scale, double* O, double* lse) {
    const long long half = k_window / 2;
#pragma omp parallel for schedule(dynamic, 4)
    for (long long row = 0; row < (long long)BH * Nq; ++row) {
        const long long bh = row / Nq;
        const long long r = r_center[row];
        const long long lo = r - half > 0 ? r - half : 0;
        const long long hi = r + half + 1 < Nkv ? r + half + 1 : Nkv;
        if (lo >= hi) {
            for (int d = 0; d < D; ++d) O[(size_t)row * D + d] = 0.0;
            lse[row] = -INFINITY;
            continue;
        }
        double mx = -INFINITY;
        for (long long j = lo; j < hi; ++j) {
            double dot = 0.0;
            for (int d = 0; d < D; ++d)
                dot += (double)oracle_load_elem(Q, dtype, (size_t)row * D + d) *
                       (double)oracle_load_elem(K, dtype, ((size_t)bh * Nkv + j) * D + d);
            const double lg = dot * scale;
            if (lg > mx) mx = lg;
        }
        double l = 0.0;
        double* o = O + (size_t)row * D;
        for (int d = 0; d < D; ++d) o[d] = 0.0;
        for (long long j = lo; j < hi; ++j) {
            double dot = 0.0;
            for (int d = 0; d < D; ++d)
                dot += (double)oracle_load_elem(Q, dtype, (size_t)row * D + d) *
                       (double)oracle_load_elem(K, dtype, ((size_t)bh * Nkv + j) * D + d);
            const double p = exp(dot * scale - mx);
            l += p;
            for (int d = 0; d < D; ++d)
                o[d] += p * (double)oracle_load_elem(V, dtype, ((size_t)bh * Nkv + j) * D + d);
        }
        for (int d = 0; d < D; ++d) o[d] /= l;
        lse[row] = mx + log(l);
    }
}
