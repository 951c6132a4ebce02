// rank_local.hip -- rank-local (sorted-window) attention forward.
//
// Replaces the reference's _rank_local_fwd_kernel / rank_local_fwd_triton
// (dcr_attention/kernel/rank_local_fwd_triton.py:50-213, launcher :216-334;
// CPU twin rank_local_fwd_torch, rank_local_fwd_torch.py:21-113):
//
//   O[bh,i] = sum_{j : |j - r[bh,i]| <= k/2} softmax_j(Q[bh,i]·K[bh,j] * scale) V[bh,j]
//   LSE[bh,i] = log sum_j exp(Q[bh,i]·K[bh,j] * scale)   (natural log)
//
// over keys and values already sorted along the ordering axis, with fp32
// logits and softmax state and one rounding at the output.  The window of
// query i is the contiguous row range [max(0, r-h), min(Nkv, r+h+1)),
// h = k/2, with r as the caller passes it (the reference applies the mask
// |j - r| <= h to r unclamped, rank_local_fwd_triton.py:138-153); a window
// that misses every row (r < -h or r > Nkv - 1 + h) gives O = 0 and
// LSE = -inf, as the reference's empty-row case (:194-202).
//
// MI355X mapping.  Many queries (prefill) in fp16/bf16 run on the matrix
// cores (rank_local_mfma_kernel below: 64 queries per workgroup).  Otherwise
// one workgroup of kRlWaves waves per (query block, bh):
//   * QPW mode (many fp32 queries): wave w serves query 4*blk + w over
//     its whole window.  The queries of a block are consecutive in sorted
//     order, so their windows nearly coincide and the rows one wave loads are
//     re-read from L1/L2 by the others.
//   * SPLIT mode (few queries, decode): the waves of a workgroup split the
//     window of one query (wave w takes tiles w, w + 4, ...), and merge their
//     (m, l, o) states in LDS.
// A row is LPR lanes x 16 bytes, one wave instruction covers RPI rows and a
// tile is U instructions; two tile buffers per wave keep a tile in flight
// while the other is computed.  Each row slot keeps its own online-softmax
// state in base 2 (logits scaled by log2 e), merged once at the end.
#include <math.h>

#include "dcr_common.h"
#include "dcr_kernels.h"

namespace dcr {
namespace {

constexpr int kRlWaves = 4;
constexpr int kRlUnroll = 4;
constexpr int kRlBuffers = 2;

template <int DT, int D>
struct RlGeom {
    static constexpr int EB = ElemBytes<DT>::value;
    static constexpr int RB = D * EB;     // bytes per row
    static constexpr int LPR = RB / 16;   // lanes per row
    static constexpr int RPI = 64 / LPR;  // rows per wave instruction
    static constexpr int EPC = 16 / EB;   // elements per lane
    static constexpr int TILE = RPI * kRlUnroll;
};

template <int LPR>
__device__ __forceinline__ float rl_row_sum(float v) {
    // Sum over the LPR consecutive lanes of a row (all of them get it).
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int DT, int D>
struct RlTile {
    chunk_t k[kRlUnroll], v[kRlUnroll];
    bool valid[kRlUnroll];
};

// Where a head's sorted key/value rows live.  Sorted copies: row j of head
// bh at (bh * Nkv + j).  PERM: the caller's cache read through the sort
// permutation, row j of query head bh = row perm[bh][j] of KV head
// (b, h / n_rep), rows of KV head kvh at kvh * head_rows (the cache's row
// stride between heads); permutation entries are clamped to [0, Nkv).
struct RlSource {
    const int32_t* perm;
    long long head_rows;
    int H, n_rep;
};

// Window [lo, hi) of a query centred at r (as given) with half-width h,
// clipped to the rows [0, Nkv); empty (lo >= hi) when r is more than h rows
// outside them.  64-bit sums: r may be any int32.
__device__ __forceinline__ void rl_window(int r, int half_k, int Nkv, int& lo, int& hi) {
    const long long l = static_cast<long long>(r) - half_k;
    const long long h = static_cast<long long>(r) + half_k + 1;
    lo = static_cast<int>(l > 0 ? (l < Nkv ? l : Nkv) : 0);
    hi = static_cast<int>(h < Nkv ? (h > 0 ? h : 0) : Nkv);
}

template <bool PERM>
__device__ __forceinline__ size_t rl_head_base(const RlSource& src, size_t bh, int Nkv) {
    if constexpr (PERM) {
        const size_t b = bh / static_cast<size_t>(src.H), h = bh % static_cast<size_t>(src.H);
        const size_t kvh = b * static_cast<size_t>(src.H / src.n_rep) + h / static_cast<size_t>(src.n_rep);
        return kvh * static_cast<size_t>(src.head_rows);
    } else {
        return bh * static_cast<size_t>(Nkv);
    }
}

template <bool PERM>
__device__ __forceinline__ int rl_phys(const int32_t* __restrict__ perm_h, int r, int Nkv) {
    if constexpr (PERM) {
        const int p = perm_h[r];
        return p < 0 ? 0 : (p >= Nkv ? Nkv - 1 : p);
    } else {
        return r;
    }
}

// Rows j + u*RPI + rs of the tile starting at j; rows outside [lo, hi) are
// invalid and read row lo instead (always inside the head's rows).
template <int DT, int D, bool PERM>
__device__ __forceinline__ void rl_load(RlTile<DT, D>& t, const uint8_t* __restrict__ Kh,
                                        const uint8_t* __restrict__ Vh, int j, int lo, int hi,
                                        int rs, int li, const int32_t* __restrict__ perm_h, int Nkv) {
    using G = RlGeom<DT, D>;
#pragma unroll
    for (int u = 0; u < kRlUnroll; ++u) {
        const int row = j + u * G::RPI + rs;
        t.valid[u] = row >= lo && row < hi;
        const int pr = rl_phys<PERM>(perm_h, t.valid[u] ? row : lo, Nkv);
        const size_t off = static_cast<size_t>(pr) * G::RB + static_cast<size_t>(li) * 16;
        t.k[u] = *reinterpret_cast<const chunk_t*>(Kh + off);
        t.v[u] = *reinterpret_cast<const chunk_t*>(Vh + off);
    }
}

template <int DT, int D, bool SPLIT, bool PERM>
__global__ __launch_bounds__(64 * kRlWaves) void rank_local_kernel(
    const void* __restrict__ Q, const uint8_t* __restrict__ K, const uint8_t* __restrict__ V,
    const int32_t* __restrict__ rc, void* __restrict__ O, float* __restrict__ lse, int Nq, int Nkv,
    int half_k, float scale2, RlSource src) {
    using G = RlGeom<DT, D>;
    constexpr int LPR = G::LPR, EPC = G::EPC, U = kRlUnroll, NB = kRlBuffers, W = kRlWaves;
    static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "row must tile a wave");
    __shared__ float red[W][D + 2];

    const int lane = lane_id();
    const int w = static_cast<int>(threadIdx.x >> 6);
    const size_t bh = blockIdx.y;
    const int i = SPLIT ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.x) * W + w;
    const int li = lane % LPR;
    const int rs = lane / LPR;
    const bool active = i < Nq;
    const int qi = active ? i : Nq - 1;

    // The window clipped to the head's rows (every row read stays inside
    // them: invalid slots read row lo, and lo < Nkv whenever a tile runs).
    int lo, hi;
    rl_window(rc[bh * static_cast<size_t>(Nq) + qi], half_k, Nkv, lo, hi);
    const size_t hb = rl_head_base<PERM>(src, bh, Nkv);
    const uint8_t* Kh = K + hb * G::RB;
    const uint8_t* Vh = V + hb * G::RB;
    const int32_t* perm_h = PERM ? src.perm + bh * static_cast<size_t>(Nkv) : nullptr;
    // Tiles of this wave: aligned starts j = base + t*step.
    const int base = (lo / G::TILE) * G::TILE + (SPLIT ? w * G::TILE : 0);
    const int step = SPLIT ? W * G::TILE : G::TILE;

    RlTile<DT, D> buf[NB];
#pragma unroll
    for (int p = 0; p < NB; ++p) rl_load<DT, D, PERM>(buf[p], Kh, Vh, base + p * step, lo, hi, rs, li, perm_h, Nkv);
    float q[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e)
        q[e] = load_elem<DT>(Q, (bh * static_cast<size_t>(Nq) + qi) * D + li * EPC + e);

    float m = -INFINITY, l = 0.0f;
    float o[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) o[e] = 0.0f;

    for (int j = base; j < hi; j += NB * step) {
#pragma unroll
        for (int p = 0; p < NB; ++p) {
            const RlTile<DT, D>& cur = buf[p];
            float s[U];
            float tmax = -INFINITY;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < EPC; ++e) acc = __builtin_fmaf(q[e], chunk_elem<DT>(cur.k[u], e), acc);
                acc = rl_row_sum<LPR>(acc);
                s[u] = cur.valid[u] ? acc * scale2 : -INFINITY;
                tmax = fmaxf(tmax, s[u]);
            }
            const float m_new = fmaxf(m, tmax);
            if (m_new != -INFINITY) {
                const float alpha = exp2_hw(m - m_new);
                l *= alpha;
#pragma unroll
                for (int e = 0; e < EPC; ++e) o[e] *= alpha;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const float pr = cur.valid[u] ? exp2_hw(s[u] - m_new) : 0.0f;
                    l += pr;
#pragma unroll
                    for (int e = 0; e < EPC; ++e) o[e] = __builtin_fmaf(pr, chunk_elem<DT>(cur.v[u], e), o[e]);
                }
                m = m_new;
            }
            rl_load<DT, D, PERM>(buf[p], Kh, Vh, j + (p + NB) * step, lo, hi, rs, li, perm_h, Nkv);
        }
    }

    // Merge the row slots (lanes with the same slice li).
    float M = m;
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    const float f = (m == -INFINITY) ? 0.0f : exp2_hw(m - M);
    l *= f;
#pragma unroll
    for (int e = 0; e < EPC; ++e) o[e] *= f;
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
        l += __shfl_xor(l, off, 64);
#pragma unroll
        for (int e = 0; e < EPC; ++e) o[e] += __shfl_xor(o[e], off, 64);
    }

    constexpr float kLn2 = 0.6931471805599453f;
    if constexpr (SPLIT) {
        // Merge the waves' states in LDS; wave 0 writes the row.
        if (lane == 0) {
            red[w][0] = M;
            red[w][1] = l;
        }
        if (rs == 0) {
#pragma unroll
            for (int e = 0; e < EPC; ++e) red[w][2 + li * EPC + e] = o[e];
        }
        __syncthreads();
        if (w == 0 && active) {
            float Mw = -INFINITY;
#pragma unroll
            for (int x = 0; x < W; ++x) Mw = fmaxf(Mw, red[x][0]);
            float L = 0.0f;
            float fx[W];
#pragma unroll
            for (int x = 0; x < W; ++x) {
                fx[x] = (red[x][0] == -INFINITY) ? 0.0f : exp2_hw(red[x][0] - Mw);
                L = __builtin_fmaf(fx[x], red[x][1], L);
            }
            const size_t orow = (bh * static_cast<size_t>(Nq) + i) * D;
            // An empty window (L = 0) gives O = 0 and LSE = -inf.
            for (int d = lane; d < D; d += 64) {
                float acc = 0.0f;
#pragma unroll
                for (int x = 0; x < W; ++x) acc = __builtin_fmaf(fx[x], red[x][2 + d], acc);
                store_out<DT>(O, orow + d, L > 0.0f ? acc / L : 0.0f);
            }
            if (lane == 0) lse[bh * static_cast<size_t>(Nq) + i] = L > 0.0f ? (Mw + log2f(L)) * kLn2 : -INFINITY;
        }
    } else if (active) {
        const size_t orow = (bh * static_cast<size_t>(Nq) + i) * D;
        if (rs == 0) {
#pragma unroll
            for (int e = 0; e < EPC; ++e) store_out<DT>(O, orow + li * EPC + e, l > 0.0f ? o[e] / l : 0.0f);
        }
        if (lane == 0) lse[bh * static_cast<size_t>(Nq) + i] = l > 0.0f ? (M + log2f(l)) * kLn2 : -INFINITY;
    }
}

// ---------------------------------------------------------------------------
// Matrix-core prefill path (fp16 / bf16, scale > 0): a workgroup of 4 waves
// takes 64 consecutive (sorted) queries, 16 per wave, and walks 64-row tiles
// of the union of their windows.  Per tile the workgroup stages K (row-major)
// and V^T in LDS (two buffers, one barrier per tile); per wave:
//   S^T (64 keys x 16 queries) = K_tile · Q^T    v_mfma_f32_16x16x16 (f16/bf16),
//       exact products, fp32 accumulation;
//   masked online softmax per query in base 2 and fp32, with the scale folded
//       into the exponent's FMA: p = 2^(s·c - m·c), c = scale·log2(e) > 0, so
//       the running max m is kept on the raw dot products;
//   O (16 queries x D) += P · V_tile   the same MFMA, with P split into a high
//       and a low 16-bit part (P = hi + lo to ~2^-18 relative), so the
//       products keep the precision of an fp32 P·V.
// Computing S^T rather than S puts lane l's probabilities where the A operand
// of P·V wants them (query l % 16, keys 4*(l/16) + j): no transpose between
// the products.  MFMA 16x16x16 lane layout (checked on gfx950):
// A[l%16][4*(l/16)+j], B[4*(l/16)+j][l%16], D[4*(l/16)+v][l%16].
// A wave skips tiles outside all its queries' windows and masks only tiles
// that cross one of their window edges.  LDS row strides of D + 8 (K) and
// 72 (V^T) halves put the 16 rows one lane group reads on distinct 4-bank
// groups, so the operand reads are conflict-free.
typedef _Float16 rl_half4 __attribute__((ext_vector_type(4)));
typedef float rl_f32x4 __attribute__((ext_vector_type(4)));
typedef short rl_short4 __attribute__((ext_vector_type(4)));
typedef float rl_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 rl_bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t rl_u32x2 __attribute__((ext_vector_type(2)));

constexpr int kRlBq = 64;             // queries per workgroup
constexpr int kRlTk = 64;             // keys per tile
constexpr int kRlVstr = kRlTk + 8;    // V^T row stride (halves)

template <int DT>
struct RlMfma;
template <>
struct RlMfma<kF16> {
    typedef rl_half4 op;
    static __device__ __forceinline__ rl_f32x4 mma(op a, op b, rl_f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
    // (p0, p1) = hi + lo as packed pairs, truncating conversions: the low
    // part holds the high part's error to |e| < 2^-20 p.
    static __device__ __forceinline__ void split2(float p0, float p1, uint32_t& hi, uint32_t& lo) {
        const auto h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
        const auto r = __builtin_amdgcn_cvt_pkrtz(p0 - static_cast<float>(h[0]), p1 - static_cast<float>(h[1]));
        hi = __builtin_bit_cast(uint32_t, h);
        lo = __builtin_bit_cast(uint32_t, r);
    }
};
template <>
struct RlMfma<kBF16> {
    typedef rl_short4 op;
    static __device__ __forceinline__ rl_f32x4 mma(op a, op b, rl_f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    }
    // Round-to-nearest conversions: |e| < 2^-18 p.
    static __device__ __forceinline__ void split2(float p0, float p1, uint32_t& hi, uint32_t& lo) {
        const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(rl_f32x2{p0, p1}, rl_bf16x2));
        const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xffff0000u);
        hi = hb;
        lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(rl_f32x2{p0 - h0, p1 - h1}, rl_bf16x2));
    }
};

template <int DT, int D, bool PERM>
__global__ __launch_bounds__(256) void rank_local_mfma_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const int32_t* __restrict__ rc, uint16_t* __restrict__ O, float* __restrict__ lse, int Nq,
    int Nkv, int half_k, float scale2, RlSource src) {
    using M = RlMfma<DT>;
    using op = typename M::op;
    constexpr int NC = D / 16;                    // 16-wide d chunks
    constexpr int KSTR = D + 8;                   // K tile row stride (halves), 16-byte aligned
    constexpr int VSTR = kRlVstr;
    constexpr int CPR = D / 8;                    // 16-byte chunks per row
    constexpr int KCH = kRlTk * CPR;              // K chunks per tile
    constexpr int KPT = (KCH + 255) / 256;
    constexpr int VPAIRS = (kRlTk / 4) * CPR;     // (4-row group, chunk) pairs per tile
    constexpr int VPT = (VPAIRS + 255) / 256;
    __shared__ __align__(16) uint16_t Klds[2][kRlTk * KSTR];
    __shared__ __align__(16) uint16_t Vt[2][D * VSTR];
    __shared__ int sh_lo[4], sh_hi[4];

    const int t = static_cast<int>(threadIdx.x);
    const int lane = lane_id();
    const int w = t >> 6;
    const int g = lane >> 4;                 // lane group: k / row offset 4*g
    const int ln = lane & 15;                // query (S^T column) / d within a chunk
    const size_t bh = blockIdx.y;
    const int q0 = static_cast<int>(blockIdx.x) * kRlBq + 16 * w;
    const int qa = q0 + ln < Nq ? q0 + ln : Nq - 1;      // this lane's query (S^T layout)
    const uint16_t* Qh = Q + bh * static_cast<size_t>(Nq) * D;
    const size_t hb = rl_head_base<PERM>(src, bh, Nkv);
    const uint16_t* Kh = K + hb * D;
    const uint16_t* Vh = V + hb * D;
    const int32_t* perm_h = PERM ? src.perm + bh * static_cast<size_t>(Nkv) : nullptr;

    int lo_q, hi_q;                                                  // window [lo_q, hi_q)
    rl_window(rc[bh * static_cast<size_t>(Nq) + qa], half_k, Nkv, lo_q, hi_q);
    if (lo_q >= hi_q) {   // empty: [Nkv, 0) leaves the wave's union and mask logic unchanged
        lo_q = Nkv;
        hi_q = 0;
    }
    const uint32_t win = hi_q > lo_q ? static_cast<uint32_t>(hi_q - lo_q) : 0u;

    // The wave's union [wlo, whi) and intersection [wlo_in, whi_in) of windows.
    int wlo = lo_q, whi = hi_q, wlo_in = lo_q, whi_in = hi_q;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
        wlo = min(wlo, __shfl_xor(wlo, off, 64));
        whi = max(whi, __shfl_xor(whi, off, 64));
        wlo_in = max(wlo_in, __shfl_xor(wlo_in, off, 64));
        whi_in = min(whi_in, __shfl_xor(whi_in, off, 64));
    }
    if (lane == 0) {
        sh_lo[w] = wlo;
        sh_hi[w] = whi;
    }
    __syncthreads();
    const int ulo = min(min(sh_lo[0], sh_lo[1]), min(sh_lo[2], sh_lo[3]));
    const int uhi = max(max(sh_hi[0], sh_hi[1]), max(sh_hi[2], sh_hi[3]));

    // Q^T operand (B): lane l holds Q[query l%16][16c + 4g .. +3].
    op qB[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
        qB[c] = *reinterpret_cast<const op*>(Qh + static_cast<size_t>(qa) * D + 16 * c + 4 * g);

    float m = -INFINITY, l = 0.0f;       // raw running max, sum of 2^(s·c - m·c)
    rl_f32x4 o[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) o[c] = rl_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Tile staging.  K: thread t moves 16-byte chunks t, t + 256, ...
    // (row-major copy).  V: thread t moves the chunk at column pid / 16 of
    // rows 4*(pid % 16) .. +3 for pid = t, t + 256, ...: the four rows' halves
    // of one head-dim element are packed into one 8-byte V^T store.
    chunk_t kreg[KPT], vreg[VPT][4];
    auto gload = [&](int tile) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int cid = t + 256 * i;
            if (KCH % 256 == 0 || cid < KCH) {
                int gr = tile + cid / CPR;
                gr = rl_phys<PERM>(perm_h, gr < Nkv ? gr : Nkv - 1, Nkv);
                kreg[i] = *reinterpret_cast<const chunk_t*>(Kh + static_cast<size_t>(gr) * D + (cid % CPR) * 8);
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pid = t + 256 * i;
            if (VPAIRS % 256 == 0 || pid < VPAIRS) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    int gr = tile + 4 * (pid % 16) + rr;
                    gr = rl_phys<PERM>(perm_h, gr < Nkv ? gr : Nkv - 1, Nkv);
                    vreg[i][rr] = *reinterpret_cast<const chunk_t*>(Vh + static_cast<size_t>(gr) * D + (pid / 16) * 8);
                }
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int cid = t + 256 * i;
            if (KCH % 256 == 0 || cid < KCH)
                *reinterpret_cast<chunk_t*>(&Klds[buf][(cid / CPR) * KSTR + (cid % CPR) * 8]) = kreg[i];
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int pid = t + 256 * i;
            if (VPAIRS % 256 == 0 || pid < VPAIRS) {
                uint16_t* dst = &Vt[buf][(pid / 16) * 8 * VSTR + 4 * (pid % 16)];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t a0 = vreg[i][0][e / 2], a1 = vreg[i][1][e / 2];
                    const uint32_t a2 = vreg[i][2][e / 2], a3 = vreg[i][3][e / 2];
                    const uint32_t x = (e & 1) ? ((a0 >> 16) | (a1 & 0xffff0000u)) : ((a0 & 0xffffu) | (a1 << 16));
                    const uint32_t y = (e & 1) ? ((a2 >> 16) | (a3 & 0xffff0000u)) : ((a2 & 0xffffu) | (a3 << 16));
                    *reinterpret_cast<uint2*>(dst + e * VSTR) = make_uint2(x, y);
                }
            }
        }
    };

    const int t0 = (ulo / kRlTk) * kRlTk;
    gload(t0);
    int buf = 0;
    for (int tile = t0; tile < uhi; tile += kRlTk, buf ^= 1) {
        // Writes buffer buf: every wave has finished the tile two steps back
        // (it passed the previous barrier after computing it).
        lstore(buf);
        __syncthreads();
        if (tile + kRlTk < uhi) gload(tile + kRlTk);   // next tile in flight during compute
        if (tile >= whi || tile + kRlTk <= wlo) continue;   // outside all of this wave's windows
        const uint16_t* Kb = Klds[buf];
        const uint16_t* Vb = Vt[buf];

        // S^T subtiles: keys 16n + 4g + v, query ln (raw dot products).
        rl_f32x4 st[4];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            st[n] = rl_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const op a = *reinterpret_cast<const op*>(Kb + (16 * n + ln) * KSTR + 16 * c + 4 * g);
                st[n] = M::mma(a, qB[c], st[n]);
            }
        }
        if (!(tile >= wlo_in && tile + kRlTk <= whi_in)) {   // the tile crosses a window edge
#pragma unroll
            for (int n = 0; n < 4; ++n)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int j = tile + 16 * n + 4 * g + v;
                    st[n][v] = static_cast<uint32_t>(j - lo_q) < win ? st[n][v] : -INFINITY;
                }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int n = 0; n < 4; ++n)
            tmax = fmaxf(fmaxf(tmax, fmaxf(st[n][0], st[n][1])), fmaxf(st[n][2], st[n][3]));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m, tmax);
        const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;   // no key seen yet: l = o = 0
        const float alpha = exp2_hw((m - m_use) * scale2);
        const float mc = m_use * scale2;
        float psum = 0.0f;
        op phi[4], plo[4];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            float p[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                p[v] = exp2_hw(__builtin_fmaf(st[n][v], scale2, -mc));
                psum += p[v];
            }
            uint32_t h01, l01, h23, l23;
            M::split2(p[0], p[1], h01, l01);
            M::split2(p[2], p[3], h23, l23);
            phi[n] = __builtin_bit_cast(op, rl_u32x2{h01, h23});
            plo[n] = __builtin_bit_cast(op, rl_u32x2{l01, l23});
        }
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        l = l * alpha + psum;
        m = m_new;

        // O rows are queries 4g + v: their alpha comes from lane 4g + v.
        float a4[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) a4[v] = __shfl(alpha, 4 * g + v, 64);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int v = 0; v < 4; ++v) o[c][v] *= a4[v];
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                const op b = *reinterpret_cast<const op*>(Vb + (16 * c + ln) * VSTR + 16 * n + 4 * g);
                o[c] = M::mma(phi[n], b, o[c]);
                o[c] = M::mma(plo[n], b, o[c]);
            }
        }
    }

    // O[q][d] / l_q for the lane's rows q = 4g + v, d = 16c + ln.
    float linv[4];   // an empty window (l = 0) gives O = 0
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const float lq = __shfl(l, 4 * g + v, 64);
        linv[v] = lq > 0.0f ? 1.0f / lq : 0.0f;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int q = q0 + 4 * g + v;
        if (q < Nq) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
                store_out<DT>(O, (bh * static_cast<size_t>(Nq) + q) * D + 16 * c + ln, o[c][v] * linv[v]);
        }
    }
    if (g == 0 && q0 + ln < Nq) {
        constexpr float kLn2 = 0.6931471805599453f;
        lse[bh * static_cast<size_t>(Nq) + q0 + ln] = l > 0.0f ? (m * scale2 + log2f(l)) * kLn2 : -INFINITY;
    }
}

template <int DT, int D, bool PERM>
hipError_t launch_rl_t(const void* Q, const void* K, const void* V, const int32_t* rc, void* O,
                       float* lse, int BH, int Nq, int Nkv, int half_k, float scale,
                       const RlSource& src, hipStream_t s) {
    const float scale2 = static_cast<float>(static_cast<double>(scale) * kLog2e);
    // Few queries (decode): the waves split each query's window.
    const bool split = static_cast<long long>(Nq) * BH < 4096;
    const auto K8 = static_cast<const uint8_t*>(K);
    const auto V8 = static_cast<const uint8_t*>(V);
    if constexpr (DT != kF32) {
        // The matrix-core kernel keeps its running max on raw dot products,
        // which needs a positive scale; other scales take the VALU kernel.
        if (!split && scale2 > 0.0f && scale2 <= 3.4e38f) {
            const unsigned blocks = static_cast<unsigned>((Nq + kRlBq - 1) / kRlBq);
            launch_kernel(rank_local_mfma_kernel<DT, D, PERM>, dim3(blocks, static_cast<unsigned>(BH)), dim3(256),
                          0, s, static_cast<const uint16_t*>(Q), static_cast<const uint16_t*>(K),
                          static_cast<const uint16_t*>(V), rc, static_cast<uint16_t*>(O), lse, Nq, Nkv,
                          half_k, scale2, src);
            return hipGetLastError();
        }
    }
    if (split) {
        launch_kernel(rank_local_kernel<DT, D, true, PERM>,
                      dim3(static_cast<unsigned>(Nq), static_cast<unsigned>(BH)), dim3(64 * kRlWaves), 0, s, Q,
                      K8, V8, rc, O, lse, Nq, Nkv, half_k, scale2, src);
    } else {
        const unsigned blocks = static_cast<unsigned>((Nq + kRlWaves - 1) / kRlWaves);
        launch_kernel(rank_local_kernel<DT, D, false, PERM>, dim3(blocks, static_cast<unsigned>(BH)),
                      dim3(64 * kRlWaves), 0, s, Q, K8, V8, rc, O, lse, Nq, Nkv, half_k, scale2, src);
    }
    return hipGetLastError();
}

template <int DT, int D>
hipError_t launch_rl_any(const void* Q, const void* K, const void* V, const int32_t* rc, void* O,
                         float* lse, int BH, int Nq, int Nkv, int half_k, float scale,
                         const int32_t* perm, long long head_rows, int H, int n_rep, hipStream_t s) {
    const RlSource src{perm, head_rows, H, n_rep};
    if (perm != nullptr) return launch_rl_t<DT, D, true>(Q, K, V, rc, O, lse, BH, Nq, Nkv, half_k, scale, src, s);
    return launch_rl_t<DT, D, false>(Q, K, V, rc, O, lse, BH, Nq, Nkv, half_k, scale, src, s);
}

}  // namespace

hipError_t launch_rank_local(const void* Q, const void* K, const void* V, int dtype,
                             const int32_t* r_center, void* O, float* lse, int BH, int Nq, int Nkv,
                             int D, int half_k, float scale, const int32_t* perm, long long head_rows,
                             int H, int n_rep, hipStream_t s) {
#define DCR_RL_CASE(DTV, DV)                                                                     \
    if (dtype == DTV && D == DV)                                                                 \
        return launch_rl_any<DTV, DV>(Q, K, V, r_center, O, lse, BH, Nq, Nkv, half_k, scale, perm, head_rows, H, \
                                      n_rep, s);
    DCR_RL_CASE(kF32, 32)
    DCR_RL_CASE(kF16, 32)
    DCR_RL_CASE(kBF16, 32)
    DCR_RL_CASE(kF32, 64)
    DCR_RL_CASE(kF16, 64)
    DCR_RL_CASE(kBF16, 64)
    DCR_RL_CASE(kF32, 128)
    DCR_RL_CASE(kF16, 128)
    DCR_RL_CASE(kBF16, 128)
#undef DCR_RL_CASE
    return hipErrorInvalidValue;
}

}  // namespace dcr
