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
// h = k/2; it always holds row r (r is clamped to [0, Nkv)), so no window
// is empty.
//
// MI355X mapping: one workgroup of kRlWaves waves per (query block, bh).
//   * QPW mode (many queries, prefill): wave w serves query 4*blk + w over
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

// Rows j + u*RPI + rs of the tile starting at j; rows outside [lo, hi) are
// invalid and read row lo instead (always inside the head's rows).
template <int DT, int D>
__device__ __forceinline__ void rl_load(RlTile<DT, D>& t, const uint8_t* __restrict__ Kh,
                                        const uint8_t* __restrict__ Vh, int j, int lo, int hi,
                                        int rs, int li) {
    using G = RlGeom<DT, D>;
#pragma unroll
    for (int u = 0; u < kRlUnroll; ++u) {
        const int row = j + u * G::RPI + rs;
        t.valid[u] = row >= lo && row < hi;
        const size_t off = static_cast<size_t>(t.valid[u] ? row : lo) * G::RB + static_cast<size_t>(li) * 16;
        t.k[u] = *reinterpret_cast<const chunk_t*>(Kh + off);
        t.v[u] = *reinterpret_cast<const chunk_t*>(Vh + off);
    }
}

template <int DT, int D, bool SPLIT>
__global__ __launch_bounds__(64 * kRlWaves) void rank_local_kernel(
    const void* __restrict__ Q, const uint8_t* __restrict__ K, const uint8_t* __restrict__ V,
    const int32_t* __restrict__ rc, void* __restrict__ O, float* __restrict__ lse, int Nq, int Nkv,
    int half_k, float scale2) {
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

    // r_center is clamped to [0, Nkv) (prepare_sort_indices already does),
    // so every row read stays inside the head whatever the caller passes.
    int r = rc[bh * static_cast<size_t>(Nq) + qi];
    r = r < 0 ? 0 : (r >= Nkv ? Nkv - 1 : r);
    const int lo = r - half_k > 0 ? r - half_k : 0;
    const int hi = (r + half_k + 1 < Nkv) ? r + half_k + 1 : Nkv;
    const uint8_t* Kh = K + bh * static_cast<size_t>(Nkv) * G::RB;
    const uint8_t* Vh = V + bh * static_cast<size_t>(Nkv) * G::RB;
    // Tiles of this wave: aligned starts j = base + t*step.
    const int base = (lo / G::TILE) * G::TILE + (SPLIT ? w * G::TILE : 0);
    const int step = SPLIT ? W * G::TILE : G::TILE;

    RlTile<DT, D> buf[NB];
#pragma unroll
    for (int p = 0; p < NB; ++p) rl_load<DT, D>(buf[p], Kh, Vh, base + p * step, lo, hi, rs, li);
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
            rl_load<DT, D>(buf[p], Kh, Vh, j + (p + NB) * step, lo, hi, rs, li);
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
            for (int d = lane; d < D; d += 64) {
                float acc = 0.0f;
#pragma unroll
                for (int x = 0; x < W; ++x) acc = __builtin_fmaf(fx[x], red[x][2 + d], acc);
                store_out<DT>(O, orow + d, acc / L);
            }
            if (lane == 0) lse[bh * static_cast<size_t>(Nq) + i] = (Mw + log2f(L)) * kLn2;
        }
    } else if (active) {
        const size_t orow = (bh * static_cast<size_t>(Nq) + i) * D;
        if (rs == 0) {
#pragma unroll
            for (int e = 0; e < EPC; ++e) store_out<DT>(O, orow + li * EPC + e, o[e] / l);
        }
        if (lane == 0) lse[bh * static_cast<size_t>(Nq) + i] = (M + log2f(l)) * kLn2;
    }
}

template <int DT, int D>
hipError_t launch_rl_t(const void* Q, const void* K, const void* V, const int32_t* rc, void* O,
                       float* lse, int BH, int Nq, int Nkv, int half_k, float scale,
                       hipStream_t s) {
    const float scale2 = static_cast<float>(static_cast<double>(scale) * kLog2e);
    // Few queries (decode): the waves split each query's window.
    const bool split = static_cast<long long>(Nq) * BH < 4096;
    const auto K8 = static_cast<const uint8_t*>(K);
    const auto V8 = static_cast<const uint8_t*>(V);
    if (split) {
        launch_kernel(rank_local_kernel<DT, D, true>, dim3(static_cast<unsigned>(Nq), static_cast<unsigned>(BH)),
                      dim3(64 * kRlWaves), 0, s, Q, K8, V8, rc, O, lse, Nq, Nkv, half_k, scale2);
    } else {
        const unsigned blocks = static_cast<unsigned>((Nq + kRlWaves - 1) / kRlWaves);
        launch_kernel(rank_local_kernel<DT, D, false>, dim3(blocks, static_cast<unsigned>(BH)),
                      dim3(64 * kRlWaves), 0, s, Q, K8, V8, rc, O, lse, Nq, Nkv, half_k, scale2);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_rank_local(const void* Q, const void* K, const void* V, int dtype,
                             const int32_t* r_center, void* O, float* lse, int BH, int Nq, int Nkv,
                             int D, int half_k, float scale, hipStream_t s) {
#define DCR_RL_CASE(DTV, DV)                                                                     \
    if (dtype == DTV && D == DV)                                                                 \
        return launch_rl_t<DTV, DV>(Q, K, V, r_center, O, lse, BH, Nq, Nkv, half_k, scale, s);
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
