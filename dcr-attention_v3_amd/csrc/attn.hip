// attn.hip -- fused K/V gather + online-softmax GQA decode attention.
//
// Replaces the reference's Pass 3 (_pass3_fused_attn_kernel /
// fused_topk_attention, dcr_attention/kernel/triton/fused_attn.py:39-211;
// M1 twin _gather_kv + _fused_softmax_attention,
// qaxis_topk_reference.py:111-193):
//
//   O[b,h] = sum_j softmax_j(Q[b,h]·K[b,g,idx_j] * D^-1/2) V[b,g,idx_j],
//   g = h / n_rep, fp32 logits and fp32 (m, l, o) state, one rounding at
//   the output.
//
// MI355X mapping (split-k, FlashDecoding style; the reference runs one
// program per (b, h) with no split):
//   * grid (split, g, b); a workgroup holds the n_rep waves of one GQA
//     group, wave r serving query head g*n_rep + r.  All waves of a group
//     walk the same split of their (ascending) index lists at the same time,
//     so rows chosen by several heads of the group are fetched from HBM once
//     and re-read from L1/L2 by the others.
//   * a K (or V) row is D*elem bytes = LPR lanes x 16 bytes; one wave
//     instruction gathers RPI = 64/LPR rows, U instructions per tile, and the
//     next tile's indices and rows are loaded before the current tile is
//     used.  Each lane keeps q and o for its 16-byte slice of the head dim.
//   * the dot product is a per-lane FMA partial reduced over the LPR lanes of
//     a row with DPP adds; every row slot keeps its own online-softmax state
//     (m, l, o), so a tile needs no cross-lane max; slots merge once at the
//     end of the split.
//   * each wave writes its (m, l, o) partial; combine_kernel merges them (a
//     separate launch: merging inside the attention kernel would need a
//     device-scope fence per workgroup, which on MI355X writes back and
//     invalidates the XCD's L2 and throws away the shared-row reuse above).
// The dense comparator (all N rows, attention.py:673-739 semantics with an
// fp32 softmax) uses the same body with position = index.
#include <math.h>

#include "dcr_common.h"
#include "dcr_kernels.h"

namespace dcr {
namespace {

constexpr int kAttnUnroll = 4;

template <int DT, int D>
struct AttnGeom {
    static constexpr int EB = ElemBytes<DT>::value;
    static constexpr int RB = D * EB;      // bytes per row
    static constexpr int LPR = RB / 16;    // lanes per row
    static constexpr int RPI = 64 / LPR;   // rows per wave instruction
    static constexpr int EPC = 16 / EB;    // head-dim elements per lane
    static constexpr int TILE = RPI * kAttnUnroll;
};

// DPP lane permutations (gfx9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15-i within 16

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the LPR consecutive lanes that hold one row (all of them get it).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
    if constexpr (LPR >= 2) v += dpp<kDppQuadXor1>(v);
    if constexpr (LPR >= 4) v += dpp<kDppQuadXor2>(v);
    if constexpr (LPR >= 8) v += dpp<kDppHalfMirror>(v);
    if constexpr (LPR >= 16) v += dpp<kDppMirror>(v);
    if constexpr (LPR >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (LPR >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

template <int DT, int D>
struct Tile {
    chunk_t k[kAttnUnroll], v[kAttnUnroll];
    bool valid[kAttnUnroll];
};

// Gather the rows of tile positions [j, j + TILE) (row slot rs of each
// instruction); entries at or past j1, or with an index outside [0, N), are
// marked invalid and read row 0 instead (always mapped).
template <int DT, int D, bool DENSE>
__device__ __forceinline__ void load_tile(Tile<DT, D>& t, const uint8_t* __restrict__ Kg,
                                          const uint8_t* __restrict__ Vg,
                                          const int32_t* __restrict__ ix, int j, int j1, int rs,
                                          int N) {
    using G = AttnGeom<DT, D>;
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
        const int jj = j + u * G::RPI + rs;
        const bool in = jj < j1;
        int pos;
        if constexpr (DENSE)
            pos = jj;
        else
            pos = ix[in ? jj : j1 - 1];
        t.valid[u] = in && static_cast<unsigned>(pos) < static_cast<unsigned>(N);
        const size_t off = static_cast<size_t>(t.valid[u] ? pos : 0) * G::RB;
        t.k[u] = *reinterpret_cast<const chunk_t*>(Kg + off);
        t.v[u] = *reinterpret_cast<const chunk_t*>(Vg + off);
    }
}

// O[bh, :] = sum_c w_c o_c / sum_c w_c l_c, w_c = exp(m_c - max_c m_c): one
// wave per (b, h); lane c holds w_c (c < 64) and broadcasts it by shuffle, so
// the partial loads of the o loop are independent and pipeline.
template <int DT, int D>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ part,
                                                      void* __restrict__ O, int BH, int nsplit) {
    const size_t bh = static_cast<size_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (bh >= static_cast<size_t>(BH)) return;
    const int lane = lane_id();
    const float* pp = part + bh * static_cast<size_t>(nsplit) * (D + 2);
    constexpr int S = D + 2;

    float M = -INFINITY;
    for (int c = lane; c < nsplit; c += 64) M = fmaxf(M, pp[static_cast<size_t>(c) * S]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    float L = 0.0f, w_lane = 0.0f;
    for (int c = lane; c < nsplit; c += 64) {
        const float mc = pp[static_cast<size_t>(c) * S];
        const float w = (mc == -INFINITY) ? 0.0f : expf(mc - M);
        if (c < 64) w_lane = w;
        L = __builtin_fmaf(w, pp[static_cast<size_t>(c) * S + 1], L);
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) L += __shfl_xor(L, off, 64);

    float o[D / 64];
#pragma unroll
    for (int r = 0; r < D / 64; ++r) o[r] = 0.0f;
    const int n64 = nsplit < 64 ? nsplit : 64;
    for (int c0 = 0; c0 < n64; c0 += 8) {
        float w8[8], v8[8][D / 64];
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // eight independent loads in flight
            const int c = c0 + i;
            w8[i] = __shfl(w_lane, c & 63, 64);
#pragma unroll
            for (int r = 0; r < D / 64; ++r)
                v8[i][r] = (c < n64) ? pp[static_cast<size_t>(c) * S + 2 + r * 64 + lane] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < D / 64; ++r) o[r] = __builtin_fmaf(w8[i], v8[i][r], o[r]);
    }
    for (int c = 64; c < nsplit; ++c) {  // more than 64 splits: recompute weights
        const float mc = pp[static_cast<size_t>(c) * S];
        const float w = (mc == -INFINITY) ? 0.0f : expf(mc - M);
#pragma unroll
        for (int r = 0; r < D / 64; ++r)
            o[r] = __builtin_fmaf(w, pp[static_cast<size_t>(c) * S + 2 + r * 64 + lane], o[r]);
    }
#pragma unroll
    for (int r = 0; r < D / 64; ++r) store_out<DT>(O, bh * D + r * 64 + lane, o[r] / L);
}

template <int DT, int D, int NREP, bool DENSE>
__global__ __launch_bounds__((64 * NREP)) void attn_kernel(
    const void* __restrict__ Q, const uint8_t* __restrict__ K, const uint8_t* __restrict__ V,
    const int32_t* __restrict__ idx, float* __restrict__ part, int Hkv, int N, long long ldn, int k,
    int J, int nsplit, float scale) {
    using G = AttnGeom<DT, D>;
    constexpr int LPR = G::LPR, EPC = G::EPC, RB = G::RB, U = kAttnUnroll;
    static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "row must tile a wave");

    const int lane = lane_id();
    const int w = static_cast<int>(threadIdx.x >> 6);
    const int c = static_cast<int>(blockIdx.x);
    const int g = static_cast<int>(blockIdx.y);
    const int b = static_cast<int>(blockIdx.z);
    const int H = Hkv * NREP;
    const int h = g * NREP + w;
    const size_t bh = static_cast<size_t>(b) * H + h;
    const int li = lane % LPR;   // 16-byte slice of the row
    const int rs = lane / LPR;   // row slot within a wave instruction

    float q[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) q[e] = load_elem<DT>(Q, bh * D + li * EPC + e);

    const size_t kv_base = (static_cast<size_t>(b) * Hkv + g) * static_cast<size_t>(ldn) * RB +
                           static_cast<size_t>(li) * 16;
    const uint8_t* Kg = K + kv_base;
    const uint8_t* Vg = V + kv_base;
    const int32_t* ix = DENSE ? nullptr : idx + bh * static_cast<size_t>(k);
    const int total = DENSE ? N : k;
    const int j0 = c * J;
    const int j1 = (j0 + J < total) ? j0 + J : total;

    // Online-softmax state of this lane's row slot.
    float m = -INFINITY, l = 0.0f;
    float o[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) o[e] = 0.0f;

    Tile<DT, D> nxt;
    if (j0 < j1) load_tile<DT, D, DENSE>(nxt, Kg, Vg, ix, j0, j1, rs, N);
    for (int j = j0; j < j1; j += G::TILE) {
        const Tile<DT, D> cur = nxt;
        // Prefetch the next tile (past the end it re-reads this one: L1 hits).
        load_tile<DT, D, DENSE>(nxt, Kg, Vg, ix, (j + G::TILE < j1) ? j + G::TILE : j, j1, rs, N);

        float s[U];
        float tmax = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc = __builtin_fmaf(q[e], chunk_elem<DT>(cur.k[u], e), acc);
            acc = row_sum<LPR>(acc);
            s[u] = cur.valid[u] ? acc * scale : -INFINITY;
            tmax = fmaxf(tmax, s[u]);
        }
        const float m_new = fmaxf(m, tmax);
        if (m_new != -INFINITY) {
            const float alpha = expf(m - m_new);
            l *= alpha;
#pragma unroll
            for (int e = 0; e < EPC; ++e) o[e] *= alpha;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float p = cur.valid[u] ? expf(s[u] - m_new) : 0.0f;
                l += p;
#pragma unroll
                for (int e = 0; e < EPC; ++e) o[e] = __builtin_fmaf(p, chunk_elem<DT>(cur.v[u], e), o[e]);
            }
            m = m_new;
        }
    }

    // Merge the RPI row slots (lanes with the same slice li).
    float M = m;
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    const float f = (m == -INFINITY) ? 0.0f : expf(m - M);
    l *= f;
#pragma unroll
    for (int e = 0; e < EPC; ++e) o[e] *= f;
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
        l += __shfl_xor(l, off, 64);
#pragma unroll
        for (int e = 0; e < EPC; ++e) o[e] += __shfl_xor(o[e], off, 64);
    }
    float* pc = part + (bh * static_cast<size_t>(nsplit) + c) * (D + 2);
    if (lane == 0) {
        pc[0] = M;
        pc[1] = l;
    }
    if (rs == 0) {
#pragma unroll
        for (int e = 0; e < EPC; ++e) pc[2 + li * EPC + e] = o[e];
    }
}

// Rows per split: enough workgroups to fill the chip (~2 per CU), at least
// two tiles per wave.
int split_rows(int groups, int total, int tile) {
    const int target_splits = (512 + groups - 1) / groups;
    int J = (total + target_splits - 1) / target_splits;
    if (J < 2 * tile) J = 2 * tile;
    J = (J + tile - 1) / tile * tile;
    return J;
}

template <int DT, int D, int NREP, bool DENSE>
hipError_t launch_attn_t(const void* Q, const void* K, const void* V, const int32_t* idx,
                         float* part, void* O, int B, int Hkv, int N, long long ldn, int k,
                         int nsplit, hipStream_t s) {
    const int total = DENSE ? N : k;
    const int J = (total + nsplit - 1) / nsplit;
    const dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(D)));
    launch_kernel(attn_kernel<DT, D, NREP, DENSE>, grid, dim3(64 * NREP), 0, s,
        Q, static_cast<const uint8_t*>(K), static_cast<const uint8_t*>(V), idx, part, Hkv, N, ldn, k,
        J, nsplit, scale);
    (void)O;
    return hipGetLastError();
}

template <int DT, int D, bool DENSE>
hipError_t launch_attn_rep(const void* Q, const void* K, const void* V, const int32_t* idx,
                           float* part, void* O, int B, int H, int Hkv, int N, long long ldn, int k,
                           int nsplit, hipStream_t s) {
    switch (H / Hkv) {
        case 1: return launch_attn_t<DT, D, 1, DENSE>(Q, K, V, idx, part, O, B, Hkv, N, ldn, k, nsplit, s);
        case 2: return launch_attn_t<DT, D, 2, DENSE>(Q, K, V, idx, part, O, B, Hkv, N, ldn, k, nsplit, s);
        case 4: return launch_attn_t<DT, D, 4, DENSE>(Q, K, V, idx, part, O, B, Hkv, N, ldn, k, nsplit, s);
        case 8: return launch_attn_t<DT, D, 8, DENSE>(Q, K, V, idx, part, O, B, Hkv, N, ldn, k, nsplit, s);
        default: return hipErrorInvalidValue;
    }
}

template <bool DENSE>
hipError_t launch_attn_any(const void* Q, const void* K, const void* V, int dtype,
                           const int32_t* idx, float* part, void* O, int B, int H, int Hkv, int N,
                           long long ldn, int D, int k, int nsplit, hipStream_t s) {
#define DCR_ATTN_CASE(DTV, DV)                                                                  \
    if (dtype == DTV && D == DV)                                                                \
        return launch_attn_rep<DTV, DV, DENSE>(Q, K, V, idx, part, O, B, H, Hkv, N, ldn, k, nsplit, \
                                               s);
    DCR_ATTN_CASE(kF32, 64)
    DCR_ATTN_CASE(kF16, 64)
    DCR_ATTN_CASE(kBF16, 64)
    DCR_ATTN_CASE(kF32, 128)
    DCR_ATTN_CASE(kF16, 128)
    DCR_ATTN_CASE(kBF16, 128)
#undef DCR_ATTN_CASE
    return hipErrorInvalidValue;
}

}  // namespace

int attn_num_splits(int groups, int k) {
    const int tile = AttnGeom<kF16, 64>::TILE;  // 32 rows
    const int J = split_rows(groups, k, tile);
    return (k + J - 1) / J;
}

int dense_num_splits(int groups, int N) {
    const int tile = AttnGeom<kF16, 64>::TILE;
    const int J = split_rows(groups, N, tile);
    return (N + J - 1) / J;
}

hipError_t launch_sparse_attn(const void* Q, const void* K, const void* V, int dtype,
                              const int32_t* idx, float* part, void* O, int B, int H, int Hkv,
                              int N, long long ldn, int D, int k, int nsplit, hipStream_t s) {
    return launch_attn_any<false>(Q, K, V, dtype, idx, part, O, B, H, Hkv, N, ldn, D, k, nsplit, s);
}

hipError_t launch_dense_attn(const void* Q, const void* K, const void* V, int dtype, float* part,
                             void* O, int B, int H, int Hkv, int N, long long ldn, int D,
                             int nsplit, hipStream_t s) {
    return launch_attn_any<true>(Q, K, V, dtype, nullptr, part, O, B, H, Hkv, N, ldn, D, N, nsplit,
                                 s);
}

hipError_t launch_combine(const float* part, void* O, int dtype, int BH, int D, int nsplit,
                          hipStream_t s) {
    const unsigned grid = static_cast<unsigned>((BH + 3) / 4);
#define DCR_COMBINE_CASE(DTV, DV)                                          \
    if (dtype == DTV && D == DV) {                                         \
        launch_kernel(combine_kernel<DTV, DV>, grid, dim3(256), 0, s, part, O, BH, nsplit); \
        return hipGetLastError();                                          \
    }
    DCR_COMBINE_CASE(kF32, 64)
    DCR_COMBINE_CASE(kF16, 64)
    DCR_COMBINE_CASE(kBF16, 64)
    DCR_COMBINE_CASE(kF32, 128)
    DCR_COMBINE_CASE(kF16, 128)
    DCR_COMBINE_CASE(kBF16, 128)
#undef DCR_COMBINE_CASE
    return hipErrorInvalidValue;
}

}  // namespace dcr
