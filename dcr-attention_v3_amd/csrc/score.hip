// score.hip -- projection ("score") pass of the sparse decode path.
//
// Replaces the reference's Pass 1 (_pass1_projection_kernel /
// topk_pass1_projection, dcr_attention/kernel/triton/topk_axis_pass1.py:28-153;
// M1 twin _compute_projection_scores, qaxis_topk_reference.py:58-88):
//
//   scores[b, g*R + r, n] = bf16_rne( sum_d fp32(K[b, g, n, d]) * u[b, g*R + r, d] )
//
// with the sum evaluated as one fused-multiply-add chain over d = 0..D-1
// starting from +0 -- the order an MKL sgemm micro-kernel uses for the
// reference's einsum, so scores are bit-identical to the CPU reference.
//
// MI355X mapping.  The pass streams K once (HBM bound).  A workgroup owns a
// (b, g) KV head and a range of rows; each wave moves 64 rows per iteration:
//   1. 16-byte coalesced global loads (one wave instruction = 1 KiB of
//      consecutive K), prefetched up to two iterations ahead;
//   2. a transpose through a wave-private LDS tile (row stride padded by
//      16 bytes so the per-lane row reads are bank-conflict free), after which
//      lane l holds row l;
//   3. the dot products run on the matrix cores: v_mfma_f32_4x4x1f32 (16
//      blocks of 4 rows x 4 heads, K = 1) computes acc = a*b + acc with one
//      rounding, exactly an fma, so 64 (or 128) chained MFMAs over d give the
//      sequential fma chain bit for bit.  Operand A is lane l's K element d
//      (row 4*blk + i sits in lane 4*blk + i), operand B is u[head j][d] in
//      lane 4*blk + j, and lane 4*blk + j ends with the scores of rows
//      4*blk .. 4*blk+3 for head j.  u stays in VGPRs for the whole kernel.
// The fused form also (a) computes the group's unit query vectors from Q at
// the start (the u_Q step, overlapped with the first K loads, so the path
// needs no launch for it), and (b) accumulates the level-1 radix histogram of
// the score keys (top 8 bits of the order-preserving 16-bit key) in LDS and
// writes it as one slab per workgroup; the select kernel sums a row's slabs
// instead of making a pass over all N scores to find its bin.
// One shape whose u operand would not fit in registers (8 heads per KV head
// with D = 128) runs a VALU variant: each lane runs the fma chain of its row
// with u in SGPRs (scalar loads from a u computed by a separate launch).
#include "dcr_common.h"
#include "dcr_kernels.h"

namespace dcr {
namespace {

typedef const float __attribute__((address_space(4)))* ConstF32Ptr;
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kRowsPerWave = 64;

// nxt[i] = 16 bytes at Kg + min(base + i*1024, last_chunk).  NT: non-temporal
// loads, for when no later kernel reads K (the fp16/bf16 decode path, whose
// attention reads V only): they stream faster and leave the L2 and the
// Infinity Cache to the scores the select kernel reads next.  Otherwise
// ordinary loads, so K stays in the 256 MB Infinity Cache for the K gather
// that follows.
template <int CPR, bool NT>
__device__ __forceinline__ void load_rows(chunk_t (&nxt)[CPR], const uint8_t* __restrict__ Kg,
                                          long long base, long long last_chunk) {
#pragma unroll
    for (int i = 0; i < CPR; ++i) {
        long long off = base + static_cast<long long>(i) * 1024;
        off = off < last_chunk ? off : last_chunk;
        if constexpr (NT)
            nxt[i] = __builtin_nontemporal_load(reinterpret_cast<const chunk_t*>(Kg + off));
        else
            nxt[i] = *reinterpret_cast<const chunk_t*>(Kg + off);
    }
}

template <int DT, int D>
struct ScoreGeom {
    static constexpr int EB = ElemBytes<DT>::value;
    static constexpr int RB = D * EB;           // bytes per key row
    static constexpr int CPR = RB / 16;         // 16-byte chunks per row
    static constexpr int RSTR = CPR + 1;        // LDS row stride (chunks)
    static constexpr int EPC = 16 / EB;         // elements per chunk
    static constexpr int WAVES = (RB <= 256) ? 4 : 2;
};

// Whether the MFMA kernel serves (DT, D, NREP): u[j][d] for the group's heads
// takes ceil(NREP/4) * D VGPRs per lane.
template <int D, int NREP>
struct UseMfma {
    static constexpr bool value = ((NREP + 3) / 4) * D <= 128;
};

// What the score pass stores per (head, position):
//   kOutBf16     the bf16 score bits (the standalone projection pass);
//   kOutKeys     the order-preserving 16-bit key of the bf16 score (the fused
//                path: the select kernel reads keys without converting);
//   kOutKeysRes  the keys, plus one byte per score in a second array: the
//                8-bit residual of the fp32 dot product over its bf16
//                rounding (score_residual), from which the fp16/bf16 fused
//                path's attention rebuilds the selected positions' fp32
//                logits to 2^-15 relative (score_from_key).
// The fused forms also count the keys' top 8 bits in a level-1 histogram.
enum ScoreOut { kOutBf16 = 0, kOutKeys = 1, kOutKeysRes = 2 };

__device__ __forceinline__ uint32_t stored_score(uint32_t sb, int out) {
    return out == kOutBf16 ? sb : bf16_key(sb);
}

// Score one key row (in LDS) against the NREP u vectors of the GQA group with
// a sequential fp32 FMA chain over d, store the scores and bump the level-1
// histogram.  (VALU variant.)
template <int DT, int D, int NREP, bool HIST, int OUT>
__device__ __forceinline__ void score_rows(const chunk_t* __restrict__ myrow, ConstF32Ptr ug,
                                           uint16_t* __restrict__ scores, uint8_t* __restrict__ res,
                                           uint32_t* hist_lds, size_t head0, int N, long long ldsc,
                                           long long n) {
    constexpr int EPC = 16 / ElemBytes<DT>::value;
    constexpr int DB = 64 / NREP;    // dims per u block: NREP * DB = 64 SGPR floats
    constexpr int CPB = DB / EPC;    // K chunks per u block
    constexpr int NB = D / DB;       // u blocks per row
    static_assert(DB % EPC == 0, "u block must cover whole chunks");
    float acc[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) acc[h] = 0.0f;
#pragma unroll 1
    for (int blk = 0; blk < NB; ++blk) {
        chunk_t kc[CPB];
#pragma unroll
        for (int c = 0; c < CPB; ++c) kc[c] = myrow[blk * CPB + c];
        float uu[NREP][DB];
#pragma unroll
        for (int h = 0; h < NREP; ++h)
#pragma unroll
            for (int d = 0; d < DB; ++d) uu[h][d] = ug[h * D + blk * DB + d];
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const float kf = chunk_elem<DT>(kc[d / EPC], d % EPC);
#pragma unroll
            for (int h = 0; h < NREP; ++h) acc[h] = __builtin_fmaf(kf, uu[h][d], acc[h]);
        }
    }
    // The fused forms also write key 0 (below every real key) at the padding
    // positions N <= n < ldsc, so the select kernel reads whole rows.
    if (n < N || (OUT != kOutBf16 && n < ldsc)) {
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
            const uint32_t sb = f32_to_bf16_bits(acc[h]);
            const size_t at = (head0 + h) * static_cast<size_t>(ldsc) + static_cast<size_t>(n);
            scores[at] = static_cast<uint16_t>(n < N ? stored_score(sb, OUT) : 0u);
            if constexpr (OUT == kOutKeysRes) res[at] = static_cast<uint8_t>(n < N ? score_residual(acc[h], sb) : 0u);
            if constexpr (HIST)
                if (n < N) atomicAdd(&hist_lds[h * kHist1Bins + (bf16_key(sb) >> kHist2Bits)], 1u);
        }
    }
}

// Tiles of 64 rows: workgroup x owns the contiguous block of WAVES * ITERS
// tiles starting at tile x * WAVES * ITERS, and wave w takes tile it * WAVES +
// w of it in round it.  The grid has at most floor(tiles / (WAVES * ITERS))
// workgroups per group, so the unrolled rounds never start past N; the tiles
// after the last block are dealt one per wave in turn (tail_row0, stepping by
// tail_step).
struct TileMap {
    long long wg_row0, tail_row0, tail_step;
    int wave, waves;
    // x: the workgroup's index among the nx workgroups of its group.
    __device__ TileMap(int waves_, int iters, int wave_, int x, int nx)
        : wg_row0(static_cast<long long>(x) * waves_ * iters * kRowsPerWave),
          tail_row0((static_cast<long long>(nx) * waves_ * iters +
                     static_cast<long long>(x) * waves_ + wave_) * kRowsPerWave),
          tail_step(static_cast<long long>(nx) * waves_ * kRowsPerWave),
          wave(wave_), waves(waves_) {}
    __device__ long long row0(int it) const {
        return wg_row0 + (static_cast<long long>(it) * waves + wave) * kRowsPerWave;
    }
};

// Level-1 histogram slabs: workgroup x of a group writes its NREP x 256-bin
// histograms to hist[(head0 + h) * nx + x][256] (a slab per workgroup, no
// atomics, nothing to clear beforehand).
template <int NREP, int THREADS>
__device__ __forceinline__ void write_slabs(const uint32_t* hist_lds, slab_t* __restrict__ hist,
                                            size_t head0, int x, int nx) {
    slab_t* slab = hist + (head0 * nx + x) * kHist1Bins;
    for (int i = static_cast<int>(threadIdx.x); i < NREP * kHist1Bins; i += THREADS) {
        const int h = i / kHist1Bins;
        slab[static_cast<size_t>(h) * nx * kHist1Bins + (i % kHist1Bins)] = static_cast<slab_t>(hist_lds[i]);
    }
}

// The MFMA kernel's level-1 histogram: HC copies of NREP x 256 bins in LDS,
// lanes spread over the copies by their row block, so that lanes whose scores
// fall in the same binade (most of a tile's scores share a few) do not all
// update one LDS word.  Rows of bins are padded so that one bin of the
// different heads and copies sits in different banks.
template <int NREP, int HC_ = 16 / NREP>
struct HistCopies {
    static constexpr int HC = HC_;                       // copies
    static constexpr int HS = kHist1Bins + 8;            // words per head
    static constexpr int CS = NREP * HS + 2;             // words per copy
    static constexpr int WORDS = HC * CS;
};

template <int NREP, int THREADS, class HCp>
__device__ __forceinline__ void write_slabs_copies(const uint32_t* hist_lds, slab_t* __restrict__ hist,
                                                   size_t head0, int x, int nx) {
    slab_t* slab = hist + (head0 * nx + x) * kHist1Bins;
    for (int i = static_cast<int>(threadIdx.x); i < NREP * kHist1Bins; i += THREADS) {
        const int h = i / kHist1Bins, bin = i % kHist1Bins;
        uint32_t sum = 0u;
#pragma unroll
        for (int c = 0; c < HCp::HC; ++c) sum += hist_lds[c * HCp::CS + h * HCp::HS + bin];
        slab[static_cast<size_t>(h) * nx * kHist1Bins + bin] = static_cast<slab_t>(sum);
    }
}

// The workgroup's (x, group) in XCD order (grid (nx, groups)).
struct ScoreWg {
    int x, nx, bg;
    __device__ ScoreWg() {
        nx = static_cast<int>(gridDim.x);
        const unsigned idx = xcd_order(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
        x = static_cast<int>(idx % gridDim.x);
        bg = static_cast<int>(idx / gridDim.x);  // b * Hkv + g
    }
};

// The wave's remainder tiles from row r0 on, stepping by `step`: each tile's
// rows are loaded while the previous tile is scored (a runtime loop, so the
// next tile waits in a second buffer).
template <int CPR, bool NTK, class F>
__device__ __forceinline__ void tail_rounds(const uint8_t* __restrict__ Kg, long long r0, long long step,
                                            int N, int lane, long long last_chunk, F&& process) {
    constexpr int RB = CPR * 16;
    if (r0 >= N) return;
    chunk_t nxt[CPR];
    load_rows<CPR, NTK>(nxt, Kg, r0 * RB + lane * 16, last_chunk);
    for (long long rr = r0; rr < N; rr += step) {
        chunk_t cur[CPR];
#pragma unroll
        for (int i = 0; i < CPR; ++i) cur[i] = nxt[i];
        if (rr + step < N) load_rows<CPR, NTK>(nxt, Kg, (rr + step) * RB + lane * 16, last_chunk);
        process(cur, rr);
    }
}

// VALU variant (u given in global memory, read with scalar loads).
template <int DT, int D, int NREP, bool HIST, int ITERS, int OUT, bool NTK>
__global__ __launch_bounds__((64 * ScoreGeom<DT, D>::WAVES)) void score_kernel(
    const uint8_t* __restrict__ K, const float* __restrict__ u, uint16_t* __restrict__ scores,
    uint8_t* __restrict__ res, slab_t* __restrict__ hist, int Hkv, int N, long long ldn,
    long long ldsc) {
    using G = ScoreGeom<DT, D>;
    constexpr int CPR = G::CPR, RSTR = G::RSTR, RB = G::RB, WAVES = G::WAVES;
    constexpr int PD = (CPR <= 8 && ITERS > 1) ? 2 : 1;  // 64-row blocks in flight per wave

    __shared__ chunk_t stage[WAVES][kRowsPerWave * RSTR];
    __shared__ uint32_t hist_lds[HIST ? NREP * kHist1Bins : 1];

    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x >> 6);
    const ScoreWg wg;
    const int bg = wg.bg;
    const int b = bg / Hkv;
    const int g = bg - b * Hkv;
    const size_t head0 = static_cast<size_t>(b) * Hkv * NREP + static_cast<size_t>(g) * NREP;
    const uint8_t* Kg = K + static_cast<size_t>(bg) * static_cast<size_t>(ldn) * RB;
    ConstF32Ptr ug = (ConstF32Ptr)(u + head0 * D);

    if constexpr (HIST) {
        for (int i = static_cast<int>(threadIdx.x); i < NREP * kHist1Bins; i += 64 * WAVES)
            hist_lds[i] = 0u;
        __syncthreads();
    }

    chunk_t* st = stage[wave];
    const TileMap tm(WAVES, ITERS, wave, wg.x, wg.nx);
    const long long last_chunk = static_cast<long long>(N) * RB - 16;
    auto process = [&](const chunk_t (&data)[CPR], long long row0) {
#pragma unroll
        for (int i = 0; i < CPR; ++i) {
            const int ci = i * 64 + lane;
            st[(ci / CPR) * RSTR + (ci % CPR)] = data[i];
        }
        __builtin_amdgcn_wave_barrier();
        score_rows<DT, D, NREP, HIST, OUT>(st + lane * RSTR, ug, scores, res, hist_lds, head0, N,
                                           ldsc, row0 + lane);
        __builtin_amdgcn_wave_barrier();
    };

    // Main rounds: fully unrolled, so each block waits for its own loads only.
    chunk_t buf[PD][CPR];
#pragma unroll
    for (int p = 0; p < PD; ++p) load_rows<CPR, NTK>(buf[p], Kg, tm.row0(p) * RB + lane * 16, last_chunk);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int p = it % PD;
        chunk_t cur[CPR];
#pragma unroll
        for (int i = 0; i < CPR; ++i) cur[i] = buf[p][i];
        if (it + PD < ITERS) load_rows<CPR, NTK>(buf[p], Kg, tm.row0(it + PD) * RB + lane * 16, last_chunk);
        process(cur, tm.row0(it));
    }
    // Remainder tiles, one ahead in flight.
    tail_rounds<CPR, NTK>(Kg, tm.tail_row0, tm.tail_step, N, lane, last_chunk, process);

    if constexpr (HIST) {
        __syncthreads();
        write_slabs<NREP, 64 * WAVES>(hist_lds, hist, head0, wg.x, wg.nx);
    }
}

// MFMA variant.  UQ = true: uq points at Q (dtype DT) and the workgroup
// computes its group's u itself (unit_row, the same code and order as
// uq_kernel); UQ = false: uq points at u (fp32).  OUT: see ScoreOut.
template <int DT, int D, int NREP, bool HIST, int ITERS, bool UQ, int OUT, bool NTK>
__global__ __launch_bounds__((64 * ScoreGeom<DT, D>::WAVES)) void score_mfma_kernel(
    const uint8_t* __restrict__ K, const void* __restrict__ uq, float eps,
    uint16_t* __restrict__ scores, uint8_t* __restrict__ res, slab_t* __restrict__ hist, int Hkv,
    int N, long long ldn, long long ldsc) {
    using G = ScoreGeom<DT, D>;
    constexpr int CPR = G::CPR, RSTR = G::RSTR, RB = G::RB, WAVES = G::WAVES, EPC = G::EPC;
    constexpr int NCH = (NREP + 3) / 4;                    // 4-head MFMA chains
    constexpr int PD = (CPR <= 8 && ITERS > 1) ? 2 : 1;  // 64-row blocks in flight per wave

    __shared__ chunk_t stage[WAVES][kRowsPerWave * RSTR];
    // u rows padded by 4 floats: the 16-byte reads of the four heads of a
    // chain (lanes 4b..4b+3) then fall in different banks.
    __shared__ __align__(16) float u_lds[NREP][D + 4];
    // D > 64: u is read from LDS in the chain instead of living in 128
    // VGPRs, and the histogram has one copy, so that two workgroups (eight
    // waves) fit on a CU; D = 64 keeps u in registers and four copies.
    constexpr bool ULDS = D > 64;
    using HCp = HistCopies<NREP, ULDS ? 1 : 16 / NREP>;
    __shared__ uint32_t hist_lds[HIST ? HCp::WORDS : 1];

    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x >> 6);
    const ScoreWg wg;
    const int bg = wg.bg;
    const int b = bg / Hkv;
    const int g = bg - b * Hkv;
    const size_t head0 = static_cast<size_t>(b) * Hkv * NREP + static_cast<size_t>(g) * NREP;
    const uint8_t* Kg = K + static_cast<size_t>(bg) * static_cast<size_t>(ldn) * RB;

    chunk_t* st = stage[wave];
    const TileMap tm(WAVES, ITERS, wave, wg.x, wg.nx);
    const long long last_chunk = static_cast<long long>(N) * RB - 16;

    chunk_t buf[PD][CPR];
#pragma unroll
    for (int p = 0; p < PD; ++p) load_rows<CPR, NTK>(buf[p], Kg, tm.row0(p) * RB + lane * 16, last_chunk);

    // u of the group's heads into LDS, then into registers: ub[c][d] =
    // u[4c + (lane & 3)][d] (zero for padding heads >= NREP).
    if constexpr (UQ) {
        for (int h = wave; h < NREP; h += WAVES)
            unit_row<DT, D>(uq, (head0 + h) * static_cast<size_t>(D), eps, &u_lds[h][0]);
    } else {
        const float* u = static_cast<const float*>(uq) + head0 * D;
        for (int i = static_cast<int>(threadIdx.x); i < NREP * D; i += 64 * WAVES)
            u_lds[i / D][i % D] = u[i];
    }
    if constexpr (HIST) {
        for (int i = static_cast<int>(threadIdx.x); i < HCp::WORDS; i += 64 * WAVES)
            hist_lds[i] = 0u;
    }
    __syncthreads();
    float ub[NCH][ULDS ? 1 : D];
    if constexpr (!ULDS) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int j = 4 * c + (lane & 3);
            const float* urow = &u_lds[j < NREP ? j : 0][0];
#pragma unroll
            for (int d = 0; d < D; d += 4) {
                const f32x4 t = *reinterpret_cast<const f32x4*>(urow + d);
#pragma unroll
                for (int e = 0; e < 4; ++e) ub[c][d + e] = (j < NREP) ? t[e] : 0.0f;
            }
        }
    }

    const int jl = lane & 3;          // head within a chain
    const int r0 = lane & ~3;         // first of the lane's four output rows
    const int hcopy = (lane >> 2) % HCp::HC;  // histogram copy of the lane's row block
    const bool n_vec4 = (ldsc % 4) == 0;  // one store of four scores
    // Stage a tile (64 rows from row0) through LDS, run the MFMA chains, store
    // the bf16 scores and count them in the histogram.
    auto process = [&](const chunk_t (&data)[CPR], long long row0) {
#pragma unroll
        for (int i = 0; i < CPR; ++i) {
            const int ci = i * 64 + lane;
            st[(ci / CPR) * RSTR + (ci % CPR)] = data[i];
        }
        __builtin_amdgcn_wave_barrier();
        f32x4 acc[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const chunk_t* myrow = st + lane * RSTR;
        if constexpr (ULDS) {
            // One chain (NCH = 1): lane 4b + j multiplies by u[j][d] (heads
            // j >= NREP read head 0; their results are never stored).  The
            // empty asm keeps the compiler from hoisting these LDS reads out
            // of the tile loop into registers.
            static_assert(NCH == 1 && EPC % 4 == 0, "LDS-operand form covers one chain");
            asm volatile("" ::: "memory");
            const float* urow = &u_lds[(lane & 3) < NREP ? (lane & 3) : 0][0];
#pragma unroll
            for (int i = 0; i < CPR; ++i) {
                const chunk_t kc = myrow[i];
#pragma unroll
                for (int e4 = 0; e4 < EPC; e4 += 4) {
                    const f32x4 uv = *reinterpret_cast<const f32x4*>(urow + i * EPC + e4);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(chunk_elem<DT>(kc, e4 + e), uv[e], acc[0], 0,
                                                                    0, 0);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < CPR; ++i) {
                const chunk_t kc = myrow[i];
#pragma unroll
                for (int e = 0; e < EPC; ++e) {
                    const float a = chunk_elem<DT>(kc, e);
#pragma unroll
                    for (int c = 0; c < NCH; ++c)
                        acc[c] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, ub[c][i * EPC + e], acc[c], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();

        const long long n0 = row0 + r0;  // rows n0 .. n0+3, head 4c + jl
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int h = 4 * c + jl;
            if (h >= NREP) continue;
            uint32_t sb[4], sk[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                sb[v] = f32_to_bf16_bits(acc[c][v]);
                sk[v] = stored_score(sb[v], OUT);
            }
            const size_t rowoff = (head0 + h) * static_cast<size_t>(ldsc);
            uint16_t* out = scores + rowoff;
            if (n_vec4 && n0 + 3 < N) {
                *reinterpret_cast<uint2*>(out + n0) = make_uint2(sk[0] | (sk[1] << 16), sk[2] | (sk[3] << 16));
                if constexpr (OUT == kOutKeysRes)
                    *reinterpret_cast<uint32_t*>(res + rowoff + n0) =
                        score_residual(acc[c][0], sb[0]) | (score_residual(acc[c][1], sb[1]) << 8) |
                        (score_residual(acc[c][2], sb[2]) << 16) | (score_residual(acc[c][3], sb[3]) << 24);
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (n0 + v < N) {
                        out[n0 + v] = static_cast<uint16_t>(sk[v]);
                        if constexpr (OUT == kOutKeysRes)
                            res[rowoff + n0 + v] = static_cast<uint8_t>(score_residual(acc[c][v], sb[v]));
                    } else if (OUT != kOutBf16 && n0 + v < ldsc) {
                        out[n0 + v] = 0;  // fused forms: key 0 at the padding positions
                    }
                }
            }
            if constexpr (HIST) {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (n0 + v < N)
                        atomicAdd(&hist_lds[hcopy * HCp::CS + h * HCp::HS + (bf16_key(sb[v]) >> kHist2Bits)], 1u);
            }
        }
    };

    // Main rounds, then the wave's first tile after the last block (when N
    // is not a multiple of the blocks' rows: tail_row0 < N) as one more
    // round: fully unrolled, so each block waits for its own loads only, and
    // that tile's loads go out PD rounds ahead like the others (its address
    // clamped, and nothing scored, where the wave has no such tile).
    const bool has_tail = tm.tail_row0 < N;
    auto round_row0 = [&](int it) { return it < ITERS ? tm.row0(it) : tm.tail_row0; };
#pragma unroll
    for (int it = 0; it <= ITERS; ++it) {
        const int p = it % PD;
        chunk_t cur[CPR];
#pragma unroll
        for (int i = 0; i < CPR; ++i) cur[i] = buf[p][i];
        // The next tile's loads go out at raised wave priority, ahead of the
        // other waves' MFMA, LDS and store work (C5 step 597.7 -> 594.3 us,
        // C2 unchanged).
        if (it + PD <= ITERS) {
            __builtin_amdgcn_s_setprio(3);
            load_rows<CPR, NTK>(buf[p], Kg, round_row0(it + PD) * RB + lane * 16, last_chunk);
            __builtin_amdgcn_s_setprio(0);
        }
        if (it < ITERS || has_tail) process(cur, round_row0(it));
    }
    // Further remainder tiles (more than one per wave: a grid capped at the
    // resident workgroups, or few workgroups per group), one ahead in flight.
    tail_rounds<CPR, NTK>(Kg, tm.tail_row0 + tm.tail_step, tm.tail_step, N, lane, last_chunk, process);

    if constexpr (HIST) {
        __syncthreads();
        write_slabs_copies<NREP, 64 * WAVES, HCp>(hist_lds, hist, head0, wg.x, wg.nx);
    }
}

// Rounds per wave: the largest of 8, 4, 2, 1 that still gives at least 1024
// workgroups counted twice over (half the device at 4 resident workgroups
// per CU), and no more than 4 when that already gives 4096 workgroups.  A
// pure function of the shape, so the host can size the histogram slabs
// without a device query.
// Workgroups per group for ITERS rounds: floor(tiles / (WAVES * ITERS)), at least 1.
template <int DT, int D>
long long score_nx(int N, int iters) {
    using G = ScoreGeom<DT, D>;
    const long long tiles = (N + kRowsPerWave - 1) / kRowsPerWave;
    const long long nx = tiles / (static_cast<long long>(G::WAVES) * iters);
    return nx > 0 ? nx : 1;
}

template <int DT, int D>
int score_iters(long long groups, int N) {
    // Shapes with workgroups to spare run 4 rounds: at 4096 and more
    // workgroups of 4 rounds (16+ per CU) the shorter per-wave streams finish
    // together better (C5: 416 -> 390 us); smaller shapes keep 8 (C2: 4
    // rounds is 28.4 -> 32.8 us).
    if (groups * score_nx<DT, D>(N, 4) >= 4096) return 4;
    int iters = 8;
    while (iters > 1) {
        if (groups * score_nx<DT, D>(N, iters) * 2 >= 1024) break;
        iters /= 2;
    }
    return iters;
}

// Score workgroups resident at once: 256 CUs, two workgroups each (the MFMA
// kernel's VGPRs and LDS allow two).
constexpr long long kScoreResidentWgs = 512;

// Workgroups per group for ITERS rounds.  With 8 rounds (grids of fewer
// than 4096 four-round workgroups) a grid larger than one resident round of
// workgroups would run its last ones as a further, partly empty round (C2
// shapes at N = 34816: 544 workgroups, score pass 29 -> 38.5 us for 6 % more
// rows); instead the grid is capped at the resident count and the rows left
// over are dealt one tile per wave in turn, scored as further prefetched
// rounds -- when that takes no more rounds per resident slot than the
// uncapped grid (many groups cap at too few workgroups to fill the device:
// 320 groups -> 320 workgroups).  Larger shapes (4 rounds) keep their many
// workgroups, whose finishing times the dispatcher evens out.
template <int DT, int D>
long long score_grid_nx(long long groups, int N, int iters) {
    using G = ScoreGeom<DT, D>;
    const long long nx = score_nx<DT, D>(N, iters);
    if (iters != 8 || groups * nx <= kScoreResidentWgs) return nx;
    const long long cap = kScoreResidentWgs / groups;
    if (cap < 1) return nx;
    const long long tiles = (N + kRowsPerWave - 1) / kRowsPerWave;
    // Rounds per slot: uncapped, its rounds of resident workgroups times
    // ITERS, plus one where tiles follow the last block; capped, the group's
    // tiles over its waves.
    const long long uncapped = (groups * nx + kScoreResidentWgs - 1) / kScoreResidentWgs * iters +
                               (tiles > nx * G::WAVES * iters ? 1 : 0);
    const long long capped = (tiles + cap * G::WAVES - 1) / (cap * G::WAVES);
    if (capped > uncapped) return nx;
    // Slab counts stay 16-bit: a workgroup counts at most ceil(tiles / cap) tiles.
    if ((tiles + cap - 1) / cap * kRowsPerWave > 0xffff) return nx;
    return cap;
}

template <int DT, int D>
int score_slabs_t(long long groups, int N) {
    // Uncapped, a workgroup counts at most its block and as many tail tiles
    // again; a capped grid checks its own bound (score_grid_nx).
    static_assert(2 * ScoreGeom<DT, D>::WAVES * 8 * kRowsPerWave <= 0xffff, "slab counts fit slab_t");
    return static_cast<int>(score_grid_nx<DT, D>(groups, N, score_iters<DT, D>(groups, N)));
}

struct ScoreArgs {
    const void* K;
    const void* uq;   // Q (fused) or u
    float eps;
    float* u_out;     // fused VALU fallback: where the separate u launch writes u
    uint16_t* scores; // bf16 bits or keys (ScoreOut)
    uint8_t* res;     // score residual bytes (kOutKeysRes) or null
    slab_t* hist;     // slabs (fused) or null
    int B, Hkv, N;
    long long ldn;
    long long ldsc;   // row stride of scores and residuals (>= N)
    bool valu;        // the VALU form even where the MFMA form fits
};

template <int DT, int D, int NREP, int OUT, int ITERS>
hipError_t launch_score_it(const ScoreArgs& a, hipStream_t s) {
    using G = ScoreGeom<DT, D>;
    constexpr bool FUSED = OUT != kOutBf16;
    // With the residuals stored, the attention rebuilds its logits from them
    // and never reads K again: stream K past the caches.
    constexpr bool NTK = OUT == kOutKeysRes;
    const long long groups = static_cast<long long>(a.B) * a.Hkv;
    const dim3 grid(static_cast<unsigned>(score_grid_nx<DT, D>(groups, a.N, ITERS)), static_cast<unsigned>(groups));
    const auto K8 = static_cast<const uint8_t*>(a.K);
    if constexpr (UseMfma<D, NREP>::value) {
        if (!a.valu) {
            launch_kernel(score_mfma_kernel<DT, D, NREP, FUSED, ITERS, FUSED, OUT, NTK>, grid,
                          dim3(64 * G::WAVES), 0, s, K8, a.uq, a.eps, a.scores, a.res, a.hist, a.Hkv, a.N,
                          a.ldn, a.ldsc);
            return hipGetLastError();
        }
    }
    const float* u = static_cast<const float*>(a.uq);
    if constexpr (FUSED) {
        const hipError_t e = launch_uq(a.uq, DT, a.u_out, a.B * a.Hkv * NREP, D, a.eps, nullptr, 0, s);
        if (e != hipSuccess) return e;
        u = a.u_out;
    }
    launch_kernel(score_kernel<DT, D, NREP, FUSED, ITERS, OUT, NTK>, grid, dim3(64 * G::WAVES), 0, s,
                  K8, u, a.scores, a.res, a.hist, a.Hkv, a.N, a.ldn, a.ldsc);
    return hipGetLastError();
}

template <int DT, int D, int NREP, int OUT>
hipError_t launch_score_h(const ScoreArgs& a, hipStream_t s) {
    switch (score_iters<DT, D>(static_cast<long long>(a.B) * a.Hkv, a.N)) {
        case 8: return launch_score_it<DT, D, NREP, OUT, 8>(a, s);
        case 4: return launch_score_it<DT, D, NREP, OUT, 4>(a, s);
        case 2: return launch_score_it<DT, D, NREP, OUT, 2>(a, s);
        default: return launch_score_it<DT, D, NREP, OUT, 1>(a, s);
    }
}

template <int DT, int D, int NREP>
hipError_t launch_score_t(const ScoreArgs& a, int out, hipStream_t s) {
    // fused forms: u from Q and level-1 histogram slabs; otherwise u given, no histogram.
    switch (out) {
        case kOutKeysRes: return launch_score_h<DT, D, NREP, kOutKeysRes>(a, s);
        case kOutKeys: return launch_score_h<DT, D, NREP, kOutKeys>(a, s);
        default: return launch_score_h<DT, D, NREP, kOutBf16>(a, s);
    }
}

template <int DT, int D>
hipError_t launch_score_rep(const ScoreArgs& a, int n_rep, int out, hipStream_t s) {
    switch (n_rep) {
        case 1: return launch_score_t<DT, D, 1>(a, out, s);
        case 2: return launch_score_t<DT, D, 2>(a, out, s);
        case 4: return launch_score_t<DT, D, 4>(a, out, s);
        case 8: return launch_score_t<DT, D, 8>(a, out, s);
        default: return hipErrorInvalidValue;
    }
}

template <int DT>
hipError_t launch_score_d(const ScoreArgs& a, int n_rep, int D, int out, hipStream_t s) {
    switch (D) {
        case 64: return launch_score_rep<DT, 64>(a, n_rep, out, s);
        case 128: return launch_score_rep<DT, 128>(a, n_rep, out, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_score_any(const ScoreArgs& a, int kv_dtype, int n_rep, int D, int out,
                            hipStream_t s) {
    switch (kv_dtype) {
        case kF32: return launch_score_d<kF32>(a, n_rep, D, out, s);
        case kF16: return launch_score_d<kF16>(a, n_rep, D, out, s);
        case kBF16: return launch_score_d<kBF16>(a, n_rep, D, out, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

int score_slabs(int kv_dtype, int B, int Hkv, int N, int D) {
    const long long groups = static_cast<long long>(B) * Hkv;
    switch (kv_dtype) {
        case kF32: return D == 64 ? score_slabs_t<kF32, 64>(groups, N) : score_slabs_t<kF32, 128>(groups, N);
        case kF16: return D == 64 ? score_slabs_t<kF16, 64>(groups, N) : score_slabs_t<kF16, 128>(groups, N);
        default: return D == 64 ? score_slabs_t<kBF16, 64>(groups, N) : score_slabs_t<kBF16, 128>(groups, N);
    }
}

hipError_t launch_score(const void* K, int kv_dtype, const float* u, uint16_t* scores, int B,
                        int Hkv, int n_rep, int N, int D, long long ldn, hipStream_t s) {
    const ScoreArgs a{K, u, 0.0f, nullptr, scores, nullptr, nullptr, B, Hkv, N, ldn, N, false};
    return launch_score_any(a, kv_dtype, n_rep, D, kOutBf16, s);
}

hipError_t launch_score_fused(const void* K, const void* Q, int dtype, float eps, float* u_out,
                              uint16_t* keys, uint8_t* res, long long ldsc, slab_t* hist, int B,
                              int Hkv, int n_rep, int N, int D, long long ldn, bool valu, hipStream_t s) {
    const ScoreArgs a{K, Q, eps, u_out, keys, res, hist, B, Hkv, N, ldn, ldsc, valu};
    return launch_score_any(a, dtype, n_rep, D, res != nullptr ? kOutKeysRes : kOutKeys, s);
}

}  // namespace dcr
