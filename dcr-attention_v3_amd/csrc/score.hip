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
//      consecutive K), prefetched one iteration ahead;
//   2. a transpose through a wave-private LDS tile (row stride padded by
//      16 bytes so the per-lane row reads are bank-conflict free);
//   3. each lane runs the sequential FMA chain of its own row for all R query
//      heads of the GQA group; u is wave-uniform and is read with scalar loads
//      into SGPRs in blocks of 64 floats, so each FMA is one VALU op
//      (v_fma_mix_f32 for fp16 keys) with an SGPR operand.
// The optional level-1 radix histogram of the score keys (top 8 bits of the
// order-preserving 16-bit key: one bin per binade) is accumulated in LDS and
// flushed to global memory with atomics once per workgroup (few bins are
// non-zero); the select kernel then needs no pass over all N scores to find
// its bin.
#include "dcr_common.h"
#include "dcr_kernels.h"

namespace dcr {
namespace {

typedef const float __attribute__((address_space(4)))* ConstF32Ptr;

constexpr int kRowsPerWave = 64;

// nxt[i] = 16 bytes at Kg + min(base + i*1024, last_chunk).  Ordinary
// (temporal) loads on purpose: K read here stays in the 256 MB Infinity Cache
// for the gather that follows (non-temporal loads stream ~8% faster here but
// make the gather miss it and cost more than they save).
template <int CPR>
__device__ __forceinline__ void load_rows(chunk_t (&nxt)[CPR], const uint8_t* __restrict__ Kg,
                                          long long base, long long last_chunk) {
#pragma unroll
    for (int i = 0; i < CPR; ++i) {
        long long off = base + static_cast<long long>(i) * 1024;
        off = off < last_chunk ? off : last_chunk;
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

// Score one key row (in LDS) against the NREP u vectors of the GQA group with
// a sequential fp32 FMA chain over d, store the bf16 scores and bump the
// level-1 histogram.
template <int DT, int D, int NREP, bool HIST>
__device__ __forceinline__ void score_rows(const chunk_t* __restrict__ myrow, ConstF32Ptr ug,
                                           uint16_t* __restrict__ scores, uint32_t* hist_lds,
                                           size_t head0, int N, long long n) {
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
    if (n < N) {
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
            const uint32_t sb = f32_to_bf16_bits(acc[h]);
            scores[(head0 + h) * static_cast<size_t>(N) + static_cast<size_t>(n)] =
                static_cast<uint16_t>(sb);
            if constexpr (HIST) atomicAdd(&hist_lds[h * kHist1Bins + (bf16_key(sb) >> kHist2Bits)], 1u);
        }
    }
}

template <int DT, int D, int NREP, bool HIST, int ITERS>
__global__ __launch_bounds__((64 * ScoreGeom<DT, D>::WAVES)) void score_kernel(
    const uint8_t* __restrict__ K, const float* __restrict__ u, uint16_t* __restrict__ scores,
    uint32_t* __restrict__ hist1, int Hkv, int N, long long ldn) {
    using G = ScoreGeom<DT, D>;
    constexpr int CPR = G::CPR, RSTR = G::RSTR, RB = G::RB, WAVES = G::WAVES;
    // Blocks of 64 rows in flight per wave (register budget: 32 VGPRs each
    // for 128-byte rows).
    constexpr int PD = (CPR <= 8 && ITERS > 1) ? 2 : 1;

    __shared__ chunk_t stage[WAVES][kRowsPerWave * RSTR];
    __shared__ uint32_t hist_lds[HIST ? NREP * kHist1Bins : 1];

    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x >> 6);
    const int bg = static_cast<int>(blockIdx.y);  // b * Hkv + g
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
    const long long wg_row0 = static_cast<long long>(blockIdx.x) * (WAVES * kRowsPerWave * ITERS);
    // A wave's 64 rows are one contiguous 64*RB-byte span; load i covers bytes
    // [i*1024, i*1024+1024) of it.  Past the last row the offset is clamped to
    // the last chunk of K (those lanes' scores are never stored).
    const long long last_chunk = static_cast<long long>(N) * RB - 16;
    auto rows_of = [&](int it) {
        return wg_row0 + (static_cast<long long>(it) * WAVES + wave) * kRowsPerWave;
    };

    // The iteration loop is fully unrolled so the compiler can wait for each
    // block's own loads only, keeping the next PD-1 blocks in flight.
    chunk_t buf[PD][CPR];
#pragma unroll
    for (int p = 0; p < PD; ++p) load_rows<CPR>(buf[p], Kg, rows_of(p) * RB + lane * 16, last_chunk);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int p = it % PD;
        // Stage this iteration's rows (row-major, padded) into the wave's tile.
#pragma unroll
        for (int i = 0; i < CPR; ++i) {
            const int ci = i * 64 + lane;
            st[(ci / CPR) * RSTR + (ci % CPR)] = buf[p][i];
        }
        __builtin_amdgcn_wave_barrier();
        if (it + PD < ITERS) load_rows<CPR>(buf[p], Kg, rows_of(it + PD) * RB + lane * 16, last_chunk);
        score_rows<DT, D, NREP, HIST>(st + lane * RSTR, ug, scores, hist_lds, head0, N, rows_of(it) + lane);
        __builtin_amdgcn_wave_barrier();
    }

    if constexpr (HIST) {
        __syncthreads();
        for (int i = static_cast<int>(threadIdx.x); i < NREP * kHist1Bins; i += 64 * WAVES) {
            const uint32_t v = hist_lds[i];
            if (v != 0u) atomicAdd(hist1 + head0 * kHist1Bins + i, v);
        }
    }
}

// Workgroups of `kernel` resident on the whole device at once.
template <typename Kernel>
int resident_workgroups(Kernel kernel, int block) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    return cus * per_cu;
}

template <int DT, int D, int NREP, bool HIST, int ITERS>
hipError_t launch_score_it(const void* K, const float* u, uint16_t* scores, uint32_t* hist1, int B,
                           int Hkv, int N, long long ldn, hipStream_t s) {
    using G = ScoreGeom<DT, D>;
    const long long rows_per_wg = static_cast<long long>(G::WAVES) * kRowsPerWave * ITERS;
    const dim3 grid(static_cast<unsigned>((N + rows_per_wg - 1) / rows_per_wg),
                    static_cast<unsigned>(B * Hkv));
    launch_kernel(score_kernel<DT, D, NREP, HIST, ITERS>, grid, dim3(64 * G::WAVES), 0, s,
        static_cast<const uint8_t*>(K), u, scores, hist1, Hkv, N, ldn);
    return hipGetLastError();
}

// Rows per workgroup: 8 iterations per wave (2048 rows for 4 waves) unless
// that leaves fewer workgroups than half the device holds at once.
template <int DT, int D, int NREP, bool HIST>
hipError_t launch_score_h(const void* K, const float* u, uint16_t* scores, uint32_t* hist1, int B,
                          int Hkv, int N, long long ldn, hipStream_t s) {
    using G = ScoreGeom<DT, D>;
    static const int resident =
        resident_workgroups(score_kernel<DT, D, NREP, HIST, 8>, 64 * G::WAVES);
    const long long groups = static_cast<long long>(B) * Hkv;
    int iters = 8;
    while (iters > 1) {
        const long long rows_per_wg = static_cast<long long>(G::WAVES) * kRowsPerWave * iters;
        if (groups * ((N + rows_per_wg - 1) / rows_per_wg) * 2 >= resident) break;
        iters /= 2;
    }
    switch (iters) {
        case 8: return launch_score_it<DT, D, NREP, HIST, 8>(K, u, scores, hist1, B, Hkv, N, ldn, s);
        case 4: return launch_score_it<DT, D, NREP, HIST, 4>(K, u, scores, hist1, B, Hkv, N, ldn, s);
        case 2: return launch_score_it<DT, D, NREP, HIST, 2>(K, u, scores, hist1, B, Hkv, N, ldn, s);
        default: return launch_score_it<DT, D, NREP, HIST, 1>(K, u, scores, hist1, B, Hkv, N, ldn, s);
    }
}

template <int DT, int D, int NREP>
hipError_t launch_score_t(const void* K, const float* u, uint16_t* scores, uint32_t* hist1, int B,
                          int Hkv, int N, long long ldn, hipStream_t s) {
    if (hist1 != nullptr) return launch_score_h<DT, D, NREP, true>(K, u, scores, hist1, B, Hkv, N, ldn, s);
    return launch_score_h<DT, D, NREP, false>(K, u, scores, hist1, B, Hkv, N, ldn, s);
}

template <int DT, int D>
hipError_t launch_score_rep(const void* K, const float* u, uint16_t* scores, uint32_t* hist1, int B,
                            int Hkv, int n_rep, int N, long long ldn, hipStream_t s) {
    switch (n_rep) {
        case 1: return launch_score_t<DT, D, 1>(K, u, scores, hist1, B, Hkv, N, ldn, s);
        case 2: return launch_score_t<DT, D, 2>(K, u, scores, hist1, B, Hkv, N, ldn, s);
        case 4: return launch_score_t<DT, D, 4>(K, u, scores, hist1, B, Hkv, N, ldn, s);
        case 8: return launch_score_t<DT, D, 8>(K, u, scores, hist1, B, Hkv, N, ldn, s);
        default: return hipErrorInvalidValue;
    }
}

template <int DT>
hipError_t launch_score_d(const void* K, const float* u, uint16_t* scores, uint32_t* hist1, int B,
                          int Hkv, int n_rep, int N, int D, long long ldn, hipStream_t s) {
    switch (D) {
        case 64: return launch_score_rep<DT, 64>(K, u, scores, hist1, B, Hkv, n_rep, N, ldn, s);
        case 128: return launch_score_rep<DT, 128>(K, u, scores, hist1, B, Hkv, n_rep, N, ldn, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_score(const void* K, int kv_dtype, const float* u, uint16_t* scores,
                        uint32_t* hist1, int B, int Hkv, int n_rep, int N, int D, long long ldn,
                        hipStream_t s) {
    switch (kv_dtype) {
        case kF32: return launch_score_d<kF32>(K, u, scores, hist1, B, Hkv, n_rep, N, D, ldn, s);
        case kF16: return launch_score_d<kF16>(K, u, scores, hist1, B, Hkv, n_rep, N, D, ldn, s);
        case kBF16: return launch_score_d<kBF16>(K, u, scores, hist1, B, Hkv, n_rep, N, D, ldn, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dcr
