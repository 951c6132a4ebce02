// fused.hip -- the whole sparse decode step of one layer in one launch (gfx950).
//
// Computes what the three-launch sequence (score.hip -> select.hip ->
// attn.hip) computes, and what the reference's topk_qaxis_attention composes
// (dcr_attention/kernel/triton/topk_axis.py:58-90; M1
// qaxis_topk_reference.py:200-259): u_Q, the bf16 projection score of every
// cached key, the exact top-k per (batch, query head) with ties toward the
// lower index, and the fp32 softmax attention over the selected rows.  The
// indices (when requested) are bit-identical to the three-launch path; the
// output agrees within fp32 rounding.
//
// MI355X mapping.  One launch of 256 workgroups, one per CU (its LDS use
// leaves room for no second one), 32 on each of the 8 XCDs.  The hardware
// deals workgroups to XCDs round robin, so the workgroups of one XCD share
// blockIdx % 8 and blockIdx / 8 numbers them 0..31 (their rank); the XCD
// itself is read from the XCC_ID register.  XCD x owns the (batch, KV-head)
// groups x, x + 8, ...; each of its workgroups owns one contiguous chunk of
// positions of one of those groups and carries it through four phases, with
// the XCD's workgroups meeting at a barrier between phases:
//   1. score: stream the chunk's K rows once (16-byte non-temporal loads, a
//      transpose through LDS, a v_mfma_f32_4x4x1f32 chain over d that is
//      bit-identical to the sequential fma chain of the reference's CPU
//      einsum), store each score's 16-bit order-preserving key and 8-bit
//      residual, and count the keys' top 8 bits (level-1 histogram);
//   2. from the group's level-1 histograms (the row's, summed over chunks)
//      find each head's bin T1 holding its k-th key; count the chunk's keys
//      inside T1 by their low 8 bits (level 2), the keys above T1 and the
//      largest score;
//   3. from the group's level-2 histograms find each head's exact threshold
//      key T and its tie quota, and this chunk's share of the ties (those of
//      earlier chunks come first, so ties go to the lower positions); select
//      the chunk's positions (key > T, or key == T within the quota), and for
//      every position any of the group's heads selected gather its V row
//      once and add it, weighted by each selecting head's
//      exp(logit - row max), into that head's sums; the logit is the score
//      rebuilt from key + residual (2^-16 relative) times max(|q|, eps)/sqrt(D);
//   4. merge the chunks' sums of each row and round once to the output dtype.
// The only data that cross workgroups are the histograms and the per-chunk
// sums, all inside one XCD's L2; no index list round-trips through HBM.
//
// Barriers.  Each workgroup writes its own 64-bit slot of its XCD's flag
// block (a plain store after all its stores completed; it lands in the XCD's
// L2) with tag | round, and wave 0 polls the XCD's 32 slots (L1 invalidated
// before each poll) until all hold the tag with a round >= its own.  The tag
// is a hash of a per-call nonce and a per-XCD launch counter kept in the
// workspace (advanced by every launch), so neither a graph replay nor stale
// workspace contents can satisfy a barrier early.  Every wait is bounded: on
// expiry the workgroup sets g_fused_err and carries on, so a launch always
// drains.  The scheme needs all 256 workgroups resident at once, which one
// workgroup per CU on an otherwise idle 256-CU device gives; work from other
// streams delays the barriers until it finishes and frees its CUs.
#include <math.h>

#include "dcr_common.h"
#include "dcr_kernels.h"
#include "dcr_radix.h"

namespace dcr {

// Sticky error word of the fused path: bit 0 = a phase barrier gave up.
__device__ uint32_t g_fused_err;

namespace {

constexpr int kFusedPPT = 4;             // positions per thread in phases 2 and 3
constexpr int kFusedU = 4;               // V gather instructions per tile
constexpr int kFusedHist2Stride = 260;   // words per (row, chunk) level-2 record
constexpr int kP1Mode = 0;               // phase-1 tile order (see the kernel)
constexpr int kP1Depth = 2;              // phase-1 tiles in flight per wave (1 or 2)
constexpr uint32_t kSpinMax = 1u << 21;  // barrier polls before giving up (~2 s)

// The workgroup's XCD (0..7) from the hardware register XCC_ID.
__device__ __forceinline__ uint32_t xcc_id() {
    return static_cast<uint32_t>(__builtin_amdgcn_s_getreg((31 << 11) | 20)) & 0x7u;
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {  // splitmix64 finaliser
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Barrier of the XCD's 32 workgroups (see the file comment).
__device__ void xcd_barrier(uint64_t* flags, int rank, uint64_t tag, uint32_t round) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads and stores are complete
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(flags + rank, tag | round, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (threadIdx.x < 64) {
        const int lane = static_cast<int>(threadIdx.x);
        bool done = false;
        for (uint32_t it = 0; it < kSpinMax; ++it) {
            asm volatile("buffer_inv sc0" ::: "memory");
            const uint64_t v = lane < kFusedWgPerXcd ? __builtin_nontemporal_load(flags + lane) : (tag | round);
            const bool ok = (v & ~0xffffull) == tag && (v & 0xffffull) >= round;
            if (__all(ok)) {
                done = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!done && lane == 0) atomicOr(&g_fused_err, 1u);
    }
    __syncthreads();
}

// Loads of the per-chunk records (written by other workgroups of the XCD and
// read once, from its L2) issued kBatch at a time, so that a sum over up to
// 32 chunks waits for a few load latencies instead of one per chunk.
constexpr int kBatch = 8;

// sum over cc < n of src[cc * stride]
__device__ __forceinline__ uint32_t sum_chunks(const uint32_t* src, size_t stride, int n) {
    uint32_t s = 0u;
    for (int c0 = 0; c0 < n; c0 += kBatch) {
        uint32_t v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) v[j] = c0 + j < n ? src[static_cast<size_t>(c0 + j) * stride] : 0u;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) s += v[j];
    }
    return s;
}

// Exclusive prefix sums over the block of W packed words (two 16-bit
// counters each; every block total stays below 2^16), in thread order.
template <int W>
__device__ __forceinline__ void block_scan_packed(const uint32_t (&v)[W], uint32_t (&excl)[W],
                                                  uint32_t (&total)[W], uint32_t* wsum /*[W][16]*/) {
    const int lane = lane_id();
    const int w = static_cast<int>(threadIdx.x >> 6);
    const int nw = static_cast<int>(blockDim.x >> 6);
    uint32_t inc[W];
#pragma unroll
    for (int i = 0; i < W; ++i) {
        inc[i] = wave_inclusive_scan(v[i]);
        if (lane == 63) wsum[i * 16 + w] = inc[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < W; ++i) {
        uint32_t before = 0, all = 0;
        for (int j = 0; j < nw; ++j) {
            const uint32_t s = wsum[i * 16 + j];
            before += j < w ? s : 0u;
            all += s;
        }
        excl[i] = before + inc[i] - v[i];
        total[i] = all;
    }
    __syncthreads();
}

template <int D, int NREP, int WAVES>
struct FusedSmem {
    static constexpr int CPR = D * 2 / 16;          // 16-byte chunks per K row
    static constexpr int HS = kHist1Bins + 8;       // level-1 words per head (padded)
    static constexpr int HC = 2;                    // level-1 histogram copies
    static constexpr int CS = NREP * HS + 2;        // words per copy
    static constexpr int EPW = 64 * kFusedPPT;      // gather entries per wave and sub-chunk, at most
    static constexpr int NP = NREP == 4 ? 4 : (NREP == 2 ? 2 : 1);
    union {
        chunk_t stage[WAVES][64 * CPR];             // phase 1: K tile transposes
        struct {
            uint32_t epos[WAVES][EPW];              // phase 3: gather lists (positions,
            __align__(16) float ep[WAVES][EPW][NP]; //   each head's weight)
            float red[WAVES][NREP][D + 1];          // phase 3: the waves' sums
        } g;
    } big;
    __align__(16) float u[NREP][D + 4];             // unit query vectors (rows padded)
    uint32_t hist1[HC * CS];
    uint32_t h1[NREP][kHist1Bins];    // phase 2: the row's level 1; phase 3: earlier chunks' level 2
    uint32_t h2[NREP][kHist2Bins];    // this chunk's level 2
    uint32_t h2tot[NREP][kHist2Bins]; // phase 3: the row's level 2
    uint32_t wsum[2 * 16];
    uint32_t T1[NREP], above1[NREP], T2[NREP], above2[NREP], gt1[NREP], smax[NREP];
    uint32_t quota[NREP], outoff[NREP];
    float qscale[NREP], mlog[NREP];
    uint64_t tag;
};

struct FusedArgs {
    const void* Q;
    const uint8_t* K;
    const uint8_t* V;
    void* O;
    int32_t* idx;       // [B*H][k] or null
    uint16_t* keys;     // [B*H][ldsc]
    uint8_t* res;       // [B*H][ldsc]
    uint32_t* hist1p;   // [B*H][chunks][256]
    uint32_t* hist2p;   // [B*H][chunks][260]: level-2 bins, keys above T1, ordered max score
    float* part;        // [B*H][chunks][D + 1]: l, o
    FusedCtl* ctl;
    uint64_t nonce;
    float eps, scale;
    long long ldn, ldsc;
    int N, k, chunks, P, gx;
};

template <int DT, int D, int NREP, int WAVES, bool EMIT>
__global__ __launch_bounds__(64 * WAVES) void fused_decode_kernel(FusedArgs a) {
    constexpr int THREADS = 64 * WAVES;
    constexpr int RB = D * 2;                       // bytes per K/V row (fp16/bf16)
    constexpr int CPR = RB / 16;
    constexpr int EPC = 8;                          // elements per 16-byte chunk
    constexpr int LPR = CPR;                        // lanes per V row in the gather
    constexpr int RPI = 64 / LPR;                   // V rows per gather instruction
    constexpr int TILE = RPI * kFusedU;
    constexpr int SUB = THREADS * kFusedPPT;        // positions per sub-chunk
    constexpr int W2 = (NREP + 1) / 2;              // packed words for NREP counters
    using SM = FusedSmem<D, NREP, WAVES>;
    static_assert(NREP <= 4 && WAVES >= NREP && WAVES <= 16, "one MFMA chain, a wave per head");
    static_assert(kFusedWgPerXcd * kFusedXcds == 256, "grid of 256 workgroups");
    __shared__ SM sm;

    const int t = static_cast<int>(threadIdx.x);
    const int lane = lane_id();
    const int wave = t >> 6;
    const uint32_t x = xcc_id();
    const int rank = static_cast<int>(blockIdx.x) / kFusedXcds;
    const int gi = rank / a.chunks;
    const int c = rank % a.chunks;
    const int bg = static_cast<int>(x) + kFusedXcds * gi;  // b * Hkv + g
    const size_t head0 = static_cast<size_t>(bg) * NREP;    // row (b * H + h) of head 0
    const uint8_t* Kg = a.K + static_cast<size_t>(bg) * static_cast<size_t>(a.ldn) * RB;
    const uint8_t* Vg = a.V + static_cast<size_t>(bg) * static_cast<size_t>(a.ldn) * RB;
    const int p0 = c * a.P;
    const int p1 = (p0 + a.P < a.N) ? p0 + a.P : a.N;      // positions [p0, p1); may be empty
    const uint32_t kk = static_cast<uint32_t>(a.k);
    uint64_t* flags = a.ctl->flags[x];

    // ------------------------------------------------------------ phase 1
    // The wave's tiles (64 rows each): m-th at row tile_row0(m), ntw of them.
    //   kP1Mode 0: the chunk's tiles w, w + WAVES, ... (each workgroup streams
    //              its own chunk);
    //   kP1Mode 1: the group's tiles (m * chunks + c) * WAVES + w (the group's
    //              workgroups sweep its rows side by side).
    // Which workgroup scores a row does not matter to the later phases: the
    // keys are stored by position and the level-1 counts are summed per row.
    const int ntg = (a.N + 63) / 64;  // the group's tiles
    int ntw;
    if constexpr (kP1Mode == 0) {
        const int ntile = p1 > p0 ? (p1 - p0 + 63) / 64 : 0;
        ntw = ntile > wave ? (ntile - wave + WAVES - 1) / WAVES : 0;
    } else {
        const int first = c * WAVES + wave;
        ntw = ntg > first ? (ntg - first + a.chunks * WAVES - 1) / (a.chunks * WAVES) : 0;
    }
    auto tile_row0 = [&](int m) -> long long {
        if constexpr (kP1Mode == 0) return static_cast<long long>(p0) + (static_cast<long long>(m) * WAVES + wave) * 64;
        else return ((static_cast<long long>(m) * a.chunks + c) * WAVES + wave) * 64;
    };
    const long long last_chunk = static_cast<long long>(a.N) * RB - 16;
    chunk_t buf0[CPR], buf1[CPR];
    auto load_tile = [&](chunk_t (&dst)[CPR], int m) {
        const long long base = tile_row0(m) * RB + lane * 16;
#pragma unroll
        for (int i = 0; i < CPR; ++i) {
            long long off = base + static_cast<long long>(i) * 1024;
            off = off < last_chunk ? off : last_chunk;
            dst[i] = __builtin_nontemporal_load(reinterpret_cast<const chunk_t*>(Kg + off));
        }
    };
    // Unconditional loads (a tile past the chunk's end reads the group's last
    // 16 bytes, in bounds, and is never processed), so that every wait in the
    // tile loop below counts the same loads on every path.
    load_tile(buf0, 0);
    if constexpr (kP1Depth == 2) load_tile(buf1, 1);

    if (t == 0) {
        const uint32_t ctr = __builtin_nontemporal_load(&a.ctl->ctr[x][0]);
        sm.tag = mix64(a.nonce ^ (static_cast<uint64_t>(ctr) * 0x9E3779B97F4A7C15ull)) & ~0xffffull;
    }
    for (int h = wave; h < NREP; h += WAVES)
        unit_row<DT, D>(a.Q, (head0 + h) * static_cast<size_t>(D), a.eps, &sm.u[h][0]);
    for (int i = t; i < SM::HC * SM::CS; i += THREADS) sm.hist1[i] = 0u;
    __syncthreads();
    const uint64_t tag = sm.tag;

    chunk_t* st = sm.big.stage[wave];
    // A tile (64 rows) goes through LDS, 16-byte chunk (row, i) at
    // row * CPR + (i ^ swz(row)): conflict-free writes and per-row reads.
    auto swz = [](int row) { return CPR == 8 ? ((row >> 1) & 7) : (row & 15); };
    auto stage = [&](const chunk_t (&data)[CPR]) {
#pragma unroll
        for (int i = 0; i < CPR; ++i) {
            const int ci = i * 64 + lane;
            const int row = ci / CPR, cc = ci % CPR;
            st[row * CPR + (cc ^ swz(row))] = data[i];
        }
        __builtin_amdgcn_wave_barrier();
    };
    // Byte offset of the lane's row, chunk 0 ^ swz: chunk i of the row is at
    // rd ^ (16 i) (the row starts on a multiple of RB, a power of two above 16 i).
    int rd = lane * RB + swz(lane) * 16;
    // Run the MFMA chain over the staged tile (rows from row0), store keys and
    // residuals, count level 1.
    auto compute = [&](long long row0) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // lane 4b + j multiplies by u[j][d] (heads j >= NREP read head 0 and are not stored);
        // the empty asm statements keep these LDS reads and their addresses inside the
        // tile loop (hoisted, they would cost registers the loads in flight need).
        asm volatile("" : "+v"(rd) :: "memory");
        const float* urow = &sm.u[(lane & 3) < NREP ? (lane & 3) : 0][0];
        const char* stb = reinterpret_cast<const char*>(st);
#pragma unroll
        for (int i = 0; i < CPR; ++i) {
            const chunk_t kc = *reinterpret_cast<const chunk_t*>(stb + (rd ^ (i * 16)));
#pragma unroll
            for (int e4 = 0; e4 < EPC; e4 += 4) {
                const f32x4 uv = *reinterpret_cast<const f32x4*>(urow + i * EPC + e4);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc = __builtin_amdgcn_mfma_f32_4x4x1f32(chunk_elem<DT>(kc, e4 + e), uv[e], acc, 0, 0, 0);
            }
        }
        __builtin_amdgcn_wave_barrier();
        const int jl = lane & 3;
        if (jl < NREP) {
            const long long n0 = row0 + (lane & ~3);
            uint32_t sb[4], sk[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                sb[v] = f32_to_bf16_bits(acc[v]);
                sk[v] = bf16_key(sb[v]);
            }
            const size_t rowoff = (head0 + jl) * static_cast<size_t>(a.ldsc);
            if (n0 + 3 < a.N) {
                *reinterpret_cast<uint2*>(a.keys + rowoff + n0) = make_uint2(sk[0] | (sk[1] << 16), sk[2] | (sk[3] << 16));
                *reinterpret_cast<uint32_t*>(a.res + rowoff + n0) =
                    score_residual(acc[0], sb[0]) | (score_residual(acc[1], sb[1]) << 8) |
                    (score_residual(acc[2], sb[2]) << 16) | (score_residual(acc[3], sb[3]) << 24);
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (n0 + v < a.N) {
                        a.keys[rowoff + n0 + v] = static_cast<uint16_t>(sk[v]);
                        a.res[rowoff + n0 + v] = static_cast<uint8_t>(score_residual(acc[v], sb[v]));
                    }
            }
            const int hcopy = (lane >> 2) % SM::HC;
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (n0 + v < a.N) atomicAdd(&sm.hist1[hcopy * SM::CS + jl * SM::HS + (sk[v] >> kHist2Bits)], 1u);
        }
    };
    // A buffer is staged to LDS and reloaded with a later tile before the
    // tile is multiplied out, so kP1Depth tiles are in flight meanwhile.
    if constexpr (kP1Depth == 2) {
        for (int m = 0; m < ntw; m += 2) {
            stage(buf0);
            load_tile(buf0, m + 2);
            compute(tile_row0(m));
            stage(buf1);
            load_tile(buf1, m + 3);
            if (m + 1 < ntw) compute(tile_row0(m + 1));
        }
    } else {
        for (int m = 0; m < ntw; ++m) {
            stage(buf0);
            load_tile(buf0, m + 1);
            compute(tile_row0(m));
        }
    }
    __syncthreads();
    for (int i = t; i < NREP * kHist1Bins; i += THREADS) {
        const int h = i / kHist1Bins, bin = i % kHist1Bins;
        uint32_t s = 0u;
#pragma unroll
        for (int cp = 0; cp < SM::HC; ++cp) s += sm.hist1[cp * SM::CS + h * SM::HS + bin];
        a.hist1p[((head0 + h) * a.chunks + c) * kHist1Bins + bin] = s;
    }
    xcd_barrier(flags, rank, tag, 1u);

    // ------------------------------------------------------------ phase 2
    for (int i = t; i < NREP * kHist1Bins; i += THREADS) {
        const int h = i / kHist1Bins, bin = i % kHist1Bins;
        sm.h1[h][bin] = sum_chunks(a.hist1p + (head0 + h) * a.chunks * kHist1Bins + bin, kHist1Bins, a.chunks);
        sm.h2[h][bin] = 0u;
    }
    if (t < NREP) {
        sm.T1[t] = 0u;
        sm.above1[t] = 0u;
        sm.gt1[t] = 0u;
        sm.smax[t] = 0u;
    }
    __syncthreads();
    if (wave < NREP) {
        uint32_t c4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c4[i] = sm.h1[wave][255 - 4 * lane - i];
        find_bin_regs(c4, kk, &sm.T1[wave], &sm.above1[wave]);
    }
    __syncthreads();
    {
        uint32_t T1r[NREP], gtc[NREP];
        float smx[NREP];
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
            T1r[h] = sm.T1[h];
            gtc[h] = 0u;
            smx[h] = -INFINITY;
        }
        for (int sb0 = p0; sb0 < p1; sb0 += SUB) {
            const int pos = sb0 + t * kFusedPPT;
            if (pos < p1) {
#pragma unroll
                for (int h = 0; h < NREP; ++h) {
                    const size_t ro = (head0 + h) * static_cast<size_t>(a.ldsc) + pos;
                    const uint2 kw = *reinterpret_cast<const uint2*>(a.keys + ro);
                    const uint32_t r4 = *reinterpret_cast<const uint32_t*>(a.res + ro);
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        if (pos + v >= p1) continue;
                        const uint32_t key = ((v < 2 ? kw.x : kw.y) >> ((v & 1) * 16)) & 0xffffu;
                        const uint32_t b1 = key >> kHist2Bits;
                        if (b1 == T1r[h]) atomicAdd(&sm.h2[h][key & (kHist2Bins - 1)], 1u);
                        gtc[h] += b1 > T1r[h] ? 1u : 0u;
                        smx[h] = fmaxf(smx[h], score_from_key(key, (r4 >> (8 * v)) & 0xffu));
                    }
                }
            }
        }
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                gtc[h] += __shfl_xor(gtc[h], off, 64);
                smx[h] = fmaxf(smx[h], __shfl_xor(smx[h], off, 64));
            }
            if (lane == 0) {
                if (gtc[h] != 0u) atomicAdd(&sm.gt1[h], gtc[h]);
                atomicMax(&sm.smax[h], ordered_bits(smx[h]));
            }
        }
    }
    __syncthreads();
    for (int i = t; i < NREP * (kHist2Bins + 2); i += THREADS) {
        const int h = i / (kHist2Bins + 2), bin = i % (kHist2Bins + 2);
        const uint32_t v = bin < kHist2Bins ? sm.h2[h][bin] : (bin == kHist2Bins ? sm.gt1[h] : sm.smax[h]);
        a.hist2p[((head0 + h) * a.chunks + c) * kFusedHist2Stride + bin] = v;
    }
    xcd_barrier(flags, rank, tag, 2u);

    // ------------------------------------------------------------ phase 3
    for (int i = t; i < NREP * kHist2Bins; i += THREADS) {
        const int h = i / kHist2Bins, bin = i % kHist2Bins;
        const uint32_t* src = a.hist2p + (head0 + h) * a.chunks * kFusedHist2Stride + bin;
        const uint32_t pre = sum_chunks(src, kFusedHist2Stride, c);  // earlier chunks
        sm.h2tot[h][bin] = pre + sum_chunks(src + static_cast<size_t>(c) * kFusedHist2Stride, kFusedHist2Stride,
                                            a.chunks - c);
        sm.h1[h][bin] = pre;
    }
    if (t < NREP) {
        const uint32_t* src = a.hist2p + (head0 + t) * a.chunks * kFusedHist2Stride;
        uint32_t mx = 0u;
        for (int c0 = 0; c0 < a.chunks; c0 += kBatch) {
            uint32_t m[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j)
                m[j] = c0 + j < a.chunks ? src[static_cast<size_t>(c0 + j) * kFusedHist2Stride + kHist2Bins + 1] : 0u;
#pragma unroll
            for (int j = 0; j < kBatch; ++j) mx = m[j] > mx ? m[j] : mx;
        }
        sm.smax[t] = mx;
        sm.gt1[t] = sum_chunks(src + kHist2Bins, kFusedHist2Stride, c);  // keys above T1 in earlier chunks
        sm.T2[t] = 0u;
        sm.above2[t] = 0u;
    }
    __syncthreads();
    if (wave < NREP) {
        const int h = wave;
        uint32_t c4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c4[i] = sm.h2tot[h][255 - 4 * lane - i];
        find_bin_regs(c4, kk - sm.above1[h], &sm.T2[h], &sm.above2[h]);
        const float qn = row_norm<DT, D>(a.Q, (head0 + h) * static_cast<size_t>(D), a.eps);
        if (lane == 0) sm.qscale[h] = qn * a.scale;
    }
    __syncthreads();
    if (wave < NREP) {
        const int h = wave;
        const uint32_t T2 = sm.T2[h];
        // earlier chunks' level-2 counts above T2 (for the index offsets)
        uint32_t s = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int bin = 255 - 4 * lane - i;
            s += static_cast<uint32_t>(bin) > T2 ? sm.h1[h][bin] : 0u;
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) {
            const uint32_t need = kk - sm.above1[h] - sm.above2[h];  // ties at T that are selected
            const uint32_t tiepre = sm.h1[h][T2];                    // ties in earlier chunks
            const uint32_t ties = sm.h2[h][T2];                      // ties in this chunk
            const uint32_t left = need > tiepre ? need - tiepre : 0u;
            sm.quota[h] = left < ties ? left : ties;
            sm.outoff[h] = sm.gt1[h] + s + (need < tiepre ? need : tiepre);
            sm.mlog[h] = from_ordered(sm.smax[h]) * sm.qscale[h];
        }
    }
    __syncthreads();

    // block-uniform per-head values, kept in scalar registers
    auto uni32 = [](uint32_t v) { return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v))); };
    auto unif = [](float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); };
    uint32_t T[NREP], quota[NREP], tie_carry[NREP], sel_carry[NREP], outoff[NREP];
    float qs[NREP], mlog[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        T[h] = uni32((sm.T1[h] << kHist2Bits) | sm.T2[h]);
        quota[h] = uni32(sm.quota[h]);
        outoff[h] = uni32(sm.outoff[h]);
        qs[h] = unif(sm.qscale[h]);
        mlog[h] = unif(sm.mlog[h]);
        tie_carry[h] = 0u;
        sel_carry[h] = 0u;
    }
    const int li = lane % LPR;  // 16-byte slice of a V row
    const int rs = lane / LPR;  // row slot within a gather instruction
    float l[NREP], o[NREP][EPC];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPC; ++e) o[h][e] = 0.0f;
    }
    uint32_t* epos = sm.big.g.epos[wave];
    float (*ep)[SM::NP] = sm.big.g.ep[wave];
    auto key_of = [](const uint2& kw, int v) { return ((v < 2 ? kw.x : kw.y) >> ((v & 1) * 16)) & 0xffffu; };

    for (int sb0 = p0; sb0 < p1; sb0 += SUB) {
        const int pos = sb0 + t * kFusedPPT;
        uint2 kw[NREP];
        uint32_t r4[NREP], gtb[NREP], eqb[NREP];
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
            gtb[h] = 0u;
            eqb[h] = 0u;
            kw[h] = make_uint2(0u, 0u);
            r4[h] = 0u;
            if (pos < p1) {
                const size_t ro = (head0 + h) * static_cast<size_t>(a.ldsc) + pos;
                kw[h] = *reinterpret_cast<const uint2*>(a.keys + ro);
                r4[h] = *reinterpret_cast<const uint32_t*>(a.res + ro);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t key = key_of(kw[h], v);
                const bool in = pos + v < p1;
                gtb[h] |= (in && key > T[h]) ? (1u << v) : 0u;
                eqb[h] |= (in && key == T[h]) ? (1u << v) : 0u;
            }
        }
        // tie ranks: ties of this chunk in position order take the quota
        uint32_t cnt[W2], excl[W2], tot[W2];
#pragma unroll
        for (int i = 0; i < W2; ++i) cnt[i] = 0u;
#pragma unroll
        for (int h = 0; h < NREP; ++h) cnt[h >> 1] |= static_cast<uint32_t>(__builtin_popcount(eqb[h])) << ((h & 1) * 16);
        block_scan_packed<W2>(cnt, excl, tot, sm.wsum);
        uint32_t selb[NREP];
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
            uint32_t rank_t = tie_carry[h] + ((excl[h >> 1] >> ((h & 1) * 16)) & 0xffffu);
            uint32_t take = 0u;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (eqb[h] & (1u << v)) {
                    take |= rank_t < quota[h] ? (1u << v) : 0u;
                    ++rank_t;
                }
            }
            selb[h] = gtb[h] | take;
            tie_carry[h] = uni32(tie_carry[h] + ((tot[h >> 1] >> ((h & 1) * 16)) & 0xffffu));
        }
        if constexpr (EMIT) {
#pragma unroll
            for (int i = 0; i < W2; ++i) cnt[i] = 0u;
#pragma unroll
            for (int h = 0; h < NREP; ++h)
                cnt[h >> 1] |= static_cast<uint32_t>(__builtin_popcount(selb[h])) << ((h & 1) * 16);
            block_scan_packed<W2>(cnt, excl, tot, sm.wsum);
#pragma unroll
            for (int h = 0; h < NREP; ++h) {
                uint32_t off = outoff[h] + sel_carry[h] + ((excl[h >> 1] >> ((h & 1) * 16)) & 0xffffu);
                int32_t* out = a.idx + (head0 + h) * static_cast<size_t>(a.k);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if ((selb[h] & (1u << v)) && off < kk) out[off++] = pos + v;
                sel_carry[h] = uni32(sel_carry[h] + ((tot[h >> 1] >> ((h & 1) * 16)) & 0xffffu));
            }
        }
        // the positions any head selected, with each head's weight
        // exp(logit - row max), into the wave's list
        uint32_t uni = 0u;
#pragma unroll
        for (int h = 0; h < NREP; ++h) uni |= selb[h];
        const uint32_t n = static_cast<uint32_t>(__builtin_popcount(uni));
        const uint32_t incl = wave_inclusive_scan(n);
        const uint32_t cntw = uni32(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63)));
        uint32_t slot = incl - n;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (!(uni & (1u << v))) continue;
            epos[slot] = static_cast<uint32_t>(pos + v);
#pragma unroll
            for (int h = 0; h < NREP; ++h) {
                float p = 0.0f;
                if (selb[h] & (1u << v))
                    p = expf(score_from_key(key_of(kw[h], v), (r4[h] >> (8 * v)) & 0xffu) * qs[h] - mlog[h]);
                ep[slot][h] = p;
            }
            ++slot;
        }
        __syncthreads();
        // gather the listed V rows: RPI per instruction, kFusedU instructions
        // per tile, the next tile's rows in flight while one is added up
        auto fetch = [&](chunk_t (&vv)[kFusedU], uint32_t e0) {
#pragma unroll
            for (int u = 0; u < kFusedU; ++u) {
                const uint32_t ei = e0 + static_cast<uint32_t>(u * RPI + rs);
                const uint32_t pv = epos[ei < cntw ? ei : 0u];
                vv[u] = *reinterpret_cast<const chunk_t*>(Vg + static_cast<size_t>(pv) * RB + li * 16);
            }
        };
        auto accumulate = [&](const chunk_t (&vv)[kFusedU], uint32_t e0) {
#pragma unroll
            for (int u = 0; u < kFusedU; ++u) {
                const uint32_t ei = e0 + static_cast<uint32_t>(u * RPI + rs);
                float pp[NREP];
#pragma unroll
                for (int h = 0; h < NREP; ++h) pp[h] = ei < cntw ? ep[ei][h] : 0.0f;
#pragma unroll
                for (int e = 0; e < EPC; ++e) {
                    const float ve = chunk_elem<DT>(vv[u], e);
#pragma unroll
                    for (int h = 0; h < NREP; ++h) o[h][e] = __builtin_fmaf(pp[h], ve, o[h][e]);
                }
#pragma unroll
                for (int h = 0; h < NREP; ++h) l[h] += pp[h];
            }
        };
        // The fetches are unconditional (entries past the list's end read the
        // first entry's row again and weigh it 0), so that every wait counts
        // the same loads on every path and the next tile stays in flight.
        if (cntw > 0u) {
            chunk_t va[kFusedU], vb[kFusedU];
            fetch(va, 0u);
            fetch(vb, TILE);
            for (uint32_t e0 = 0; e0 < cntw; e0 += 2 * TILE) {
                accumulate(va, e0);
                fetch(va, e0 + 2 * TILE);
                accumulate(vb, e0 + TILE);
                fetch(vb, e0 + 3 * TILE);
            }
        }
        __syncthreads();  // the list is rewritten by the next sub-chunk
    }

    // the row slots' and the waves' sums, then this chunk's record per head
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) {
            l[h] += __shfl_xor(l[h], off, 64);
#pragma unroll
            for (int e = 0; e < EPC; ++e) o[h][e] += __shfl_xor(o[h][e], off, 64);
        }
        if (lane == 0) sm.big.g.red[wave][h][0] = l[h];
        if (rs == 0) {
#pragma unroll
            for (int e = 0; e < EPC; ++e) sm.big.g.red[wave][h][1 + li * EPC + e] = o[h][e];
        }
    }
    __syncthreads();
    for (int i = t; i < NREP * (D + 1); i += THREADS) {
        const int h = i / (D + 1), d = i % (D + 1);
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) s += sm.big.g.red[w][h][d];
        a.part[((head0 + h) * a.chunks + c) * (D + 1) + d] = s;
    }
    xcd_barrier(flags, rank, tag, 3u);

    // ------------------------------------------------------------ phase 4
    // the XCD's gx * NREP rows, dealt round robin over its 32 workgroups
    for (int r = rank; r < a.gx * NREP; r += kFusedWgPerXcd) {
        const int gi2 = r / NREP, h = r % NREP;
        const size_t row = (static_cast<size_t>(x) + kFusedXcds * static_cast<size_t>(gi2)) * NREP + h;
        const float* src = a.part + row * a.chunks * (D + 1);
        for (int d = t; d < D; d += THREADS) {
            float L = 0.0f, S = 0.0f;
            for (int c0 = 0; c0 < a.chunks; c0 += kBatch) {
                float lv[kBatch], sv[kBatch];
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    const bool in = c0 + j < a.chunks;
                    const size_t o = static_cast<size_t>(c0 + j) * (D + 1);
                    lv[j] = in ? src[o] : 0.0f;
                    sv[j] = in ? src[o + 1 + d] : 0.0f;
                }
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {  // chunk order, as before
                    L += lv[j];
                    S += sv[j];
                }
            }
            store_out<DT>(a.O, row * D + d, S / L);
        }
    }
    if (rank == 0 && t == 0) {
        const uint32_t ctr = a.ctl->ctr[x][0];
        a.ctl->ctr[x][0] = ctr + 1u;  // every workgroup of this XCD read it before barrier 1
    }
}

template <int DT, int D, int NREP, int WAVES>
hipError_t launch_fused_t(const FusedArgs& a, bool emit, hipStream_t s) {
    if (emit)
        launch_kernel(fused_decode_kernel<DT, D, NREP, WAVES, true>, dim3(kFusedXcds * kFusedWgPerXcd),
                      dim3(64 * WAVES), 0, s, a);
    else
        launch_kernel(fused_decode_kernel<DT, D, NREP, WAVES, false>, dim3(kFusedXcds * kFusedWgPerXcd),
                      dim3(64 * WAVES), 0, s, a);
    return hipGetLastError();
}

template <int DT, int D>
hipError_t launch_fused_rep(const FusedArgs& a, int n_rep, bool emit, hipStream_t s) {
    constexpr int W = D == 64 ? 16 : 8;
    switch (n_rep) {
        case 1: return launch_fused_t<DT, D, 1, W>(a, emit, s);
        case 2: return launch_fused_t<DT, D, 2, W>(a, emit, s);
        case 4: return launch_fused_t<DT, D, 4, W>(a, emit, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

FusedShape fused_shape(int dtype, int B, int H, int Hkv, int N, int D, int k) {
    FusedShape f{};
    f.ok = false;
    const int n_rep = Hkv > 0 ? H / Hkv : 0;
    const int G = B * Hkv;
    if ((dtype != kF16 && dtype != kBF16) || (D != 64 && D != 128) || (n_rep != 1 && n_rep != 2 && n_rep != 4) ||
        G <= 0 || G % kFusedXcds != 0 || k <= 0 || k >= N)
        return f;
    const int gx = G / kFusedXcds;
    if (gx > kFusedWgPerXcd || kFusedWgPerXcd % gx != 0) return f;
    f.gx = gx;
    f.chunks = kFusedWgPerXcd / gx;
    const int per = (N + f.chunks - 1) / f.chunks;
    f.P = (per + 63) / 64 * 64;
    // the select phases count in 16-bit fields per sub-chunk and in uint32 per row
    f.ok = true;
    return f;
}

hipError_t launch_fused_decode(const void* Q, const void* K, const void* V, int dtype, void* O,
                               int32_t* idx, uint16_t* keys, uint8_t* res, uint32_t* hist1p,
                               uint32_t* hist2p, float* part, FusedCtl* ctl, uint64_t nonce, float eps,
                               int B, int H, int Hkv, int N, long long ldn, long long ldsc, int D, int k,
                               const FusedShape& f, hipStream_t s) {
    (void)B;
    FusedArgs a{};
    a.Q = Q;
    a.K = static_cast<const uint8_t*>(K);
    a.V = static_cast<const uint8_t*>(V);
    a.O = O;
    a.idx = idx;
    a.keys = keys;
    a.res = res;
    a.hist1p = hist1p;
    a.hist2p = hist2p;
    a.part = part;
    a.ctl = ctl;
    a.nonce = nonce;
    a.eps = eps;
    a.scale = static_cast<float>(1.0 / sqrt(static_cast<double>(D)));
    a.ldn = ldn;
    a.ldsc = ldsc;
    a.N = N;
    a.k = k;
    a.chunks = f.chunks;
    a.P = f.P;
    a.gx = f.gx;
    const int n_rep = H / Hkv;
    const bool emit = idx != nullptr;
    if (dtype == kF16) return D == 64 ? launch_fused_rep<kF16, 64>(a, n_rep, emit, s) : launch_fused_rep<kF16, 128>(a, n_rep, emit, s);
    if (dtype == kBF16) return D == 64 ? launch_fused_rep<kBF16, 64>(a, n_rep, emit, s) : launch_fused_rep<kBF16, 128>(a, n_rep, emit, s);
    return hipErrorInvalidValue;
}

uint32_t* fused_error_word() {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_fused_err)) != hipSuccess) return nullptr;
    return static_cast<uint32_t*>(p);
}

}  // namespace dcr
