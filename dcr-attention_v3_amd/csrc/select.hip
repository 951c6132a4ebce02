// select.hip -- exact top-K selection over bf16 score rows.
//
// Replaces the reference's Pass 2 (topk_pass2_select,
// dcr_attention/kernel/triton/topk_axis_pass2.py:16-43; M1 twin
// _select_topk_indices, qaxis_topk_reference.py:91-108), which runs a full
// stable argsort of every row.  The contract is the same: for each row, the
// k positions that a stable descending sort of the scores lists first (ties
// toward the lower index), returned in ascending index order, int32.
//
// Algorithm (radix select on the order-preserving 16-bit key, no sort):
//   1. level-1 histogram of key >> 5 (2048 bins) -- produced by the score
//      kernel (fused) or by hist_kernel;
//   2. one workgroup of 1024 threads per row: a reverse block scan of the
//      level-1 histogram finds the bin T1 holding the k-th largest key;
//   3. the row's keys are loaded once into registers (each thread owns a
//      contiguous run of KPT positions); a 32-bin level-2 histogram of the
//      keys in bin T1 gives the exact threshold key T and the number of ties
//      at T that are selected (need = k - #{key > T});
//   4. one block-wide exclusive scan of the packed (ties, above) counts gives
//      every thread its output offset and how many ties precede it; threads
//      then emit key > T, and key == T while the tie quota lasts, in position
//      order -- so the output is ascending with no sort.
#include "dcr_common.h"
#include "dcr_kernels.h"

namespace dcr {
namespace {

constexpr int kSelectThreads = 1024;
constexpr int kSelectWaves = kSelectThreads / 64;

template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
    const int lane = lane_id();
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const T y = __shfl_up(v, off, 64);
        if (lane >= off) v += y;
    }
    return v;
}

// Exclusive prefix sum over the 1024 threads of the block, in thread order.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* wsum) {
    const int lane = lane_id();
    const int w = static_cast<int>(threadIdx.x >> 6);
    const T incl = wave_inclusive_scan(v);
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    if (w == 0) {
        const T s = (lane < kSelectWaves) ? wsum[lane] : T(0);
        const T si = wave_inclusive_scan(s);
        if (lane < kSelectWaves) wsum[lane] = si - s;
    }
    __syncthreads();
    const T r = wsum[w] + incl - v;
    __syncthreads();
    return r;
}

// Level-1 histogram of a slice of one score row.
__global__ __launch_bounds__(256) void hist_kernel(const uint16_t* __restrict__ scores,
                                                   uint32_t* __restrict__ hist1, int N,
                                                   int per_block) {
    __shared__ uint32_t h[kHist1Bins];
    for (int i = static_cast<int>(threadIdx.x); i < kHist1Bins; i += 256) h[i] = 0u;
    __syncthreads();
    const size_t row = blockIdx.y;
    const uint16_t* s = scores + row * static_cast<size_t>(N);
    const int p0 = static_cast<int>(blockIdx.x) * per_block;
    const int p1 = (p0 + per_block < N) ? p0 + per_block : N;
    for (int p = p0 + static_cast<int>(threadIdx.x); p < p1; p += 256)
        atomicAdd(&h[bf16_key(s[p]) >> kHist2Bits], 1u);
    __syncthreads();
    uint32_t* hg = hist1 + row * kHist1Bins;
    for (int i = static_cast<int>(threadIdx.x); i < kHist1Bins; i += 256)
        if (h[i] != 0u) atomicAdd(hg + i, h[i]);
}

// Keys of positions [p, p + SEG) as packed 16-bit pairs; positions >= N get
// key 0, below every real key (real keys are >= 0x007F).
template <int SEG>
__device__ __forceinline__ void load_keys(uint32_t (&kw)[SEG / 2], const uint16_t* __restrict__ srow,
                                          int N, int p, bool vec_ok) {
#pragma unroll
    for (int v = 0; v < SEG / 8; ++v) {
        const int q = p + v * 8;
        if (vec_ok && q + 8 <= N) {
            const chunk_t c = *reinterpret_cast<const chunk_t*>(srow + q);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                kw[v * 4 + j] = bf16_key(c[j] & 0xffffu) | (bf16_key(c[j] >> 16) << 16);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = (q + 2 * j < N) ? bf16_key(srow[q + 2 * j]) : 0u;
                const uint32_t hi = (q + 2 * j + 1 < N) ? bf16_key(srow[q + 2 * j + 1]) : 0u;
                kw[v * 4 + j] = lo | (hi << 16);
            }
        }
    }
}

template <int SEG>
__device__ __forceinline__ uint32_t key_at(const uint32_t (&kw)[SEG / 2], int j) {
    return (kw[j >> 1] >> ((j & 1) * 16)) & 0xffffu;
}

// One workgroup per row; thread t owns positions [t*KPT, (t+1)*KPT), walked
// in segments of SEG <= 32 keys.  With a single segment the keys stay in
// registers across the passes; otherwise each pass re-reads them (from L2).
template <int KPT>
__global__ __launch_bounds__(kSelectThreads) void select_kernel(const uint16_t* __restrict__ scores,
                                                                const uint32_t* __restrict__ hist1,
                                                                int32_t* __restrict__ idx, int N,
                                                                int k) {
    constexpr int SEG = KPT < 32 ? KPT : 32;
    constexpr int NSEG = KPT / SEG;
    static_assert(SEG % 8 == 0 && KPT % SEG == 0, "keys are loaded in chunks of 8");
    __shared__ uint32_t wsum32[kSelectWaves];
    __shared__ unsigned long long wsum64[kSelectWaves];
    __shared__ uint32_t h2[kHist2Bins];
    __shared__ uint32_t sh_T1, sh_above1, sh_T, sh_need;

    const int t = static_cast<int>(threadIdx.x);
    const size_t row = blockIdx.x;
    const uint16_t* srow = scores + row * static_cast<size_t>(N);
    const uint32_t* hrow = hist1 + row * kHist1Bins;
    const uint32_t kk = static_cast<uint32_t>(k);
    const int p0 = t * KPT;
    const bool vec_ok = (N % 8) == 0 && (reinterpret_cast<uintptr_t>(scores) & 15u) == 0;

    // Keys first: their loads overlap the level-1 scan below.
    uint32_t kw[SEG / 2];
    if constexpr (NSEG == 1) load_keys<SEG>(kw, srow, N, p0, vec_ok);

    // --- 1. level-1 bin T1 holding the k-th largest key ---------------------
    // Thread t owns bins 2047-2t and 2046-2t; scanning in that order makes the
    // exclusive prefix the count of keys in higher bins.
    static_assert(kHist1Bins == 2 * kSelectThreads, "two level-1 bins per thread");
    const uint32_t c0 = hrow[kHist1Bins - 1 - 2 * t];
    const uint32_t c1 = hrow[kHist1Bins - 2 - 2 * t];
    if (t < kHist2Bins) h2[t] = 0u;
    if (t == 0) {  // defaults if the histogram were inconsistent (then fewer than k are written)
        sh_T1 = 0u;
        sh_above1 = 0u;
        sh_T = 0xffffu;
        sh_need = 0u;
    }
    const uint32_t above = block_exclusive_scan<uint32_t>(c0 + c1, wsum32);
    if (above < kk && above + c0 >= kk) {
        sh_T1 = static_cast<uint32_t>(kHist1Bins - 1 - 2 * t);
        sh_above1 = above;
    } else if (above + c0 < kk && above + c0 + c1 >= kk) {
        sh_T1 = static_cast<uint32_t>(kHist1Bins - 2 - 2 * t);
        sh_above1 = above + c0;
    }

    __syncthreads();  // sh_T1 / sh_above1 / h2 zeroing visible

    // --- 2. level-2 histogram inside T1, exact threshold T ------------------
    const uint32_t T1 = sh_T1;
    for (int sg = 0; sg < NSEG; ++sg) {
        if constexpr (NSEG > 1) load_keys<SEG>(kw, srow, N, p0 + sg * SEG, vec_ok);
#pragma unroll
        for (int j = 0; j < SEG; ++j) {
            const uint32_t key = key_at<SEG>(kw, j);
            if ((key >> kHist2Bits) == T1) atomicAdd(&h2[key & (kHist2Bins - 1)], 1u);
        }
    }
    __syncthreads();
    if (t < 64) {
        // lane l owns level-2 bin 31-l (descending), again an exclusive scan
        const uint32_t c = (t < kHist2Bins) ? h2[kHist2Bins - 1 - t] : 0u;
        const uint32_t incl = wave_inclusive_scan(c);
        const uint32_t ex = incl - c;
        const uint32_t need1 = kk - sh_above1;
        if (t < kHist2Bins && ex < need1 && incl >= need1) {
            sh_T = (T1 << kHist2Bits) | static_cast<uint32_t>(kHist2Bins - 1 - t);
            sh_need = need1 - ex;  // ties at T that are selected
        }
    }
    __syncthreads();
    const uint32_t T = sh_T;
    const uint32_t need = sh_need;

    // --- 3. offsets: one scan of packed (ties << 32 | above) ---------------
    uint32_t gt = 0u, eq = 0u;
    for (int sg = 0; sg < NSEG; ++sg) {
        if constexpr (NSEG > 1) load_keys<SEG>(kw, srow, N, p0 + sg * SEG, vec_ok);
#pragma unroll
        for (int j = 0; j < SEG; ++j) {
            const uint32_t key = key_at<SEG>(kw, j);
            gt += (key > T) ? 1u : 0u;
            eq += (key == T) ? 1u : 0u;
        }
    }
    const unsigned long long packed =
        (static_cast<unsigned long long>(eq) << 32) | static_cast<unsigned long long>(gt);
    const unsigned long long ex = block_exclusive_scan<unsigned long long>(packed, wsum64);
    uint32_t eq_before = static_cast<uint32_t>(ex >> 32);
    const uint32_t gt_before = static_cast<uint32_t>(ex & 0xffffffffull);
    uint32_t pos = gt_before + (eq_before < need ? eq_before : need);

    // --- 4. emit in position order ------------------------------------------
    int32_t* out = idx + row * static_cast<size_t>(k);
    if (gt != 0u || (eq != 0u && eq_before < need)) {
        for (int sg = 0; sg < NSEG; ++sg) {
            if constexpr (NSEG > 1) load_keys<SEG>(kw, srow, N, p0 + sg * SEG, vec_ok);
#pragma unroll
            for (int j = 0; j < SEG; ++j) {
                const uint32_t key = key_at<SEG>(kw, j);
                bool take = key > T;
                if (key == T) {
                    take = eq_before < need;
                    ++eq_before;
                }
                if (take && pos < kk) out[pos++] = p0 + sg * SEG + j;
            }
        }
    }
}

template <int KPT>
hipError_t launch_select_t(const uint16_t* scores, const uint32_t* hist1, int32_t* idx, int rows,
                           int N, int k, hipStream_t s) {
    select_kernel<KPT><<<rows, kSelectThreads, 0, s>>>(scores, hist1, idx, N, k);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_hist(const uint16_t* scores, uint32_t* hist1, int rows, int N, hipStream_t s) {
    const int per_block = 4096;
    const dim3 grid(static_cast<unsigned>((N + per_block - 1) / per_block), static_cast<unsigned>(rows));
    hist_kernel<<<grid, 256, 0, s>>>(scores, hist1, N, per_block);
    return hipGetLastError();
}

hipError_t launch_select(const uint16_t* scores, const uint32_t* hist1, int32_t* idx, int rows,
                         int N, int k, hipStream_t s) {
    const int kpt_min = (N + kSelectThreads - 1) / kSelectThreads;
    if (kpt_min <= 8) return launch_select_t<8>(scores, hist1, idx, rows, N, k, s);
    if (kpt_min <= 16) return launch_select_t<16>(scores, hist1, idx, rows, N, k, s);
    if (kpt_min <= 32) return launch_select_t<32>(scores, hist1, idx, rows, N, k, s);
    if (kpt_min <= 64) return launch_select_t<64>(scores, hist1, idx, rows, N, k, s);
    if (kpt_min <= 128) return launch_select_t<128>(scores, hist1, idx, rows, N, k, s);
    return hipErrorInvalidValue;
}

}  // namespace dcr
