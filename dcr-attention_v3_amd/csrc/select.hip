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
//   1. level-1 histogram of key >> 8 (256 bins: sign and the top 7 exponent
//      bits), as slabs of partial histograms -- produced by the score kernel
//      (fused, one slab per score workgroup) or by hist_kernel;
//   2. one workgroup of 1024 threads per row; it sums the row's slabs, and
//      wave 0 scans the histogram from the top and finds the bin T1 holding
//      the k-th largest key;
//   3. the row's keys are loaded once (each thread owns a contiguous run of
//      KPT positions); a 256-bin level-2 histogram of the keys inside T1
//      gives the exact threshold key T and the number of ties at T that are
//      selected (need = k - #{key > T});
//   4. one block-wide exclusive scan of the (ties, above) counts gives every
//      thread its output offset and how many ties precede it; threads emit
//      key > T, and key == T while the tie quota lasts, in position order --
//      the output is ascending with no sort.  Rows with k <= kStageCap are
//      assembled in LDS and copied out with coalesced stores.
// Wave scans use DPP row shifts / row broadcasts (no LDS permutes).
#include <type_traits>

#include "dcr_common.h"
#include "dcr_kernels.h"
#include "dcr_radix.h"

namespace dcr {
namespace {

constexpr int kSelectThreads = 1024;
constexpr int kSelectWaves = kSelectThreads / 64;
constexpr int kStageCap = 16384;  // output indices staged in LDS (64 KiB)

// Exclusive prefix sums of two counters over the threads of the block (up to
// 1024, a whole number of waves), in thread order.
__device__ __forceinline__ void block_exclusive_scan2(uint32_t a, uint32_t b, uint32_t& ea,
                                                      uint32_t& eb, uint32_t* wsum /*[2*16]*/) {
    const int lane = lane_id();
    const int w = static_cast<int>(threadIdx.x >> 6);
    const uint32_t ia = wave_inclusive_scan(a);
    const uint32_t ib = wave_inclusive_scan(b);
    if (lane == 63) {
        wsum[w] = ia;
        wsum[kSelectWaves + w] = ib;
    }
    __syncthreads();
    if (w == 0) {
        // Row 0 (lanes 0-15) scans the 16 wave totals of a, row 2 (lanes
        // 32-47) those of b; rows 1 and 3 hold zeros.
        const int nw = static_cast<int>(blockDim.x >> 6);
        const uint32_t sa = (lane < nw) ? wsum[lane] : 0u;
        const uint32_t sb = (lane >= 32 && lane < 32 + nw) ? wsum[kSelectWaves + lane - 32] : 0u;
        const uint32_t own = (lane < 32) ? sa : sb;
        const uint32_t s = row16_inclusive_scan(own);
        if (lane < kSelectWaves) wsum[lane] = s - own;
        if (lane >= 32 && lane < 32 + kSelectWaves) wsum[kSelectWaves + lane - 32] = s - own;
    }
    __syncthreads();
    ea = wsum[w] + ia - a;
    eb = wsum[kSelectWaves + w] + ib - b;
}

constexpr int kHistSlabRows = 4096;  // positions per hist_kernel slab

// Level-1 histogram of a slice of one score row, written as that slice's slab
// (all 256 bins; nothing needs clearing beforehand).
__global__ __launch_bounds__(256) void hist_kernel(const uint16_t* __restrict__ scores,
                                                   slab_t* __restrict__ hist1, int N,
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
    slab_t* hg = hist1 + (row * gridDim.x + blockIdx.x) * kHist1Bins;
    for (int i = static_cast<int>(threadIdx.x); i < kHist1Bins; i += 256) hg[i] = static_cast<slab_t>(h[i]);
}

// Keys of positions [p, p + SEG) as packed 16-bit pairs; positions >= N get
// key 0, below every real key (real keys are >= 0x007F).  KEYS: the row
// holds order-preserving keys already, padded with key 0 up to the row
// stride (the fused score pass stores them so; the caller passes the stride
// as N), so whole 16-byte groups are loaded or zeroed; otherwise bf16 score
// bits, converted here.  vec_ok: the row is 16-byte aligned.
template <int SEG, bool KEYS>
__device__ __forceinline__ void load_keys(uint32_t (&kw)[SEG / 2], const uint16_t* __restrict__ srow,
                                          int N, int p, bool vec_ok) {
    if constexpr (KEYS) {
#pragma unroll
        for (int v = 0; v < SEG / 8; ++v) {
            const int q = p + v * 8;
            chunk_t c = {0u, 0u, 0u, 0u};
            if (q < N) c = *reinterpret_cast<const chunk_t*>(srow + q);
#pragma unroll
            for (int j = 0; j < 4; ++j) kw[v * 4 + j] = c[j];
        }
        return;
    }
#pragma unroll
    for (int v = 0; v < SEG / 8; ++v) {
        const int q = p + v * 8;
        if (vec_ok && q + 8 <= N) {
            const chunk_t c = *reinterpret_cast<const chunk_t*>(srow + q);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                kw[v * 4 + j] = KEYS ? c[j] : (bf16_key(c[j] & 0xffffu) | (bf16_key(c[j] >> 16) << 16));
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = (q + 2 * j < N) ? (KEYS ? srow[q + 2 * j] : bf16_key(srow[q + 2 * j])) : 0u;
                const uint32_t hi =
                    (q + 2 * j + 1 < N) ? (KEYS ? srow[q + 2 * j + 1] : bf16_key(srow[q + 2 * j + 1])) : 0u;
                kw[v * 4 + j] = lo | (hi << 16);
            }
        }
    }
}

template <int SEG>
__device__ __forceinline__ uint32_t key_at(const uint32_t (&kw)[SEG / 2], int j) {
    return (kw[j >> 1] >> ((j & 1) * 16)) & 0xffffu;
}

// Bit masks of the SEG keys of a segment: 32-bit up to 32 keys (no dead
// upper-half work), 64-bit up to 64.
template <int SEG>
using kmask = typename std::conditional<(SEG <= 32), uint32_t, uint64_t>::type;

__device__ __forceinline__ int mask_ctz(uint32_t m) { return __builtin_ctz(m); }
__device__ __forceinline__ int mask_ctz(uint64_t m) { return __builtin_ctzll(m); }
__device__ __forceinline__ uint32_t mask_popc(uint32_t m) { return __builtin_popcount(m); }
__device__ __forceinline__ uint32_t mask_popc(uint64_t m) { return __builtin_popcountll(m); }

// Bit j set for each of the SEG keys with key > T (gt) or key == T (eq).
template <int SEG>
__device__ __forceinline__ void key_masks(const uint32_t (&kw)[SEG / 2], uint32_t T, kmask<SEG>& gtm,
                                          kmask<SEG>& eqm) {
    using kmask_t = kmask<SEG>;
    static_assert(SEG <= 64, "one mask bit per key");
    gtm = 0u;
    eqm = 0u;
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
        const uint32_t key = key_at<SEG>(kw, j);
        gtm |= static_cast<kmask_t>(key > T ? 1u : 0u) << j;
        eqm |= static_cast<kmask_t>(key == T ? 1u : 0u) << j;
    }
}

// Index of the r-th lowest set bit of m (1 <= r <= popcount(m)).
template <typename kmask_t>
__device__ __forceinline__ int nth_bit(kmask_t m, uint32_t r) {
    for (uint32_t i = 1; i < r; ++i) m &= m - 1u;
    return mask_ctz(m);
}

// The n lowest set bits of m.
template <typename kmask_t>
__device__ __forceinline__ kmask_t lowest_bits(kmask_t m, uint32_t n) {
    kmask_t r = 0u;
    for (uint32_t i = 0; i < n && m != 0u; ++i) {
        const kmask_t b = m & (0u - m);
        r |= b;
        m ^= b;
    }
    return r;
}

// One workgroup per row (SPLIT = 1), or two (SPLIT = 2: blockIdx.y = h, for
// rows too few to fill the device); thread t owns positions [t*KPT, (t+1)*KPT), walked
// in segments of SEG <= 64 keys.  KPT is N/1024 rounded up to a multiple of 8
// (or to 96 / 128) and the workgroup has just enough waves to cover the row,
// so no wave runs the passes over padding.  With a single segment the keys stay in
// registers across the passes; otherwise each pass re-reads them (from L2).
// Per segment the comparisons against T are folded into two 32-bit masks, so
// the emission loop runs once per selected key, not once per key.
// SPLIT = 2: both workgroups of a row load all its keys and build its level-2
// histogram (the first half's threads into a histogram of their own), so both
// find T and know how many keys the first half selects; workgroup h then runs
// the mask, scan and emission passes over half h of the row only (the threads
// of the other half idle), at that half's output offset and tie quota.  The
// passes that dominate the kernel (VALU bound) so run on twice the CUs.
template <int KPT, bool KEYS, int SPLIT>
__global__ __launch_bounds__(kSelectThreads) void select_kernel(const uint16_t* __restrict__ scores,
                                                                const slab_t* __restrict__ hist1,
                                                                int nslab,
                                                                int32_t* __restrict__ idx,
                                                                uint32_t* __restrict__ sel,
                                                                uint32_t* __restrict__ ticket,
                                                                int n_rep, int N, int ldsc, int k) {
    constexpr int SEG = KPT <= 64 ? KPT : KPT / 2;  // keys per segment (held in registers)
    constexpr int NSEG = KPT / SEG;
    static_assert(SEG % 8 == 0 && KPT % SEG == 0, "keys are loaded in chunks of 8");
    static_assert(kHist1Bins == 256 && kHist2Bins == 256, "find_bin_regs scans 256 bins");
    __shared__ uint32_t wsum[2 * kSelectWaves];
    __shared__ uint32_t h1[kHist1Bins];
    __shared__ uint32_t h2[kHist2Bins];
    __shared__ uint32_t h2a[SPLIT == 2 ? kHist2Bins : 1];  // first half's level 2 (SPLIT)
    __shared__ uint32_t sh_T1, sh_above1, sh_T2, sh_above2;
    __shared__ uint32_t sh_gt1a, sh_above2a, sh_eqa;  // first half: above T1, above T, at T (SPLIT)
    __shared__ int32_t stage[kStageCap];

    const int t = static_cast<int>(threadIdx.x);
    const size_t row = xcd_order(blockIdx.x, gridDim.x);  // rows of a group on one XCD
    const uint16_t* srow = scores + row * static_cast<size_t>(ldsc);
    const uint32_t kk = static_cast<uint32_t>(k);
    const int p0 = t * KPT;
    const bool vec_ok = (ldsc % 8) == 0 && (reinterpret_cast<uintptr_t>(scores) & 15u) == 0;
    static_assert(SPLIT == 1 || SPLIT == 2, "one or two workgroups per row");
    const int hsel = SPLIT == 2 ? static_cast<int>(blockIdx.y) : 0;
    const int half_threads = static_cast<int>(blockDim.x) / SPLIT;  // a multiple of 64 (host)
    const bool first_half = SPLIT == 2 && t < half_threads;
    const bool mine = SPLIT == 1 || (t / half_threads) == hsel;      // wave-uniform

    // Thread t sums bins t, t + nthreads, ... over the row's slabs; the slab
    // loads are issued before the key loads, so the sums do not wait behind
    // them (loads complete in issue order).
    const int nthreads = static_cast<int>(blockDim.x);
    uint32_t hsum[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int bin = t + i * nthreads;
        if (bin >= kHist1Bins) break;
        const slab_t* hrow = hist1 + row * static_cast<size_t>(nslab) * kHist1Bins + bin;
        // Sixteen independent loads per round, so one round trip covers them.
        for (int x0 = 0; x0 < nslab; x0 += 16) {
            uint32_t v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j)
                v[j] = (x0 + j < nslab) ? hrow[static_cast<size_t>(x0 + j) * kHist1Bins] : 0u;
#pragma unroll
            for (int j = 0; j < 16; ++j) hsum[i] += v[j];
        }
    }
    uint32_t kw[SEG / 2];
    if constexpr (NSEG == 1) load_keys<SEG, KEYS>(kw, srow, KEYS ? ldsc : N, p0, vec_ok);

    // --- 1. level-1 bin T1 holding the k-th largest key (wave 0) -----------
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int bin = t + i * nthreads;
        if (bin >= kHist1Bins) break;
        h1[bin] = hsum[i];
        h2[bin] = 0u;
        if constexpr (SPLIT == 2) h2a[bin] = 0u;
    }
    if (t == 0) {  // defaults if the histogram were inconsistent (then fewer than k are written)
        const uint32_t r32 = static_cast<uint32_t>(row);
        if (ticket != nullptr && hsel == 0 && r32 % static_cast<uint32_t>(n_rep) == 0u)
            ticket[r32 / static_cast<uint32_t>(n_rep)] = 0u;
        sh_T1 = 0u;
        sh_above1 = 0u;
        sh_T2 = 0u;
        sh_above2 = 0u;
        sh_gt1a = 0u;
        sh_above2a = 0u;
        sh_eqa = 0u;
    }
    __syncthreads();
    if (t < 64) {
        uint32_t c1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c1[i] = h1[255 - 4 * t - i];
        find_bin_regs(c1, kk, &sh_T1, &sh_above1);
    }
    __syncthreads();

    // --- 2. level-2 histogram inside T1, exact threshold T ------------------
    const uint32_t T1 = sh_T1;
    uint32_t* h2mine = first_half ? h2a : h2;
    uint32_t gt1 = 0u;  // SPLIT: this thread's keys above bin T1
    for (int sg = 0; sg < NSEG; ++sg) {
        if constexpr (NSEG > 1) load_keys<SEG, KEYS>(kw, srow, KEYS ? ldsc : N, p0 + sg * SEG, vec_ok);
#pragma unroll
        for (int j = 0; j < SEG; ++j) {
            const uint32_t key = key_at<SEG>(kw, j);
            if ((key >> kHist2Bits) == T1) atomicAdd(&h2mine[key & (kHist2Bins - 1)], 1u);
            if constexpr (SPLIT == 2) gt1 += (key >> kHist2Bits) > T1 ? 1u : 0u;
        }
    }
    if constexpr (SPLIT == 2) {
        if (first_half) {
            const uint32_t w = wave_inclusive_scan(gt1);
            if ((t & 63) == 63) atomicAdd(&sh_gt1a, w);
        }
    }
    __syncthreads();
    if (t < 64) {
        // T's level-2 bin from both halves' counts; with SPLIT also the first
        // half's keys above T and at T.
        uint32_t c2[4], c2a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c2a[i] = SPLIT == 2 ? h2a[255 - 4 * t - i] : 0u;
            c2[i] = h2[255 - 4 * t - i] + c2a[i];
        }
        const uint32_t need2 = kk - sh_above1;
        const uint32_t sum = c2[0] + c2[1] + c2[2] + c2[3];
        const uint32_t suma = c2a[0] + c2a[1] + c2a[2] + c2a[3];
        uint32_t above = wave_inclusive_scan(sum) - sum;
        uint32_t abovea = wave_inclusive_scan(suma) - suma;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (above < need2 && above + c2[i] >= need2) {
                sh_T2 = static_cast<uint32_t>(255 - 4 * t - i);
                sh_above2 = above;
                sh_above2a = abovea;
                sh_eqa = c2a[i];
            }
            above += c2[i];
            abovea += c2a[i];
        }
    }
    __syncthreads();
    const uint32_t T = (T1 << kHist2Bits) | sh_T2;
    const uint32_t need = kk - sh_above1 - sh_above2;  // ties at T that are selected
    // This workgroup's half: where its output starts and its share of the ties.
    uint32_t base = 0u, quota = need, count = kk;
    if constexpr (SPLIT == 2) {
        const uint32_t eq_first = sh_eqa < need ? sh_eqa : need;
        const uint32_t count_first = sh_gt1a + sh_above2a + eq_first;
        base = hsel == 0 ? 0u : count_first;
        quota = hsel == 0 ? need : need - eq_first;
        count = hsel == 0 ? count_first : kk - count_first;
    }

    // --- 3. offsets: one scan of the (ties, above) counts --------------------
    using kmask_t = kmask<SEG>;
    kmask_t gtm = 0u, eqm = 0u;
    uint32_t gt = 0u, eq = 0u;
    if (mine) {
        for (int sg = 0; sg < NSEG; ++sg) {
            if constexpr (NSEG > 1) load_keys<SEG, KEYS>(kw, srow, KEYS ? ldsc : N, p0 + sg * SEG, vec_ok);
            key_masks<SEG>(kw, T, gtm, eqm);
            gt += mask_popc(gtm);
            eq += mask_popc(eqm);
        }
    }
    uint32_t eq_before, gt_before;
    block_exclusive_scan2(eq, gt, eq_before, gt_before, wsum);
    uint32_t pos = base + gt_before + (eq_before < quota ? eq_before : quota);

    // --- the selection as (T, position of the last selected tie) ------------
    if (sel != nullptr) {
        if (t == 0 && hsel == 0) sel[2 * row] = T;
        if (eq_before < quota && quota <= eq_before + eq) {  // this thread holds the need-th tie
            uint32_t r = quota - eq_before;
            for (int sg = 0; sg < NSEG; ++sg) {
                if constexpr (NSEG > 1) {
                    load_keys<SEG, KEYS>(kw, srow, KEYS ? ldsc : N, p0 + sg * SEG, vec_ok);
                    key_masks<SEG>(kw, T, gtm, eqm);
                }
                const uint32_t ne = mask_popc(eqm);
                if (r <= ne) {
                    sel[2 * row + 1] = static_cast<uint32_t>(p0 + sg * SEG + nth_bit(eqm, r));
                    break;
                }
                r -= ne;
            }
        }
    }
    if (idx == nullptr) return;  // uniform over the block

    // --- 4. emit in position order ------------------------------------------
    const bool staged = k <= kStageCap;
    int32_t* out = idx + row * static_cast<size_t>(k);
    uint32_t ties_left = eq_before < quota ? quota - eq_before : 0u;  // this thread's tie quota
    if (gt != 0u || (eq != 0u && ties_left != 0u)) {
        for (int sg = 0; sg < NSEG; ++sg) {
            if constexpr (NSEG > 1) {
                load_keys<SEG, KEYS>(kw, srow, KEYS ? ldsc : N, p0 + sg * SEG, vec_ok);
                key_masks<SEG>(kw, T, gtm, eqm);
            }
            const uint32_t ne = mask_popc(eqm);
            kmask_t take = gtm | (ties_left >= ne ? eqm : lowest_bits(eqm, ties_left));
            ties_left -= (ties_left >= ne ? ne : ties_left);
            const int pbase = p0 + sg * SEG;
            while (take != 0u && pos < kk) {
                const int j = mask_ctz(take);
                take &= take - 1u;
                if (staged)
                    stage[pos - base] = pbase + j;
                else
                    out[pos] = pbase + j;
                ++pos;
            }
        }
    }
    if (staged) {
        __syncthreads();
        for (int i = t; i < static_cast<int>(count); i += nthreads) out[base + i] = stage[i];
    }
}

// ---------------------------------------------------------------------------
// Chunked form for rows too few to fill the device (e.g. B = 1 at N = 128K:
// 32 rows): each row is cut into nchunk chunks of 1024 * KPT positions, one
// workgroup per (row, chunk), in two launches.
//   pass 1 (select_chunk_hist_kernel): every workgroup finds the row's
//     level-1 bin T1 from the slabs, and writes the level-2 histogram of its
//     chunk's keys inside T1 plus the count of its keys above T1
//     (part[row][chunk][0..255], [256]); chunk 0 also writes (T1, above1).
//   pass 2 (select_chunk_emit_kernel): every workgroup sums the row's
//     level-2 histograms to the exact threshold T and tie quota, takes the
//     (above, ties) counts of the chunks before its own from the same partial
//     histograms, and emits its chunk's selected positions at that offset --
//     the same output as the one-workgroup kernel.
constexpr int kPartStride = kHist2Bins + 1;

// Level-1 slab sum spread over the whole 1024-thread block: thread t takes
// bin t % 256 of the slabs x = t / 256, t / 256 + 4, ... (sixteen loads in
// flight per round; one round up to 64 slabs).  slab_first issues the first
// round into v (before the caller's key loads, which then overlap it);
// slab_rest adds the other rounds and returns the partial sum, which the
// caller adds into a zeroed LDS h1 with an atomic.
constexpr int kSlabGroups = kSelectThreads / kHist1Bins;  // 4

__device__ __forceinline__ const slab_t* slab_base(const slab_t* __restrict__ hist1, size_t row,
                                                     int nslab, int t) {
    return hist1 + row * static_cast<size_t>(nslab) * kHist1Bins +
           static_cast<size_t>(t / kHist1Bins) * kHist1Bins + (t % kHist1Bins);
}

__device__ __forceinline__ void slab_first(uint32_t (&v)[16], const slab_t* __restrict__ hist1, size_t row,
                                           int nslab, int t) {
    const slab_t* p = slab_base(hist1, row, nslab, t);
    const int g = t / kHist1Bins;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int x = g + j * kSlabGroups;
        v[j] = x < nslab ? p[static_cast<size_t>(j) * kSlabGroups * kHist1Bins] : 0u;
    }
}

__device__ __forceinline__ uint32_t slab_rest(const uint32_t (&v)[16], const slab_t* __restrict__ hist1,
                                              size_t row, int nslab, int t) {
    uint32_t acc = 0u;
#pragma unroll
    for (int j = 0; j < 16; ++j) acc += v[j];
    const slab_t* p = slab_base(hist1, row, nslab, t);
    const int g = t / kHist1Bins;
    for (int j0 = 16; g + j0 * kSlabGroups < nslab; j0 += 16) {
        uint32_t w[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int x = g + (j0 + j) * kSlabGroups;
            w[j] = x < nslab ? p[static_cast<size_t>(j0 + j) * kSlabGroups * kHist1Bins] : 0u;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) acc += w[j];
    }
    return acc;
}

template <int KPT, bool KEYS>
__global__ __launch_bounds__(kSelectThreads) void select_chunk_hist_kernel(
    const uint16_t* __restrict__ scores, const slab_t* __restrict__ hist1, int nslab,
    uint32_t* __restrict__ part, uint32_t* __restrict__ rowinfo, int N, int ldsc, int k) {
    static_assert(KPT % 8 == 0 && KPT <= 64, "chunk keys stay in registers");
    __shared__ uint32_t h1[kHist1Bins];
    __shared__ uint32_t h2[kHist2Bins];
    __shared__ uint32_t sh_T1, sh_above1, sh_gt1;
    const int t = static_cast<int>(threadIdx.x);
    const int nthreads = static_cast<int>(blockDim.x);
    const size_t row = blockIdx.x;
    const int c = static_cast<int>(blockIdx.y);
    const int nchunk = static_cast<int>(gridDim.y);
    const uint16_t* srow = scores + row * static_cast<size_t>(ldsc);
    const bool vec_ok = (ldsc % 8) == 0 && (reinterpret_cast<uintptr_t>(scores) & 15u) == 0;

    uint32_t sv[16];
    slab_first(sv, hist1, row, nslab, t);
    uint32_t kw[KPT / 2];
    load_keys<KPT, KEYS>(kw, srow, KEYS ? ldsc : N, c * (kSelectThreads * KPT) + t * KPT, vec_ok);
    for (int b = t; b < kHist2Bins; b += nthreads) {
        h1[b] = 0u;
        h2[b] = 0u;
    }
    if (t == 0) {
        sh_T1 = 0u;
        sh_above1 = 0u;
        sh_gt1 = 0u;
    }
    __syncthreads();
    {
        const uint32_t part = slab_rest(sv, hist1, row, nslab, t);
        if (part != 0u) atomicAdd(&h1[t % kHist1Bins], part);
    }
    __syncthreads();
    if (t < 64) {
        uint32_t c1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c1[i] = h1[255 - 4 * t - i];
        find_bin_regs(c1, static_cast<uint32_t>(k), &sh_T1, &sh_above1);
    }
    __syncthreads();
    const uint32_t T1 = sh_T1;
    uint32_t gt1 = 0u;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const uint32_t key = key_at<KPT>(kw, j);
        const uint32_t b1 = key >> kHist2Bits;
        if (b1 == T1) atomicAdd(&h2[key & (kHist2Bins - 1)], 1u);
        gt1 += (b1 > T1) ? 1u : 0u;
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) gt1 += __shfl_xor(gt1, off, 64);
    if ((t & 63) == 0 && gt1 != 0u) atomicAdd(&sh_gt1, gt1);
    __syncthreads();
    uint32_t* pc = part + (row * nchunk + c) * static_cast<size_t>(kPartStride);
    for (int b = t; b < kHist2Bins; b += nthreads) pc[b] = h2[b];
    if (t == 0) {
        pc[kHist2Bins] = sh_gt1;
        if (c == 0) {
            rowinfo[2 * row] = T1;
            rowinfo[2 * row + 1] = sh_above1;
        }
    }
}

template <int KPT, bool KEYS>
__global__ __launch_bounds__(kSelectThreads) void select_chunk_emit_kernel(
    const uint16_t* __restrict__ scores, const uint32_t* __restrict__ part,
    const uint32_t* __restrict__ rowinfo, int32_t* __restrict__ idx, uint32_t* __restrict__ sel,
    uint32_t* __restrict__ ticket, int n_rep, int N, int ldsc, int k) {
    static_assert(KPT % 8 == 0 && KPT <= 64, "chunk keys stay in registers");
    constexpr int CHUNK = kSelectThreads * KPT;
    __shared__ uint32_t wsum[2 * kSelectWaves];
    __shared__ uint32_t h2[kHist2Bins];
    __shared__ uint32_t pre2[kHist2Bins];
    __shared__ uint32_t sh_T2, sh_above2, sh_gtc;
    constexpr int STAGE = CHUNK < kStageCap ? CHUNK : kStageCap;
    __shared__ int32_t stage[STAGE];
    const int t = static_cast<int>(threadIdx.x);
    const int nthreads = static_cast<int>(blockDim.x);
    const size_t row = blockIdx.x;
    const int c = static_cast<int>(blockIdx.y);
    const int nchunk = static_cast<int>(gridDim.y);
    const uint16_t* srow = scores + row * static_cast<size_t>(ldsc);
    const bool vec_ok = (ldsc % 8) == 0 && (reinterpret_cast<uintptr_t>(scores) & 15u) == 0;
    const uint32_t kk = static_cast<uint32_t>(k);
    const int p0 = c * CHUNK + t * KPT;

    // Totals over all chunks and prefix over the chunks before this one.
    const uint32_t* prow = part + row * nchunk * static_cast<size_t>(kPartStride);
    for (int b = t; b <= kHist2Bins; b += nthreads) {
        uint32_t tot = 0u, pre = 0u;
        for (int x = 0; x < nchunk; ++x) {
            const uint32_t v = prow[static_cast<size_t>(x) * kPartStride + b];
            tot += v;
            pre += (x < c) ? v : 0u;
        }
        if (b < kHist2Bins) {
            h2[b] = tot;
            pre2[b] = pre;
        } else {
            sh_gtc = pre;  // keys above T1 in earlier chunks
        }
    }
    uint32_t kw[KPT / 2];
    load_keys<KPT, KEYS>(kw, srow, KEYS ? ldsc : N, p0, vec_ok);
    const uint32_t T1 = rowinfo[2 * row];
    const uint32_t above1 = rowinfo[2 * row + 1];
    if (t == 0) {
        const uint32_t r32 = static_cast<uint32_t>(row);
        if (c == 0 && ticket != nullptr && r32 % static_cast<uint32_t>(n_rep) == 0u)
            ticket[r32 / static_cast<uint32_t>(n_rep)] = 0u;
        sh_T2 = 0u;
        sh_above2 = 0u;
    }
    __syncthreads();
    if (t < 64) {
        uint32_t c2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c2[i] = h2[255 - 4 * t - i];
        find_bin_regs(c2, kk - above1, &sh_T2, &sh_above2);
    }
    __syncthreads();
    const uint32_t T2 = sh_T2;
    const uint32_t T = (T1 << kHist2Bits) | T2;
    const uint32_t need = kk - above1 - sh_above2;

    // (above, ties) counts of the earlier chunks.
    uint32_t gpart = 0u;
    for (int b = t; b < kHist2Bins; b += nthreads) gpart += (static_cast<uint32_t>(b) > T2) ? pre2[b] : 0u;
    using kmask_t = kmask<KPT>;
    kmask_t gtm, eqm;
    key_masks<KPT>(kw, T, gtm, eqm);
    const uint32_t gt = mask_popc(gtm), eq = mask_popc(eqm);
    uint32_t eq_before, gt_before;
    block_exclusive_scan2(eq, gt, eq_before, gt_before, wsum);
    // Block sum of gpart (wsum is free again after the scan's final read).
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) gpart += __shfl_xor(gpart, off, 64);
    __syncthreads();
    if ((t & 63) == 0) wsum[t >> 6] = gpart;
    __syncthreads();
    uint32_t gt_chunk = sh_gtc;
    for (int w = 0; w < (nthreads >> 6); ++w) gt_chunk += wsum[w];
    const uint32_t eq_chunk = pre2[T2];

    const uint32_t gtb = gt_chunk + gt_before;
    const uint32_t eqb = eq_chunk + eq_before;
    if (sel != nullptr) {
        if (c == 0 && t == 0) sel[2 * row] = T;
        if (eqb < need && need <= eqb + eq)  // this thread holds the need-th tie of the row
            sel[2 * row + 1] = static_cast<uint32_t>(p0 + nth_bit(eqm, need - eqb));
    }
    if (idx == nullptr) return;  // uniform over the block
    uint32_t pos = gtb + (eqb < need ? eqb : need);
    const uint32_t pos0 = gt_chunk + (eq_chunk < need ? eq_chunk : need);  // chunk's first slot
    uint32_t ties_left = eqb < need ? need - eqb : 0u;
    int32_t* out = idx + row * static_cast<size_t>(k);
    const uint32_t ne = eq;
    kmask_t take = gtm | (ties_left >= ne ? eqm : lowest_bits(eqm, ties_left));
    while (take != 0u && pos < kk) {
        const int j = mask_ctz(take);
        take &= take - 1u;
        if (CHUNK <= kStageCap)
            stage[pos - pos0] = p0 + j;
        else
            out[pos] = p0 + j;
        ++pos;
    }
    if (CHUNK <= kStageCap) {
        // The chunk's slots end where the next thread's would begin: the
        // last thread's final pos (clamped to k).
        __shared__ uint32_t sh_end;
        if (t == nthreads - 1) sh_end = pos;
        __syncthreads();
        const uint32_t cnt = sh_end - pos0;
        for (uint32_t i = t; i < cnt; i += nthreads) out[pos0 + i] = stage[i];
    }
}

template <int KPT, bool KEYS>
hipError_t launch_select_t(const uint16_t* scores, int ldsc, const slab_t* hist1, int nslab,
                           int32_t* idx, uint32_t* sel, uint32_t* ticket, int n_rep, int rows, int N,
                           int k, hipStream_t s) {
    // Just enough whole waves to cover the row at KPT keys per thread.
    int threads = (N + KPT - 1) / KPT;
    threads = (threads + 63) / 64 * 64;
    // Two workgroups per row when the rows fill at most half the device and
    // the row's keys stay in registers; each half is a whole number of waves
    // (threads rounded up to 128: positions past the row read as key 0).
    if (KPT <= 64 && rows <= 128) {
        const int threads2 = (threads + 127) / 128 * 128;
        launch_kernel(select_kernel<KPT, KEYS, 2>, dim3(rows, 2), dim3(threads2), 0, s, scores, hist1, nslab,
                      idx, sel, ticket, n_rep, N, ldsc, k);
        return hipGetLastError();
    }
    launch_kernel(select_kernel<KPT, KEYS, 1>, dim3(rows), dim3(threads), 0, s, scores, hist1, nslab,
                  idx, sel, ticket, n_rep, N, ldsc, k);
    return hipGetLastError();
}

}  // namespace

int hist_slabs(int N) { return (N + kHistSlabRows - 1) / kHistSlabRows; }

hipError_t launch_hist(const uint16_t* scores, slab_t* hist1, int rows, int N, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(hist_slabs(N)), static_cast<unsigned>(rows));
    launch_kernel(hist_kernel, grid, dim3(256), 0, s, scores, hist1, N, kHistSlabRows);
    return hipGetLastError();
}

// Chunks per row for the two-launch form (1 = one workgroup per row): used
// when the rows alone would fill less than half the device.
int select_chunks(int rows, int N, int* kpt_out) {
    int kpt = 32;
    // One workgroup per row when that fills the device or the row is short,
    // and the row fits one workgroup's registers (kMaxSelectN).
    if ((rows >= 128 || N <= 2 * kSelectThreads * 8) && N <= kMaxSelectN) return (*kpt_out = 0, 1);
    const int want = (256 + rows - 1) / rows;  // chunks per row to reach ~256 workgroups
    const int per = (N + want - 1) / want;     // positions per chunk
    kpt = (per + kSelectThreads - 1) / kSelectThreads;
    kpt = kpt <= 8 ? 8 : (kpt <= 16 ? 16 : (kpt <= 32 ? 32 : 64));
    *kpt_out = kpt;
    return (N + kSelectThreads * kpt - 1) / (kSelectThreads * kpt);
}

size_t select_part_words(int rows, int N) {
    int kpt = 0;
    const int nchunk = select_chunks(rows, N, &kpt);
    if (nchunk <= 1) return 0;
    return static_cast<size_t>(rows) * nchunk * kPartStride + 2 * static_cast<size_t>(rows);
}

template <bool KEYS>
hipError_t launch_select_v(const uint16_t* scores, int ldsc, const slab_t* hist1, int nslab,
                           int32_t* idx, uint32_t* sel, uint32_t* ticket, int n_rep, int rows, int N,
                           int k, uint32_t* part, hipStream_t s) {
    int ckpt = 0;
    const int nchunk = select_chunks(rows, N, &ckpt);
    if (nchunk > 1) {
        uint32_t* rowinfo = part + static_cast<size_t>(rows) * nchunk * kPartStride;
        const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>(nchunk));
#define DCR_CHUNK_CASE(KPT)                                                                      \
        if (ckpt == KPT) {                                                                       \
            launch_kernel(select_chunk_hist_kernel<KPT, KEYS>, grid, dim3(kSelectThreads), 0, s,  \
                          scores, hist1, nslab, part, rowinfo, N, ldsc, k);                      \
            hipError_t e = hipGetLastError();                                                    \
            if (e != hipSuccess) return e;                                                       \
            launch_kernel(select_chunk_emit_kernel<KPT, KEYS>, grid, dim3(kSelectThreads), 0, s,  \
                          scores, part, rowinfo, idx, sel, ticket, n_rep, N, ldsc, k);           \
            return hipGetLastError();                                                            \
        }
        DCR_CHUNK_CASE(8)
        DCR_CHUNK_CASE(16)
        DCR_CHUNK_CASE(32)
        DCR_CHUNK_CASE(64)
#undef DCR_CHUNK_CASE
        return hipErrorInvalidValue;
    }
    const int kpt_min = (N + kSelectThreads - 1) / kSelectThreads;
#define DCR_SELECT_CASE(KPT)                                                                    \
    if (kpt_min <= KPT)                                                                         \
        return launch_select_t<KPT, KEYS>(scores, ldsc, hist1, nslab, idx, sel, ticket, n_rep, rows, \
                                          N, k, s);
    DCR_SELECT_CASE(8)
    DCR_SELECT_CASE(16)
    DCR_SELECT_CASE(24)
    DCR_SELECT_CASE(32)
    DCR_SELECT_CASE(40)
    DCR_SELECT_CASE(48)
    DCR_SELECT_CASE(64)
    DCR_SELECT_CASE(96)
    DCR_SELECT_CASE(128)
#undef DCR_SELECT_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_select(const uint16_t* scores, int ldsc, const slab_t* hist1, int nslab,
                         int32_t* idx, uint32_t* ticket, int n_rep, int rows, int N, int k,
                         uint32_t* part, hipStream_t s) {
    return launch_select_v<false>(scores, ldsc, hist1, nslab, idx, nullptr, ticket, n_rep, rows, N, k,
                                  part, s);
}

hipError_t launch_select_keys(const uint16_t* keys, int ldsc, const slab_t* hist1, int nslab,
                              int32_t* idx, uint32_t* sel, uint32_t* ticket, int n_rep, int rows,
                              int N, int k, uint32_t* part, hipStream_t s) {
    return launch_select_v<true>(keys, ldsc, hist1, nslab, idx, sel, ticket, n_rep, rows, N, k, part, s);
}

}  // namespace dcr
