// dcr_common.h -- device helpers shared by the sparse decode kernels (gfx950).
//
// Numeric contract (reference kernel_spec.md section 3; M1 oracle
// qaxis_topk_reference.py:42-259):
//   * Q and K are promoted to fp32 once; the projection accumulates in fp32
//     and is rounded to bf16 (round-to-nearest-even) as the top-K key.
//   * Attention logits and the softmax state m/l/o stay fp32; the output is
//     rounded once to the input dtype.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dcr {

enum Dtype : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// One 16-byte chunk as a native vector (HIP's uint4 class wrapper keeps
// arrays of chunks from being promoted to registers).
typedef uint32_t chunk_t __attribute__((ext_vector_type(4)));

template <int DT>
struct ElemBytes {
    static constexpr int value = (DT == kF32) ? 4 : 2;
};

// Element e (0 <= e < 16 / bytes) of a 16-byte chunk, widened to fp32.
// fp16/bf16 -> fp32 is exact.
template <int DT>
__device__ __forceinline__ float chunk_elem(const chunk_t& c, int e) {
    if constexpr (DT == kF32) {
        return __uint_as_float(c[e]);
    } else if constexpr (DT == kF16) {
        const uint32_t word = c[e >> 1];
        const uint16_t bits = (e & 1) ? static_cast<uint16_t>(word >> 16)
                                      : static_cast<uint16_t>(word & 0xffffu);
        return static_cast<float>(__builtin_bit_cast(_Float16, bits));
    } else {
        const uint32_t word = c[e >> 1];
        return (e & 1) ? __uint_as_float(word & 0xffff0000u) : __uint_as_float(word << 16);
    }
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, size_t i) {
    if constexpr (DT == kF32) {
        return static_cast<const float*>(p)[i];
    } else if constexpr (DT == kF16) {
        const uint16_t bits = static_cast<const uint16_t*>(p)[i];
        return static_cast<float>(__builtin_bit_cast(_Float16, bits));
    } else {
        return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
    }
}

// fp32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// Order-preserving 16-bit key of a bf16 score: a larger score gives a larger
// key, -0 and +0 share a key, every NaN maps to the top key (torch's sort
// puts NaN above +inf).  Real (non-NaN) keys are >= 0x007F.
__device__ __forceinline__ uint32_t bf16_key(uint32_t s) {
    const uint32_t mag = s & 0x7fffu;
    if (mag > 0x7f80u) return 0xffffu;
    if (mag == 0u) return 0x8000u;
    return (s & 0x8000u) ? (~s & 0xffffu) : (s | 0x8000u);
}

// Softmax in base 2: the attention kernels scale their logits by log2(e)
// (folded into the 1/sqrt(D) factor), so e^(s - m) = 2^(s' - m') and every
// exponential is one hardware exp2 (v_exp_f32), the partials' m included.
constexpr double kLog2e = 1.4426950408889634;
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Round fp32 to the output dtype and store element i.
template <int DT>
__device__ __forceinline__ void store_out(void* p, size_t i, float v) {
    if constexpr (DT == kF32) {
        static_cast<float*>(p)[i] = v;
    } else if constexpr (DT == kF16) {
        const _Float16 h = static_cast<_Float16>(v);  // IEEE RNE conversion
        static_cast<uint16_t*>(p)[i] = __builtin_bit_cast(uint16_t, h);
    } else {
        static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_bf16_bits(v));
    }
}

// The fp16/bf16 fused path keeps, beside each score's 16-bit key, one byte
// from which the attention rebuilds the fp32 dot product it uses as a logit:
// the residual of the fp32 value v over its bf16 rounding sb, in fp32 bit
// space, r = round((bits(v) - (sb << 16)) / 256) clamped to [-127, 127].
// fp32 bit patterns of one sign are monotonic in magnitude across binades, so
// (sb << 16) + 256 r is v to within 256 fp32 ulps (128 unless v lies on a
// bf16 rounding tie): 2^-15 relative at worst.  NaN and inf come back as NaN
// and inf; -0 and +0 share a key, so a value that rounds to a bf16 zero comes
// back as a non-negative number below 2^-126 (absolute error below 2^-125).
__device__ __forceinline__ uint32_t score_residual(float v, uint32_t sb) {
    const int32_t d = static_cast<int32_t>(__float_as_uint(v) - (sb << 16));
    int32_t r = (d + 128) >> 8;
    r = r > 127 ? 127 : (r < -127 ? -127 : r);
    return static_cast<uint32_t>(r) & 0xffu;
}

// The logit source of one selected position from its score key (bf16_key of
// sb) and residual byte: the inverse of bf16_key, then the residual added in
// bit space.
__device__ __forceinline__ float score_from_key(uint32_t key, uint32_t r8) {
    const uint32_t sb = key >= 0x8000u ? (key & 0x7fffu) : (~key & 0xffffu);
    const int32_t r = static_cast<int32_t>(r8 << 24) >> 24;
    return __uint_as_float((sb << 16) + static_cast<uint32_t>(r * 256));
}

// float <-> unsigned int preserving order (an integer max in LDS); every
// non-NaN float maps above 0, which is left free to mean "no value".
__device__ __forceinline__ uint32_t ordered_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_ordered(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// Histogram geometry for the radix select: level 1 uses the top 8 bits of
// the 16-bit key (sign and exponent: one bin per binade), level 2 the low 8.
constexpr int kHist1Bits = 8;
constexpr int kHist1Bins = 1 << kHist1Bits;  // 256
constexpr int kHist2Bits = 16 - kHist1Bits;
constexpr int kHist2Bins = 1 << kHist2Bits;  // 256

// One counter of a level-1 histogram slab.  A slab counts the positions of one
// score row that one workgroup covered: at most 4096 (hist_kernel's slice, or
// a score workgroup's block plus its share of the tail, under 2 x 4 waves x 8
// rounds x 64 rows), so 16 bits hold every count and halve the slab traffic.
using slab_t = uint16_t;

// Largest N the one-workgroup-per-row select kernel handles (1024 threads x
// 128 keys per thread; Llama-3.2-1B's max_position_embeddings is 131072).
// Longer rows take the chunked select.
constexpr int kMaxSelectN = 131072;
// Largest N of the top-K path (positions and per-row offsets stay int32).
constexpr int kMaxTopkN = 1 << 24;

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & 63u); }

// MI355X deals the workgroups of a launch to its 8 XCDs (each with its own
// L2) round robin by linear workgroup id.  xcd_order(L, T) maps linear id L
// of a T-workgroup grid to a position in the kernel's natural (group-major)
// order such that XCD j runs the contiguous block [j*T/8, (j+1)*T/8); when T
// is a multiple of 8 the score, select and attention launches therefore give
// each (batch, KV head) group to the same XCD, and every kernel reads what
// the previous one wrote from its own L2.  A bijection on [0, T) for any T.
constexpr unsigned kNumXcd = 8;
__device__ __forceinline__ unsigned xcd_order(unsigned L, unsigned T) {
    return (T % kNumXcd == 0) ? (L % kNumXcd) * (T / kNumXcd) + L / kNumXcd : L;
}

// max(||x||_2, eps) for one row x of D elements, computed by one whole wave
// (all 64 lanes call it and get the same value).  Summation order, shared
// with the CPU oracle and torch's CPU vector-norm kernel: eight strided
// accumulators acc[j] = fma(x[8i+j], x[8i+j], acc[j]), then
// acc[0] + ... + acc[7] left to right, norm = sqrt(s) (IEEE), clamped at eps.
// The library is built with -ffp-contract=off and
// -fhip-fp32-correctly-rounded-divide-sqrt, so each operation rounds once.
// D is a compile-time multiple of 8: every lane issues all its loads at once
// (lane l reads x[(l & 7) + 8i]; lanes past 7 repeat lanes 0..7's addresses),
// so the row costs one memory round trip.
template <int DT, int D>
__device__ __forceinline__ float row_norm(const void* __restrict__ X, size_t base, float eps) {
    static_assert(D % 8 == 0, "the strided chains cover D exactly");
    constexpr int PER = D / 8;
    const int l8 = lane_id() & 7;
    float x[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) x[i] = load_elem<DT>(X, base + l8 + 8 * i);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) acc = __builtin_fmaf(x[i], x[i], acc);
    float s = __shfl(acc, 0, 64);
#pragma unroll
    for (int j = 1; j < 8; ++j) s = s + __shfl(acc, j, 64);
    float n = sqrtf(s);
    if (n < eps) n = eps;
    return n;
}

// u = x / max(||x||_2, eps) for one row (one whole wave; lane e writes u[e],
// u[e + 64], ...), with IEEE division.
template <int DT, int D>
__device__ __forceinline__ void unit_row(const void* __restrict__ X, size_t base, float eps,
                                         float* __restrict__ u) {
    constexpr int R = (D + 63) / 64;
    const int lane = lane_id();
    float xv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) xv[r] = (lane + 64 * r < D) ? load_elem<DT>(X, base + lane + 64 * r) : 0.0f;
    const float n = row_norm<DT, D>(X, base, eps);
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (lane + 64 * r < D) u[lane + 64 * r] = xv[r] / n;
}

}  // namespace dcr
