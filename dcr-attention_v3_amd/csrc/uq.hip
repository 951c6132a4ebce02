// uq.hip -- unit query vectors (reference _compute_u_Q,
// dcr_attention/kernel/qaxis_topk_reference.py:42-55) and a zero-fill kernel.
//
// Summation order (shared with the CPU oracle and with torch's CPU
// vector-norm kernel): eight strided accumulators
// acc[j] = fma(x[8i+j], x[8i+j], acc[j]), then acc[0] + ... + acc[7] left to
// right, a scalar tail s = s + x*x for D % 8 != 0, norm = sqrt(s) (IEEE),
// clamped at eps, u = x / norm (IEEE division).  The library is compiled with
// -ffp-contract=off and -fhip-fp32-correctly-rounded-divide-sqrt, so every
// + * / sqrt below rounds once, as written.
#include "dcr_common.h"
#include "dcr_kernels.h"

namespace dcr {
namespace {

// u for one row of runtime length D (any D > 0): the same order as
// unit_row, plus the scalar tail s = s + x*x for D % 8 != 0.
template <int DT>
__device__ __forceinline__ void unit_row_any(const void* __restrict__ X, size_t base, int D,
                                             float eps, float* __restrict__ u) {
    const int lane = lane_id();
    const int D8 = D - D % 8;
    float acc = 0.0f;
    if (lane < 8)
        for (int d = lane; d < D8; d += 8) {
            const float x = load_elem<DT>(X, base + d);
            acc = __builtin_fmaf(x, x, acc);
        }
    float s = __shfl(acc, 0, 64);
    for (int j = 1; j < 8; ++j) s = s + __shfl(acc, j, 64);
    for (int d = D8; d < D; ++d) {  // scalar tail, same order on every lane
        const float x = load_elem<DT>(X, base + d);
        const float sq = x * x;
        s = s + sq;
    }
    float n = sqrtf(s);
    if (n < eps) n = eps;
    for (int e = lane; e < D; e += 64) u[e] = load_elem<DT>(X, base + e) / n;
}

// One wave per row (DC = D as a compile-time constant, or 0 for any D).
// Every thread of the grid also helps clear zero_buf.
template <int DT, int DC>
__global__ __launch_bounds__(256) void uq_kernel(const void* __restrict__ Q, float* __restrict__ u,
                                                 int rows, int D, float eps,
                                                 uint32_t* __restrict__ zero_buf,
                                                 size_t zero_words) {
    const size_t tid = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t nthreads = static_cast<size_t>(gridDim.x) * blockDim.x;
    const size_t row = tid >> 6;

    if (row < static_cast<size_t>(rows)) {
        const size_t base = row * static_cast<size_t>(D);
        if constexpr (DC > 0)
            unit_row<DT, DC>(Q, base, eps, u + base);
        else
            unit_row_any<DT>(Q, base, D, eps, u + base);
    }

    if (zero_buf != nullptr) {
        uint4* z4 = reinterpret_cast<uint4*>(zero_buf);
        const size_t n4 = zero_words / 4;
        for (size_t i = tid; i < n4; i += nthreads) z4[i] = make_uint4(0u, 0u, 0u, 0u);
        for (size_t i = n4 * 4 + tid; i < zero_words; i += nthreads) zero_buf[i] = 0u;
    }
}

__global__ __launch_bounds__(256) void zero_kernel(uint32_t* __restrict__ p, size_t n) {
    const size_t tid = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t nthreads = static_cast<size_t>(gridDim.x) * blockDim.x;
    uint4* p4 = reinterpret_cast<uint4*>(p);
    const size_t n4 = n / 4;
    for (size_t i = tid; i < n4; i += nthreads) p4[i] = make_uint4(0u, 0u, 0u, 0u);
    for (size_t i = n4 * 4 + tid; i < n; i += nthreads) p[i] = 0u;
}

unsigned grid_for_words(size_t words) {
    const size_t g = (words / 4 + 255) / 256;
    return static_cast<unsigned>(g < 1 ? 1 : (g > 1024 ? 1024 : g));
}

}  // namespace

hipError_t launch_uq(const void* Q, int q_dtype, float* u, int rows, int D, float eps,
                     uint32_t* zero_buf, size_t zero_words, hipStream_t s) {
    unsigned grid = static_cast<unsigned>((rows + 3) / 4);  // 4 rows (waves) per block
    if (zero_buf != nullptr) {
        const unsigned gz = grid_for_words(zero_words);
        if (gz > grid) grid = gz;
    }
    if (grid < 1) grid = 1;
#define DCR_UQ_CASE(DTV, DCV)                                                                \
    launch_kernel(uq_kernel<DTV, DCV>, grid, dim3(256), 0, s, Q, u, rows, D, eps, zero_buf, \
                  zero_words)
#define DCR_UQ_DT(DTV)              \
    if (D == 64)                    \
        DCR_UQ_CASE(DTV, 64);       \
    else if (D == 128)              \
        DCR_UQ_CASE(DTV, 128);      \
    else                            \
        DCR_UQ_CASE(DTV, 0)
    switch (q_dtype) {
        case kF32: DCR_UQ_DT(kF32); break;
        case kF16: DCR_UQ_DT(kF16); break;
        default: DCR_UQ_DT(kBF16); break;
    }
#undef DCR_UQ_DT
#undef DCR_UQ_CASE
    return hipGetLastError();
}

hipError_t launch_zero(uint32_t* p, size_t n, hipStream_t s) {
    launch_kernel(zero_kernel, grid_for_words(n), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

}  // namespace dcr
