// dcr_kernels.h -- host-side launchers of the sparse decode kernels.
// Internal to libdcr_sparse_decode.so; the public C-ABI is
// include/dcr_sparse_decode.h.  Every launcher returns hipSuccess or the
// launch error and assumes its arguments were validated by the C-ABI layer.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dcr {

// Events attached to the next kernel launch of the calling thread.  The
// library's profiling mode sets them around one launcher call; the launch then
// goes through hipExtLaunchKernelGGL, which stamps the events with the
// dispatch packet's own begin and end times (no marker packets around the
// kernel, so the duration is the kernel's, as a kernel tracer reports it).
struct LaunchEvents {
    hipEvent_t start;
    hipEvent_t stop;
};
LaunchEvents& launch_events();

// When one launcher call makes several launches, the start event goes with
// the first and the stop event with every one (the last one's end stands).
template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds_bytes,
                          hipStream_t s, Args... args) {
    LaunchEvents& ev = launch_events();
    if (ev.start != nullptr || ev.stop != nullptr) {
        hipExtLaunchKernelGGL(kernel, grid, block, lds_bytes, s, ev.start, ev.stop, 0u,
                              static_cast<KArgs>(args)...);
        ev.start = nullptr;
    } else {
        kernel<<<grid, block, lds_bytes, s>>>(static_cast<KArgs>(args)...);
    }
}

// u[r, :] = Q[r, :] / max(||Q[r, :]||, eps) for r < rows (fp32 out).
// Also clears zero_words uint32 words at zero_buf (may be null).
hipError_t launch_uq(const void* Q, int q_dtype, float* u, int rows, int D, float eps,
                     uint32_t* zero_buf, size_t zero_words, hipStream_t s);

// Fill n uint32 words with zero (graph-capture-safe replacement for memset).
hipError_t launch_zero(uint32_t* p, size_t n, hipStream_t s);

// K/V rows: row n of KV head (b, g) is at ((b*Hkv + g) * ldn + n) * D elements
// (ldn >= N: the rows between consecutive KV heads; N for a contiguous cache).

// scores[b, g*n_rep + r, n] = bf16(sum_d K[b,g,n,d] * u[b, g*n_rep + r, d]).
hipError_t launch_score(const void* K, int kv_dtype, const float* u, uint16_t* scores, int B,
                        int Hkv, int n_rep, int N, int D, long long ldn, hipStream_t s);

// The same with u computed from Q (u_out receives u where a separate launch
// computes it), the scores stored as order-preserving 16-bit keys of their
// bf16 roundings (rows at stride ldsc = ceil(N/64)*64, the padding positions
// holding key 0, below every real key), the level-1 histogram of the
// keys written as slabs hist[B*H][score_slabs(...)][256], and, when res is
// not null, one residual byte per score in res (same layout; score_residual:
// with the key it rebuilds the fp32 dot product to 2^-15 relative).  valu:
// the VALU form (u by a separate launch into u_out, then score_kernel) even
// where the MFMA form fits (ceil(n_rep/4) * D <= 128); both give the same bits.
int score_slabs(int kv_dtype, int B, int Hkv, int N, int D);
hipError_t launch_score_fused(const void* K, const void* Q, int dtype, float eps, float* u_out,
                              uint16_t* keys, uint8_t* res, long long ldsc, slab_t* hist, int B,
                              int Hkv, int n_rep, int N, int D, long long ldn, bool valu, hipStream_t s);

// Level-1 histogram slabs of score rows: hist[row][hist_slabs(N)][256], one
// slab per 4096 positions.
int hist_slabs(int N);
hipError_t launch_hist(const uint16_t* scores, slab_t* hist, int rows, int N, hipStream_t s);

// Stable descending top-k of each score row (rows at stride ldsc >= N),
// written as ascending indices; the row's level-1 histogram is the sum of its
// nslab slabs.  ticket (nullable, [rows / n_rep]) is cleared for the fused
// attention that follows.
// Rows too few to fill the device are split into chunks (two launches); part
// is scratch of select_part_words(rows, N) words (may be null when that is 0).
size_t select_part_words(int rows, int N);
hipError_t launch_select(const uint16_t* scores, int ldsc, const slab_t* hist, int nslab,
                         int32_t* idx, uint32_t* ticket, int n_rep, int rows, int N, int k,
                         uint32_t* part, hipStream_t s);
// The same over rows of order-preserving keys padded with key 0 up to ldsc
// (launch_score_fused's).  idx may be null (no index list); sel (nullable,
// [rows][2]) receives each row's selection in closed form: the threshold key
// T and the position of the last selected tie -- position n is selected iff
// key(n) > T, or key(n) == T and n <= that position.
hipError_t launch_select_keys(const uint16_t* keys, int ldsc, const slab_t* hist, int nslab,
                              int32_t* idx, uint32_t* sel, uint32_t* ticket, int n_rep, int rows,
                              int N, int k, uint32_t* part, hipStream_t s);

// Softmax attention over the selected rows, split-k: writes (m, l, o)
// partials [B*H][nsplit][D+2] (groups = B * Hkv).  With ticket == null the
// partials are left for launch_combine and O is untouched; with a ticket
// array [B*Hkv] (all zero on entry) the last workgroup of each group merges
// them into O.
int attn_num_splits(int groups, int k);
hipError_t launch_sparse_attn(const void* Q, const void* K, const void* V, int dtype,
                              const int32_t* idx, float* part, uint32_t* ticket, void* O, int B,
                              int H, int Hkv, int N, long long ldn, int D, int k, int nsplit,
                              hipStream_t s);

// The same with the logits taken from the score pass instead of a K gather:
// keys and res [B*H][ldsc] (launch_score_fused's outputs) give K[n]·u for
// every position (u = q / max(||q||, eps)), read at the selected positions,
// so only V rows are gathered.  fp16 and bf16 only.
hipError_t launch_scored_attn(const void* Q, const void* V, int dtype, const int32_t* idx,
                              const uint16_t* keys, const uint8_t* res, long long ldsc, float eps,
                              float* part,
                              uint32_t* ticket, void* O, int B, int H, int Hkv, int N, long long ldn,
                              int D, int k, int nsplit, hipStream_t s);

// The same from the selection in closed form (launch_select_keys's sel)
// instead of index lists: workgroup (split, group) reads the keys and
// residual bytes of its positions for the group's n_rep heads, selects, and
// gathers the V row of every position some head selected once, adding it to
// each selecting head's sums; (m, l, o) partials [B*H][nsplit][D+2], merged
// by the group's last workgroup (ticket [B*Hkv], zero on entry).  fp16 and
// bf16 only; nsplit = union_attn_splits(N).
int union_attn_splits(int N);
hipError_t launch_union_attn(const void* Q, const void* V, int dtype, const uint32_t* sel,
                             const uint16_t* keys, const uint8_t* res, long long ldsc, float eps,
                             float* part, uint32_t* ticket, void* O, int B, int H, int Hkv, int N,
                             long long ldn, int D, hipStream_t s);

// The same over all N rows (dense decode attention), merged into O by each
// group's last workgroup: ticket [B*Hkv] 64-bit words of any contents (each
// launch leaves them ready for the next), tag a nonzero value with its low
// 20 bits clear, the same for every launch on one workspace.
int dense_num_splits(int groups, int N);
hipError_t launch_dense_attn(const void* Q, const void* K, const void* V, int dtype, float* part,
                             uint64_t* ticket, uint64_t tag, void* O, int B, int H, int Hkv, int N,
                             long long ldn, int D, int nsplit, hipStream_t s);

// Rank-local window attention: O [BH, Nq, D] and lse [BH, Nq] over sorted
// K/V rows; query i attends rows |j - r_center[i]| <= half_k.  perm null:
// K/V are sorted copies [BH, Nkv, D]; otherwise row j of query head bh is
// row perm[bh][j] of KV head (b, h / n_rep) of a cache whose heads are
// head_rows rows apart (bh = b * H + h).
hipError_t launch_rank_local(const void* Q, const void* K, const void* V, int dtype,
                             const int32_t* r_center, void* O, float* lse, int BH, int Nq, int Nkv,
                             int D, int half_k, float scale, const int32_t* perm, long long head_rows,
                             int H, int n_rep, hipStream_t s);

// The whole sparse decode step in one launch (fused.hip): 256 workgroups,
// one per CU, 32 per XCD; XCD x owns the (batch, KV-head) groups x, x + 8, ...
// and each of its workgroups one chunk of P positions of one of them, through
// score, select and attention phases separated by per-XCD barriers.  Shapes
// it serves: fp16/bf16, D in {64, 128}, n_rep in {1, 2, 4}, B * Hkv a
// multiple of 8 with (B * Hkv / 8) dividing 32.
constexpr int kFusedXcds = 8;
constexpr int kFusedWgPerXcd = 32;
struct FusedCtl {
    uint32_t ctr[kFusedXcds][32];                // per XCD (own 128-byte line): launch counter in word 0
    uint64_t flags[kFusedXcds][kFusedWgPerXcd];  // per XCD: one barrier slot per workgroup
};
struct FusedShape {
    bool ok;
    int gx;      // groups per XCD
    int chunks;  // workgroups (position chunks) per group
    int P;       // positions per chunk (a multiple of 64)
};
FusedShape fused_shape(int dtype, int B, int H, int Hkv, int N, int D, int k);
// keys, res: [B*H][ldsc]; hist1p [B*H*chunks][256]; hist2p [B*H*chunks][260];
// part [B*H*chunks][D+1]; ctl as above (any contents); idx null or [B*H][k].
hipError_t launch_fused_decode(const void* Q, const void* K, const void* V, int dtype, void* O,
                               int32_t* idx, uint16_t* keys, uint8_t* res, uint32_t* hist1p,
                               uint32_t* hist2p, float* part, FusedCtl* ctl, uint64_t nonce, float eps,
                               int B, int H, int Hkv, int N, long long ldn, long long ldsc, int D, int k,
                               const FusedShape& f, hipStream_t s);
// Device address of the fused path's sticky error word on the current device.
uint32_t* fused_error_word();

// O[b, h, :] = merge of the nsplit (m, l, o) partials, rounded to dtype.
// base2: the partials' m are base-2 logits (launch_dense_attn's); otherwise
// natural (launch_sparse_attn's, launch_scored_attn's).
hipError_t launch_combine(const float* part, void* O, int dtype, int BH, int D, int nsplit, bool base2,
                          hipStream_t s);

}  // namespace dcr
