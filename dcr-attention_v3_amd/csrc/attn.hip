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
//   * each wave writes its (m, l, o) partial.  In the fused decode path the
//     last workgroup of each GQA group merges the group's partials (ticket
//     counter, device-coherent partial stores and loads, no fences);
//     otherwise combine_kernel merges them in a second launch.
//   * fp16/bf16 decode rebuilds its logits from the score pass's key and
//     residual byte (SCORED below) and gathers V rows only.
// The dense comparator and k >= N fallback (all N rows, attention.py:673-739
// semantics with an fp32 softmax) is dense_kernel at the end of this file.
#include <math.h>

#include "dcr_common.h"
#include "dcr_kernels.h"
#include "dcr_radix.h"

namespace dcr {
namespace {

constexpr int kAttnUnroll = 4;
constexpr int kDensePrefetch = 2;  // dense pass: tile buffers per wave
// Splits per workgroup (the split count is rounded up to a multiple): two
// splits of one GQA group per workgroup (8 waves at n_rep = 4, one workgroup
// per CU at C2) trim the spread of the splits' finishing times (attention
// 20.5 -> 19.9 us at C2; 1 and 4 measured slower).
constexpr int kAttnSplitsPerWg = 2;

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

// Positions of one tile: row slot rs of instruction u holds list entry
// j + u*RPI + rs.  Entries at or past j1, or with an index outside [0, N),
// are invalid and read row 0 instead (always mapped).
struct TileIdx {
    int pos[kAttnUnroll];
    bool valid[kAttnUnroll];
};

// The gathered rows of a tile (SCORED: the positions' score keys and residual
// bytes instead of their K rows, kept raw until the tile is consumed so that
// loading a tile never waits for its own loads).
template <int DT, int D>
struct Tile {
    chunk_t k[kAttnUnroll], v[kAttnUnroll];
    uint32_t skey[kAttnUnroll], sres[kAttnUnroll];
};

template <int DT, int D, bool DENSE>
__device__ __forceinline__ void load_idx(TileIdx& t, const int32_t* __restrict__ ix, int j, int j1,
                                         int rs) {
    using G = AttnGeom<DT, D>;
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
        const int jj = j + u * G::RPI + rs;
        const bool in = jj < j1;
        const int jc = in ? jj : j1 - 1;
        if constexpr (DENSE)
            t.pos[u] = jj;
        else
            t.pos[u] = ix[jc];
        t.valid[u] = in;
    }
}

// Gather the rows of a tile: V, and K or (SCORED) the score key and residual
// byte of the row from the head's rows skey / sres.
template <int DT, int D, bool SCORED>
__device__ __forceinline__ void load_rows(Tile<DT, D>& t, TileIdx& ti,
                                          const uint8_t* __restrict__ Kg,
                                          const uint8_t* __restrict__ Vg,
                                          const uint16_t* __restrict__ skey,
                                          const uint8_t* __restrict__ sres, int N) {
    using G = AttnGeom<DT, D>;
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
        ti.valid[u] = ti.valid[u] && static_cast<unsigned>(ti.pos[u]) < static_cast<unsigned>(N);
        const int pos = ti.valid[u] ? ti.pos[u] : 0;
        const size_t off = static_cast<size_t>(pos) * G::RB;
        if constexpr (SCORED) {
            t.skey[u] = skey[pos];
            t.sres[u] = sres[pos];
        } else
            t.k[u] = *reinterpret_cast<const chunk_t*>(Kg + off);
        t.v[u] = *reinterpret_cast<const chunk_t*>(Vg + off);
    }
}

// Partial stores and loads: plain, or agent-scope relaxed atomics, which are
// coherent across the XCDs' L2 caches (stores write through to the device's
// coherence point; loads do not hit a stale line of their own L2), so the
// fused merge needs no L2 write-back or invalidation.
template <bool COHERENT>
__device__ __forceinline__ void store_part(float* p, float v) {
    if constexpr (COHERENT) {
        __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else {
        *p = v;
    }
}

template <bool COHERENT>
__device__ __forceinline__ float load_part(const float* p) {
    if constexpr (COHERENT) {
        return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    } else {
        return *p;
    }
}

constexpr int kCombineMax = 64;  // splits merged with all loads in one round trip

// O[bh, :] = sum_c w_c o_c / sum_c w_c l_c, w_c = exp(m_c - max_c m_c), for
// one (b, h) by one wave.  Every partial value is loaded before any is used
// (one memory round trip for up to kCombineMax splits); lane c holds m_c,
// l_c and w_c and broadcasts w_c by shuffle.  Summation order: M and L by
// butterfly over the lanes, o by c = 0, 1, ... in turn.
// Exponential of a softmax argument: e^x, or 2^x when the kernel keeps its
// logits in base 2 (the dense kernel: scale includes log2(e), see exp2_hw).
template <bool BASE2>
__device__ __forceinline__ float softmax_exp(float x) {
    if constexpr (BASE2) return exp2_hw(x);
    else return expf(x);
}

template <int DT, int D, bool COHERENT, bool BASE2>
__device__ __forceinline__ void combine_head(const float* __restrict__ pp, int nsplit,
                                             void* __restrict__ O, size_t bh) {
    const int lane = lane_id();
    constexpr int S = D + 2;
    constexpr int R = D / 64;
    float o[R];
#pragma unroll
    for (int r = 0; r < R; ++r) o[r] = 0.0f;
    float L = 0.0f;
    if (nsplit <= kCombineMax) {
        const float mc = lane < nsplit ? load_part<COHERENT>(pp + static_cast<size_t>(lane) * S) : -INFINITY;
        const float lc = lane < nsplit ? load_part<COHERENT>(pp + static_cast<size_t>(lane) * S + 1) : 0.0f;
        float v[kCombineMax][R];
#pragma unroll
        for (int c = 0; c < kCombineMax; ++c)
#pragma unroll
            for (int r = 0; r < R; ++r)
                v[c][r] = c < nsplit ? load_part<COHERENT>(pp + static_cast<size_t>(c) * S + 2 + r * 64 + lane) : 0.0f;
        float M = mc;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        const float w = (mc == -INFINITY) ? 0.0f : softmax_exp<BASE2>(mc - M);
        L = w * lc;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) L += __shfl_xor(L, off, 64);
#pragma unroll
        for (int c = 0; c < kCombineMax; ++c) {
            const float wc = __shfl(w, c, 64);
#pragma unroll
            for (int r = 0; r < R; ++r) o[r] = __builtin_fmaf(wc, v[c][r], o[r]);
        }
    } else {
        float M = -INFINITY;
        for (int c = lane; c < nsplit; c += 64) M = fmaxf(M, load_part<COHERENT>(pp + static_cast<size_t>(c) * S));
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        for (int c = lane; c < nsplit; c += 64) {
            const float mc = load_part<COHERENT>(pp + static_cast<size_t>(c) * S);
            const float w = (mc == -INFINITY) ? 0.0f : softmax_exp<BASE2>(mc - M);
            L = __builtin_fmaf(w, load_part<COHERENT>(pp + static_cast<size_t>(c) * S + 1), L);
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) L += __shfl_xor(L, off, 64);
        for (int c = 0; c < nsplit; ++c) {
            const float mc = load_part<COHERENT>(pp + static_cast<size_t>(c) * S);
            const float w = (mc == -INFINITY) ? 0.0f : softmax_exp<BASE2>(mc - M);
#pragma unroll
            for (int r = 0; r < R; ++r)
                o[r] = __builtin_fmaf(w, load_part<COHERENT>(pp + static_cast<size_t>(c) * S + 2 + r * 64 + lane), o[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) store_out<DT>(O, bh * D + r * 64 + lane, o[r] / L);
}

// One wave per (b, h).
template <int DT, int D, bool BASE2>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ part,
                                                      void* __restrict__ O, int BH, int nsplit) {
    const size_t bh = static_cast<size_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (bh >= static_cast<size_t>(BH)) return;
    combine_head<DT, D, false, BASE2>(part + bh * static_cast<size_t>(nsplit) * (D + 2), nsplit, O, bh);
}

// One wave's split of one head's index list, entries [j0, j1): the online
// softmax over the split's rows, then the RPI row slots merged, leaving every
// lane with the split's (M, l) and its 16-byte slice li of o (lanes of one
// slice agree).  Kg / Vg point at the head's KV group plus the lane's slice.
template <int DT, int D, bool SCORED>
__device__ __forceinline__ void gather_split(const void* __restrict__ Q, const uint8_t* __restrict__ Kg,
                                             const uint8_t* __restrict__ Vg, const int32_t* __restrict__ ix,
                                             const uint16_t* __restrict__ skey, const uint8_t* __restrict__ sres,
                                             size_t bh, float eps, float scale, int N, int j0, int j1,
                                             float& M_out, float& l_out, float (&o)[AttnGeom<DT, D>::EPC]) {
    using G = AttnGeom<DT, D>;
    constexpr int LPR = G::LPR, EPC = G::EPC, U = kAttnUnroll;
    const int lane = lane_id();
    const int li = lane % LPR;
    const int rs = lane / LPR;
    // Online-softmax state of this lane's row slot.
    float m = -INFINITY, l = 0.0f;
#pragma unroll
    for (int e = 0; e < EPC; ++e) o[e] = 0.0f;

    // Software pipeline: while tile t is computed, the rows of tile t+1 and
    // the list entries of tile t+2 are in flight, so each step waits for one
    // memory round trip instead of two (entries, then the rows they name).
    // The first two tiles' entries are requested before the query, so the
    // query's round trip overlaps theirs.
    TileIdx ti_cur, ti_nxt;
    Tile<DT, D> nxt;
    if (j0 < j1) {
        load_idx<DT, D, false>(ti_cur, ix, j0, j1, rs);
        load_idx<DT, D, false>(ti_nxt, ix, j0 + G::TILE, j1, rs);
    }
    float q[EPC];
    float qscale = scale;
    if constexpr (SCORED) {
        qscale = row_norm<DT, D>(Q, bh * D, eps) * scale;
    } else {
#pragma unroll
        for (int e = 0; e < EPC; ++e) q[e] = load_elem<DT>(Q, bh * D + li * EPC + e);
    }
    // One tile into the lane's online-softmax state.
    auto consume = [&](const Tile<DT, D>& cur, const TileIdx& ci) {
        float s[U];
        float tmax = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float acc;
            if constexpr (SCORED) {
                acc = score_from_key(cur.skey[u], cur.sres[u]);
            } else {
                acc = 0.0f;
#pragma unroll
                for (int e = 0; e < EPC; ++e) acc = __builtin_fmaf(q[e], chunk_elem<DT>(cur.k[u], e), acc);
                acc = row_sum<LPR>(acc);
            }
            s[u] = ci.valid[u] ? acc * qscale : -INFINITY;
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
                const float p = ci.valid[u] ? expf(s[u] - m_new) : 0.0f;
                l += p;
#pragma unroll
                for (int e = 0; e < EPC; ++e) o[e] = __builtin_fmaf(p, chunk_elem<DT>(cur.v[u], e), o[e]);
            }
            m = m_new;
        }
    };

    if (j0 < j1) load_rows<DT, D, SCORED>(nxt, ti_cur, Kg, Vg, skey, sres, N);
    for (int j = j0; j < j1; j += G::TILE) {
        const Tile<DT, D> cur = nxt;
        const TileIdx ci = ti_cur;
        ti_cur = ti_nxt;
        // Past the end these re-read the last entries and row 0: cache hits.
        load_rows<DT, D, SCORED>(nxt, ti_cur, Kg, Vg, skey, sres, N);
        load_idx<DT, D, false>(ti_nxt, ix, j + 2 * G::TILE, j1, rs);
        consume(cur, ci);
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
    M_out = M;
    l_out = l;
}

// FUSE: the workgroup that finishes a GQA group last (a per-group ticket,
// cleared beforehand by the select kernel) merges the group's partials and
// writes O, so no combine launch follows.  Partials are written and read
// with agent-scope atomics (store_part / load_part); each wave waits for its
// stores to complete before the workgroup takes its ticket.  No fence is
// used: on MI355X an agent-scope fence writes back (release) or invalidates
// (acquire) the whole XCD L2, which per workgroup costs more than the
// combine launch it would save.
//
// SCORED: the logits come from the score pass instead of a K gather.  keys
// and res hold, per (b, h) at row stride ldsc, the 16-bit key of the bf16
// score and the 8-bit residual of the fp32 dot product K[n]·u of every
// position n (u = q / max(||q||, eps)); score_from_key rebuilds that dot
// product to 2^-15 relative, and the logit of a selected position is it
// times max(||q||, eps) * scale, which equals q·K[n] * scale to that
// precision.  The gather reads V rows (and 3 bytes per position) only.
//
// SPW splits per workgroup: wave w serves head w % NREP of split
// blockIdx-split * SPW + w / NREP.
template <int DT, int D, int NREP, bool FUSE, bool SCORED, int SPW>
__global__ __launch_bounds__((64 * NREP * SPW)) void attn_kernel(
    const void* __restrict__ Q, const uint8_t* __restrict__ K, const uint8_t* __restrict__ V,
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ keys, const uint8_t* __restrict__ res,
    long long ldsc, float eps,
    float* __restrict__ part, uint32_t* __restrict__ ticket, void* __restrict__ O, int Hkv, int N,
    long long ldn, int k, int J, int nsplit, float scale) {
    using G = AttnGeom<DT, D>;
    constexpr int LPR = G::LPR, EPC = G::EPC, RB = G::RB;
    static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "row must tile a wave");

    const int lane = lane_id();
    const int w = static_cast<int>(threadIdx.x >> 6) % NREP;   // head within the group
    const int sl = static_cast<int>(threadIdx.x >> 6) / NREP;  // split within the workgroup
    // (split, group) in XCD order: the splits of a group run on the XCD that
    // selected its rows.
    const unsigned wid = xcd_order(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z),
                                   gridDim.x * gridDim.y * gridDim.z);
    const int c = static_cast<int>(wid % gridDim.x) * SPW + sl;
    const int g = static_cast<int>((wid / gridDim.x) % gridDim.y);
    const int b = static_cast<int>(wid / (gridDim.x * gridDim.y));
    const int H = Hkv * NREP;
    const int h = g * NREP + w;
    const size_t bh = static_cast<size_t>(b) * H + h;
    const int li = lane % LPR;   // 16-byte slice of the row
    const int rs = lane / LPR;   // row slot within a wave instruction

    const size_t kv_base = (static_cast<size_t>(b) * Hkv + g) * static_cast<size_t>(ldn) * RB +
                           static_cast<size_t>(li) * 16;
    const uint8_t* Kg = K + kv_base;
    const uint8_t* Vg = V + kv_base;
    const int32_t* ix = idx + bh * static_cast<size_t>(k);
    const uint16_t* skey = SCORED ? keys + bh * static_cast<size_t>(ldsc) : nullptr;
    const uint8_t* sres = SCORED ? res + bh * static_cast<size_t>(ldsc) : nullptr;
    const int j0 = c * J;
    const int j1 = (j0 + J < k) ? j0 + J : k;

    float M, l, o[EPC];
    gather_split<DT, D, SCORED>(Q, Kg, Vg, ix, skey, sres, bh, eps, scale, N, j0, j1, M, l, o);
    float* pc = part + (bh * static_cast<size_t>(nsplit) + c) * (D + 2);
    // The partial leaves as consecutive words: the row-slot-0 lanes put it in
    // the wave's LDS record, then lane i stores words i, i + 64, ... (for
    // D = 64 two stores per wave instead of EPC + 2 stores of scattered words,
    // each word of which is its own write-through transaction: C2 step
    // 59.1 -> 58.1 us).  Only this wave touches its record, and its LDS
    // accesses complete in order.
    __shared__ float stg[NREP * SPW][D + 2];
    float* sp = stg[threadIdx.x >> 6];
    if (lane == 0) {
        sp[0] = M;
        sp[1] = l;
    }
    if (rs == 0) {
#pragma unroll
        for (int e = 0; e < EPC; ++e) sp[2 + li * EPC + e] = o[e];
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = lane; i < D + 2; i += 64) store_part<FUSE>(pc + i, sp[i]);

    // Why the merging workgroup sees every partial, at the instruction level
    // (gfx950; tests/test_fused_merge_isa.py checks this order in the built
    // assembly of every fused instance):
    //   1. the partials are agent-scope atomic stores, emitted as
    //      `global_store_dword ... sc1`: written through past the XCD's L2
    //      to the device-coherent level, where agent-scope loads read;
    //   2. `s_waitcnt vmcnt(0)` (below) returns only when all of this wave's
    //      stores are acknowledged there -- the wait half of an agent-scope
    //      release; its other half, `buffer_wbl2 sc1`, writes back dirty L2
    //      lines of ordinary stores and has nothing to do for sc1 stores;
    //   3. `s_barrier` (__syncthreads) holds thread 0 until every wave of the
    //      workgroup has passed its wait, and thread 0 then issues the ticket
    //      RMW (`global_atomic_add`, agent scope, performed coherently);
    //   4. the workgroup whose RMW returns gridDim.x - 1 saw every other
    //      workgroup's RMW, each issued after that workgroup's stores
    //      completed; its loads of the partials are issued after the RMW's
    //      value is back (`s_waitcnt`, then a branch on it) and are agent-scope
    //      atomic loads, `global_load_dword ... sc1`, which do not hit a stale
    //      line in its own L2 or L1 -- the load half of an acquire; the other
    //      half, `buffer_inv sc1`, invalidates caches for ordinary loads, and
    //      none is used here.
    // The C++ memory model alone does not order relaxed accesses to different
    // locations; the full agent-scope release/acquire fences it would need
    // write back / invalidate the whole L2 per workgroup and cost more than
    // the merge (attention 23 -> 61 us with release, -> 90 us acq_rel).
    if constexpr (FUSE) {
        __shared__ uint32_t sh_last;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are done
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t done = __hip_atomic_fetch_add(ticket + static_cast<size_t>(b) * Hkv + g, 1u,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sh_last = (done == gridDim.x - 1u) ? 1u : 0u;
        }
        __syncthreads();
        if (sh_last != 0u && sl == 0)
            combine_head<DT, D, true, false>(part + bh * static_cast<size_t>(nsplit) * (D + 2), nsplit, O, bh);
    }
}

// One workgroup per query head: kHeadWaves waves split the head's index list
// ([w*J, w*J + J) for wave w) and merge their (m, l, o) in LDS, so there are
// no partials in HBM, no ticket and no second workgroup in the merge (which
// costs the split kernel ~3 us at C2: store write-through, wait, ticket,
// coherent loads, most of it at the tail).  Used when the heads give every CU
// two workgroups (B*H >= 512; C5: 176.8 -> 174.5 us); with fewer heads the
// split kernel's spread over all CUs wins (C2, 128 heads on 128 CUs: 20.7 ->
// 25.7 us).
constexpr int kHeadWaves = 16;
constexpr long long kHeadKernelMinHeads = 512;

template <int DT, int D, bool SCORED>
__global__ __launch_bounds__(64 * kHeadWaves) void attn_head_kernel(
    const void* __restrict__ Q, const uint8_t* __restrict__ K, const uint8_t* __restrict__ V,
    const int32_t* __restrict__ idx, const uint16_t* __restrict__ keys, const uint8_t* __restrict__ res,
    long long ldsc, float eps, void* __restrict__ O, int H, int n_rep, int N, long long ldn, int k, int J,
    float scale) {
    using G = AttnGeom<DT, D>;
    constexpr int LPR = G::LPR, EPC = G::EPC, RB = G::RB;
    __shared__ float red[kHeadWaves][D + 2];
    const int lane = lane_id();
    const int w = static_cast<int>(threadIdx.x >> 6);
    // heads in XCD order: a GQA group's heads (consecutive bh) run on one XCD
    const size_t bh = xcd_order(blockIdx.x, gridDim.x);
    const size_t b = bh / static_cast<size_t>(H);
    const size_t g = (bh % static_cast<size_t>(H)) / static_cast<size_t>(n_rep);
    const int Hkv = H / n_rep;
    const int li = lane % LPR, rs = lane / LPR;
    const size_t kv_base = (b * Hkv + g) * static_cast<size_t>(ldn) * RB + static_cast<size_t>(li) * 16;
    const int j0 = w * J;
    const int j1 = (j0 + J < k) ? j0 + J : k;
    float M, l, o[EPC];
    gather_split<DT, D, SCORED>(Q, K + kv_base, V + kv_base, idx + bh * static_cast<size_t>(k),
                                SCORED ? keys + bh * static_cast<size_t>(ldsc) : nullptr,
                                SCORED ? res + bh * static_cast<size_t>(ldsc) : nullptr, bh, eps, scale, N, j0, j1,
                                M, l, o);
    if (lane == 0) {
        red[w][0] = M;
        red[w][1] = l;
    }
    if (rs == 0) {
#pragma unroll
        for (int e = 0; e < EPC; ++e) red[w][2 + li * EPC + e] = o[e];
    }
    __syncthreads();
    // O = sum_w c_w o_w / sum_w c_w l_w, c_w = exp(m_w - max m), waves in order
    for (int d = static_cast<int>(threadIdx.x); d < D; d += 64 * kHeadWaves) {
        float Mx = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < kHeadWaves; ++ww) Mx = fmaxf(Mx, red[ww][0]);
        float L = 0.0f, S = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kHeadWaves; ++ww) {
            const float mw = red[ww][0];
            const float c = (mw == -INFINITY) ? 0.0f : expf(mw - Mx);
            L = __builtin_fmaf(c, red[ww][1], L);
            S = __builtin_fmaf(c, red[ww][2 + d], S);
        }
        store_out<DT>(O, bh * D + d, S / L);
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

struct AttnArgs {
    const void *Q, *K, *V;
    const int32_t* idx;
    const uint16_t* keys;  // score keys (SCORED only)
    const uint8_t* res;    // score residual bytes; non-null: SCORED (logits from the score pass)
    long long ldsc;
    float eps;
    float* part;
    uint32_t* ticket;  // non-null: merge in the kernel (FUSE)
    void* O;
    int B, H, Hkv, N;
    long long ldn;
    int k, nsplit;
    uint64_t* dense_ticket = nullptr;  // dense kernel: self-resetting tagged tickets [B*Hkv]
    uint64_t dense_tag = 0;
    uint32_t* err = nullptr;           // dense kernel: sticky error word
};

// The head-per-workgroup form serves a launch that merges in the kernel
// (ticket given) when its B*H heads fill the device.
inline bool use_head_kernel(const AttnArgs& a) {
    return a.ticket != nullptr && static_cast<long long>(a.B) * a.H >= kHeadKernelMinHeads;
}

template <int DT, int D, int NREP, bool FUSE, bool SCORED>
hipError_t launch_attn_t(const AttnArgs& a, hipStream_t s) {
    const float scale_h = static_cast<float>(1.0 / sqrt(static_cast<double>(D)));
    if constexpr (FUSE) {
        if (use_head_kernel(a)) {
            const int Jh = (a.k + kHeadWaves - 1) / kHeadWaves;
            launch_kernel(attn_head_kernel<DT, D, SCORED>, dim3(static_cast<unsigned>(a.B * a.H)),
                          dim3(64 * kHeadWaves), 0, s, a.Q, static_cast<const uint8_t*>(a.K),
                          static_cast<const uint8_t*>(a.V), a.idx, a.keys, a.res, a.ldsc, a.eps, a.O, a.H,
                          NREP, a.N, a.ldn, a.k, Jh, scale_h);
            return hipGetLastError();
        }
    }
    const int J = (a.k + a.nsplit - 1) / a.nsplit;
    constexpr int SPW = kAttnSplitsPerWg;
    if (a.nsplit % SPW != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(a.nsplit / SPW), static_cast<unsigned>(a.Hkv),
                    static_cast<unsigned>(a.B));
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(D)));
    launch_kernel(attn_kernel<DT, D, NREP, FUSE, SCORED, SPW>, grid, dim3(64 * NREP * SPW), 0, s, a.Q,
                  static_cast<const uint8_t*>(a.K), static_cast<const uint8_t*>(a.V), a.idx, a.keys, a.res,
                  a.ldsc, a.eps, a.part, a.ticket, a.O, a.Hkv, a.N, a.ldn, a.k, J, a.nsplit, scale);
    return hipGetLastError();
}

template <int DT, int D, int NREP>
hipError_t launch_attn_f(const AttnArgs& a, hipStream_t s) {
    if constexpr (DT != kF32) {
        // fp32 inputs keep the K gather: their 1e-5 output tolerance leaves
        // no room for the few-ulp logit difference of the scored form.
        if (a.res != nullptr) {
            if (a.ticket != nullptr) return launch_attn_t<DT, D, NREP, true, true>(a, s);
            return launch_attn_t<DT, D, NREP, false, true>(a, s);
        }
    }
    if (a.res != nullptr) return hipErrorInvalidValue;
    if (a.ticket != nullptr) return launch_attn_t<DT, D, NREP, true, false>(a, s);
    return launch_attn_t<DT, D, NREP, false, false>(a, s);
}

template <int DT, int D>
hipError_t launch_attn_rep(const AttnArgs& a, hipStream_t s) {
    switch (a.H / a.Hkv) {
        case 1: return launch_attn_f<DT, D, 1>(a, s);
        case 2: return launch_attn_f<DT, D, 2>(a, s);
        case 4: return launch_attn_f<DT, D, 4>(a, s);
        case 8: return launch_attn_f<DT, D, 8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_any(const AttnArgs& a, int dtype, int D, hipStream_t s) {
#define DCR_ATTN_CASE(DTV, DV) \
    if (dtype == DTV && D == DV) return launch_attn_rep<DTV, DV>(a, s);
    DCR_ATTN_CASE(kF32, 64)
    DCR_ATTN_CASE(kF16, 64)
    DCR_ATTN_CASE(kBF16, 64)
    DCR_ATTN_CASE(kF32, 128)
    DCR_ATTN_CASE(kF16, 128)
    DCR_ATTN_CASE(kBF16, 128)
#undef DCR_ATTN_CASE
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Dense decode attention (all N rows): the comparator and the k >= N
// fallback.  A workgroup of kDenseWaves waves owns split c of one GQA group;
// wave w walks tiles w, w + kDenseWaves, ... of the split, and every wave
// serves all NREP query heads of the group from the rows it loads, so each
// K/V row is read by one wave once (the per-head waves of attn_kernel would
// read it NREP times).  Loads run kDensePrefetch tiles ahead.  The waves'
// per-head states merge in LDS; the workgroup writes one (m, l, o) partial
// per head, and the group's last workgroup merges them into O.
constexpr int kDenseWaves = 4;

// Merge tickets that reset themselves.  The dense path is one launch, with
// no earlier launch in its call to clear a ticket, and its workspace may hold
// anything on a first use.  A group's ticket is a 64-bit word: a tag in the
// high 44 bits (one nonzero value per process, from the host) and in the low
// 20 bits the count of workgroups that took a ticket under it.  A workgroup
// whose add returns a word without the tag installs (tag, 1) with a
// compare-and-swap from the word as last seen, which makes it the first; a
// failed swap returns the current word, and once that carries the tag the
// workgroup adds again.  While the word is stale it changes only through
// each workgroup's one add and the one successful swap, so the loop ends
// after a bounded number of rounds; kTicketSpinMax bounds it regardless (on
// expiry the workgroup sets bit 1 of err and takes no part in the merge, so
// that launch's output is not valid).  The workgroup that takes ticket
// nsplit - 1 merges and stores (tag, 0), ready for the next launch on the
// workspace (graph replays included: the word is (tag, 0) again).
constexpr int kTicketCountBits = 20;
constexpr uint64_t kTicketCountMask = (uint64_t{1} << kTicketCountBits) - 1u;
constexpr uint32_t kTicketSpinMax = 1u << 16;

__device__ __forceinline__ uint32_t take_tagged_ticket(uint64_t* tk, uint64_t tag, uint32_t* err) {
    const uint64_t old = __hip_atomic_fetch_add(tk, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((old & ~kTicketCountMask) == tag) return static_cast<uint32_t>(old & kTicketCountMask);
    uint64_t cur = old + 1u;  // the word after this add, unless others added since
    for (uint32_t spin = 0; spin < kTicketSpinMax; ++spin) {
        uint64_t expected = cur;
        if (__hip_atomic_compare_exchange_strong(tk, &expected, tag | 1u, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
            return 0u;
        cur = expected;
        if ((cur & ~kTicketCountMask) == tag)
            return static_cast<uint32_t>(
                __hip_atomic_fetch_add(tk, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                kTicketCountMask);
    }
    atomicOr(err, 2u);
    return 0xffffffffu;
}

template <int DT, int D, int NREP>
__global__ __launch_bounds__(64 * kDenseWaves) void dense_kernel(
    const void* __restrict__ Q, const uint8_t* __restrict__ K, const uint8_t* __restrict__ V,
    float* __restrict__ part, uint64_t* __restrict__ ticket, uint64_t tag, uint32_t* err,
    void* __restrict__ O, int Hkv, int N, long long ldn, int J, int nsplit, float scale) {
    using G = AttnGeom<DT, D>;
    constexpr int LPR = G::LPR, EPC = G::EPC, RB = G::RB, U = kAttnUnroll, PF = kDensePrefetch;
    constexpr int W = kDenseWaves;
    static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "row must tile a wave");
    __shared__ float red[W][NREP][D + 2];

    const int lane = lane_id();
    const int w = static_cast<int>(threadIdx.x >> 6);
    const unsigned wid = xcd_order(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z),
                                   gridDim.x * gridDim.y * gridDim.z);
    const int c = static_cast<int>(wid % gridDim.x);
    const int g = static_cast<int>((wid / gridDim.x) % gridDim.y);
    const int b = static_cast<int>(wid / (gridDim.x * gridDim.y));
    const int H = Hkv * NREP;
    const size_t bh0 = static_cast<size_t>(b) * H + static_cast<size_t>(g) * NREP;
    const int li = lane % LPR;
    const int rs = lane / LPR;
    const size_t kv_base = (static_cast<size_t>(b) * Hkv + g) * static_cast<size_t>(ldn) * RB +
                           static_cast<size_t>(li) * 16;
    const uint8_t* Kg = K + kv_base;
    const uint8_t* Vg = V + kv_base;
    const int j0 = c * J;
    const int j1 = (j0 + J < N) ? j0 + J : N;
    constexpr int STEP = W * G::TILE;  // rows between a wave's consecutive tiles

    // Tiles of this wave: rows [j0 + w*TILE + i*STEP, ... + TILE).
    Tile<DT, D> buf[PF];
    TileIdx bi[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        load_idx<DT, D, true>(bi[p], nullptr, j0 + w * G::TILE + p * STEP, j1, rs);
        load_rows<DT, D, false>(buf[p], bi[p], Kg, Vg, nullptr, nullptr, N);
    }
    float q[NREP][EPC];
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
        for (int e = 0; e < EPC; ++e) q[h][e] = load_elem<DT>(Q, (bh0 + h) * D + li * EPC + e);

    float m[NREP], l[NREP], o[NREP][EPC];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPC; ++e) o[h][e] = 0.0f;
    }

    // Each buffer is consumed before it is refilled, so PF buffers are live
    // and PF - 1 tiles are in flight while one is computed.
    for (int j = j0 + w * G::TILE; j < j1; j += PF * STEP) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const Tile<DT, D>& cur = buf[p];
            const TileIdx& ci = bi[p];
#pragma unroll
            for (int h = 0; h < NREP; ++h) {
                float sc[U];
                float tmax = -INFINITY;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    float acc = 0.0f;
#pragma unroll
                    for (int e = 0; e < EPC; ++e) acc = __builtin_fmaf(q[h][e], chunk_elem<DT>(cur.k[u], e), acc);
                    acc = row_sum<LPR>(acc);
                    sc[u] = ci.valid[u] ? acc * scale : -INFINITY;
                    tmax = fmaxf(tmax, sc[u]);
                }
                const float m_new = fmaxf(m[h], tmax);
                if (m_new != -INFINITY) {
                    const float alpha = exp2_hw(m[h] - m_new);
                    l[h] *= alpha;
#pragma unroll
                    for (int e = 0; e < EPC; ++e) o[h][e] *= alpha;
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const float pr = ci.valid[u] ? exp2_hw(sc[u] - m_new) : 0.0f;
                        l[h] += pr;
#pragma unroll
                        for (int e = 0; e < EPC; ++e)
                            o[h][e] = __builtin_fmaf(pr, chunk_elem<DT>(cur.v[u], e), o[h][e]);
                    }
                    m[h] = m_new;
                }
            }
            load_idx<DT, D, true>(bi[p], nullptr, j + (p + PF) * STEP, j1, rs);
            load_rows<DT, D, false>(buf[p], bi[p], Kg, Vg, nullptr, nullptr, N);
        }
    }

    // Per head: merge the wave's row slots, then the waves (in LDS).
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        float M = m[h];
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        const float f = (m[h] == -INFINITY) ? 0.0f : exp2_hw(m[h] - M);
        float L = l[h] * f;
        float oo[EPC];
#pragma unroll
        for (int e = 0; e < EPC; ++e) oo[e] = o[h][e] * f;
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) {
            L += __shfl_xor(L, off, 64);
#pragma unroll
            for (int e = 0; e < EPC; ++e) oo[e] += __shfl_xor(oo[e], off, 64);
        }
        if (lane == 0) {
            red[w][h][0] = M;
            red[w][h][1] = L;
        }
        if (rs == 0) {
#pragma unroll
            for (int e = 0; e < EPC; ++e) red[w][h][2 + li * EPC + e] = oo[e];
        }
    }
    __syncthreads();
    // Wave w merges heads w, w + W, ... and writes the workgroup's partial.
    for (int h = w; h < NREP; h += W) {
        float Mw = -INFINITY;
#pragma unroll
        for (int x = 0; x < W; ++x) Mw = fmaxf(Mw, red[x][h][0]);
        float L = 0.0f;
        float acc[(D + 63) / 64];
#pragma unroll
        for (int r = 0; r < (D + 63) / 64; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int x = 0; x < W; ++x) {
            const float mx = red[x][h][0];
            const float f = (mx == -INFINITY) ? 0.0f : exp2_hw(mx - Mw);
            L = __builtin_fmaf(f, red[x][h][1], L);
#pragma unroll
            for (int r = 0; r < (D + 63) / 64; ++r)
                if (r * 64 + lane < D) acc[r] = __builtin_fmaf(f, red[x][h][2 + r * 64 + lane], acc[r]);
        }
        float* pc = part + ((bh0 + h) * static_cast<size_t>(nsplit) + c) * (D + 2);
        if (lane == 0) {
            store_part<true>(pc, Mw);
            store_part<true>(pc + 1, L);
        }
#pragma unroll
        for (int r = 0; r < (D + 63) / 64; ++r)
            if (r * 64 + lane < D) store_part<true>(pc + 2 + r * 64 + lane, acc[r]);
    }

    // The group's merge, in the order of attn_kernel's FUSE merge (its
    // comment gives the instruction-level argument): this wave's partial
    // stores complete, the workgroup meets, thread 0 takes the ticket, and
    // the last workgroup's agent-scope loads follow the ticket's value.
    __shared__ uint32_t sh_last;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are done
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t* tk = ticket + static_cast<size_t>(b) * Hkv + g;
        const uint32_t t = take_tagged_ticket(tk, tag, err);
        const bool last = t == static_cast<uint32_t>(nsplit) - 1u;
        if (last) __hip_atomic_store(tk, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh_last = last ? 1u : 0u;
    }
    __syncthreads();
    if (sh_last != 0u) {
        for (int h = w; h < NREP; h += W)
            combine_head<DT, D, true, true>(part + (bh0 + h) * static_cast<size_t>(nsplit) * (D + 2), nsplit, O,
                                            bh0 + h);
    }
}

template <int DT, int D, int NREP>
hipError_t launch_dense_t(const AttnArgs& a, hipStream_t s) {
    const int J = (a.N + a.nsplit - 1) / a.nsplit;
    const dim3 grid(static_cast<unsigned>(a.nsplit), static_cast<unsigned>(a.Hkv),
                    static_cast<unsigned>(a.B));
    const float scale = static_cast<float>(kLog2e / sqrt(static_cast<double>(D)));  // base-2 logits
    launch_kernel(dense_kernel<DT, D, NREP>, grid, dim3(64 * kDenseWaves), 0, s, a.Q,
                  static_cast<const uint8_t*>(a.K), static_cast<const uint8_t*>(a.V), a.part, a.dense_ticket,
                  a.dense_tag, a.err, a.O, a.Hkv, a.N, a.ldn, J, a.nsplit, scale);
    return hipGetLastError();
}

template <int DT, int D>
hipError_t launch_dense_rep(const AttnArgs& a, hipStream_t s) {
    switch (a.H / a.Hkv) {
        case 1: return launch_dense_t<DT, D, 1>(a, s);
        case 2: return launch_dense_t<DT, D, 2>(a, s);
        case 4: return launch_dense_t<DT, D, 4>(a, s);
        case 8: return launch_dense_t<DT, D, 8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Union gather: the attention of a GQA group's n_rep heads from their
// selections in closed form (T, last selected tie; select.hip's sel), one V
// read per position that any of the heads selected.
//
// Workgroup (split c, group bg) of 4 waves owns positions [c*S, c*S + S),
// S = 256 * KPT; thread t the KPT positions from c*S + t*KPT.  It
//   1. loads the positions' keys and residual bytes for every head of the
//      group (coalesced: the rows are position-ordered) and the heads' query
//      norms, and marks each head's selected positions: key > T, or key == T
//      at a position <= the last selected tie;
//   2. takes each head's largest selected logit over the split as its
//      softmax reference m (a block max in LDS);
//   3. lists, per wave, the positions some head selected, in position order,
//      with each head's weight exp(logit - m) (0 for a head that did not
//      select the position) -- a wave prefix sum over the lanes' counts;
//   4. walks the wave's list: LPR lanes x 16 bytes per V row, RPI rows per
//      instruction, kAttnUnroll instructions per tile, the next tile in
//      flight while one is added into every head's (l, o);
//   5. sums the row slots and the waves and writes each head's (m, l, o)
//      partial; the group's last workgroup (ticket) merges the group's
//      partials into O (combine_head, as the index-list kernel's FUSE merge;
//      the same instruction order, checked by tests/test_fused_merge_isa.py).
// The logit of a position is rebuilt from its key and residual byte times
// max(||q||, eps) / sqrt(D), as in attn_kernel's SCORED form.
constexpr int kUnionWaves = 4;

template <int DT, int D, int NREP, int KPT>
struct UnionSmem {
    static constexpr int EPW = 64 * KPT;   // list entries per wave, at most
    uint32_t epos[kUnionWaves][EPW];
    float ep[kUnionWaves][EPW][NREP];
    float red[kUnionWaves][NREP][D + 1];
    float qs[NREP];
    uint32_t mx[NREP];
    uint32_t last;
};

// Four waves per SIMD (VGPRs <= 128) where the heads and keys per thread
// allow: four workgroups per CU, so all 1024 of C2 are resident at once
// instead of three per CU and a second round.
template <int NREP, int KPT>
constexpr int union_min_waves() {
    return NREP <= 4 ? (KPT == 4 ? 4 : 3) : (KPT == 4 ? 2 : 1);
}

template <int DT, int D, int NREP, int KPT>
__global__ __launch_bounds__(64 * kUnionWaves, (union_min_waves<NREP, KPT>())) void union_attn_kernel(
    const void* __restrict__ Q, const uint8_t* __restrict__ V, const uint32_t* __restrict__ sel,
    const uint16_t* __restrict__ keys, const uint8_t* __restrict__ res, long long ldsc, float eps,
    float* __restrict__ part, uint32_t* __restrict__ ticket, void* __restrict__ O, long long ldn, int nsplit,
    float scale) {
    using G = AttnGeom<DT, D>;
    constexpr int LPR = G::LPR, RPI = G::RPI, EPC = G::EPC, RB = G::RB, U = kAttnUnroll, TILE = G::TILE;
    constexpr int THREADS = 64 * kUnionWaves;
    constexpr int S = THREADS * KPT;
    static_assert(KPT == 4 || KPT == 8, "keys are loaded 4 or 8 at a time");
    using SM = UnionSmem<DT, D, NREP, KPT>;
    __shared__ SM sm;

    const int t = static_cast<int>(threadIdx.x);
    const int lane = lane_id();
    const int w = t >> 6;
    // (split, group) in XCD order: a group's splits run on one XCD.
    const unsigned wid = xcd_order(blockIdx.x, gridDim.x);
    const int c = static_cast<int>(wid % static_cast<unsigned>(nsplit));
    const size_t bg = wid / static_cast<unsigned>(nsplit);   // b * Hkv + g
    const size_t head0 = bg * NREP;                          // row b * H + h of head 0
    const uint8_t* Vg = V + bg * static_cast<size_t>(ldn) * RB;
    const int pos = c * S + t * KPT;
    const bool in = pos < ldsc;  // ldsc: a multiple of 64, padded with key 0 (never selected)

    // ---- 1. keys, residuals, selections ----------------------------------
    uint32_t kw[NREP][KPT / 2], rw[NREP][KPT / 4];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        const size_t ro = (head0 + h) * static_cast<size_t>(ldsc) + (in ? pos : 0);
        if constexpr (KPT == 4) {
            const uint2 k2 = *reinterpret_cast<const uint2*>(keys + ro);
            kw[h][0] = k2.x;
            kw[h][1] = k2.y;
            rw[h][0] = *reinterpret_cast<const uint32_t*>(res + ro);
        } else {
            const uint4 k4 = *reinterpret_cast<const uint4*>(keys + ro);
            kw[h][0] = k4.x;
            kw[h][1] = k4.y;
            kw[h][2] = k4.z;
            kw[h][3] = k4.w;
            const uint2 r2 = *reinterpret_cast<const uint2*>(res + ro);
            rw[h][0] = r2.x;
            rw[h][1] = r2.y;
        }
    }
    if (t < NREP) sm.mx[t] = 0u;
    // logits in base 2 (scale * log2(e) folded in): one hardware exp2 per weight
    for (int h = w; h < NREP; h += kUnionWaves) {
        const float qn = row_norm<DT, D>(Q, (head0 + h) * static_cast<size_t>(D), eps);
        if (lane == 0) sm.qs[h] = qn * (scale * static_cast<float>(kLog2e));
    }
    auto key_of = [&](int h, int j) { return (kw[h][j >> 1] >> ((j & 1) * 16)) & 0xffffu; };
    auto res_of = [&](int h, int j) { return (rw[h][j >> 2] >> ((j & 3) * 8)) & 0xffu; };
    uint32_t selb[NREP];
    float smax[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        const uint32_t T = sel[2 * (head0 + h)];
        const uint32_t last_tie = sel[2 * (head0 + h) + 1];
        selb[h] = 0u;
        smax[h] = -INFINITY;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const uint32_t key = key_of(h, j);
            const bool take = in && (key > T || (key == T && static_cast<uint32_t>(pos + j) <= last_tie));
            selb[h] |= take ? (1u << j) : 0u;
            if (take) smax[h] = fmaxf(smax[h], score_from_key(key, res_of(h, j)));
        }
    }
    __syncthreads();  // sm.mx cleared, sm.qs written

    // ---- 2. each head's largest selected score over the split --------------
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        float v = smax[h];
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
        if (lane == 0 && v != -INFINITY) atomicMax(&sm.mx[h], ordered_bits(v));
    }
    __syncthreads();
    float qs[NREP], m[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        qs[h] = sm.qs[h];
        const uint32_t mo = sm.mx[h];
        m[h] = mo != 0u ? from_ordered(mo) * qs[h] : -INFINITY;
    }

    // ---- 3. the wave's list of positions with each head's weight ---------
    uint32_t uni = 0u;
#pragma unroll
    for (int h = 0; h < NREP; ++h) uni |= selb[h];
    const uint32_t n = static_cast<uint32_t>(__builtin_popcount(uni));
    const uint32_t incl = wave_inclusive_scan(n);
    const uint32_t cntw = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        static_cast<int>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63)))));
    uint32_t* epos = sm.epos[w];
    float (*ep)[NREP] = sm.ep[w];
    {
        uint32_t slot = incl - n;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            if (!(uni & (1u << j))) continue;
            epos[slot] = static_cast<uint32_t>(pos + j);
#pragma unroll
            for (int h = 0; h < NREP; ++h)
                ep[slot][h] = (selb[h] & (1u << j)) ? exp2_hw(score_from_key(key_of(h, j), res_of(h, j)) * qs[h] - m[h])
                                                   : 0.0f;
            ++slot;
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's list writes are done
    __builtin_amdgcn_wave_barrier();

    // ---- 4. gather the listed V rows ---------------------------------------
    const int li = lane % LPR;  // 16-byte slice of a V row
    const int rs = lane / LPR;  // row slot within a gather instruction
    float l[NREP], o[NREP][EPC];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPC; ++e) o[h][e] = 0.0f;
    }
    auto fetch = [&](chunk_t (&vv)[U], uint32_t e0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t ei = e0 + static_cast<uint32_t>(u * RPI + rs);
            const uint32_t pv = epos[ei < cntw ? ei : 0u];
            vv[u] = *reinterpret_cast<const chunk_t*>(Vg + static_cast<size_t>(pv) * RB + li * 16);
        }
    };
    auto accumulate = [&](const chunk_t (&vv)[U], uint32_t e0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
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
    // Unconditional fetches (entries past the list's end re-read the first
    // entry's row and weigh it 0): the waits count the same loads on every
    // path, so the next tile stays in flight while one is added up.  Each
    // buffer is refilled right after it is added up (not before the other is),
    // which lets the compiler keep both in place across the loop's back edge
    // (the other order made it copy a buffer there, behind a vmcnt(0)).
    if (cntw > 0u) {
        chunk_t va[U], vb[U];
        fetch(va, 0u);
        fetch(vb, TILE);
        for (uint32_t e0 = 0; e0 < cntw; e0 += 2 * TILE) {
            accumulate(va, e0);
            fetch(va, e0 + 2 * TILE);
            accumulate(vb, e0 + TILE);
            fetch(vb, e0 + 3 * TILE);
        }
    }

    // ---- 5. partials and the group's merge ---------------------------------
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
#pragma unroll
        for (int off = LPR; off < 64; off <<= 1) {
            l[h] += __shfl_xor(l[h], off, 64);
#pragma unroll
            for (int e = 0; e < EPC; ++e) o[h][e] += __shfl_xor(o[h][e], off, 64);
        }
        if (lane == 0) sm.red[w][h][0] = l[h];
        if (rs == 0) {
#pragma unroll
            for (int e = 0; e < EPC; ++e) sm.red[w][h][1 + li * EPC + e] = o[h][e];
        }
    }
    __syncthreads();
    for (int i = t; i < NREP * (D + 2); i += THREADS) {
        const int h = i / (D + 2), d = i % (D + 2);
        float v;
        if (d == 0) {
            v = m[h];
        } else {
            v = 0.0f;
#pragma unroll
            for (int ww = 0; ww < kUnionWaves; ++ww) v += sm.red[ww][h][d - 1];
        }
        store_part<true>(part + ((head0 + h) * static_cast<size_t>(nsplit) + c) * (D + 2) + d, v);
    }
    // The same order as attn_kernel's FUSE merge: this wave's partial stores
    // complete (vmcnt(0)), the workgroup meets, thread 0 takes the ticket, and
    // the last workgroup's coherent loads follow the ticket's value.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (t == 0) {
        const uint32_t done = __hip_atomic_fetch_add(ticket + bg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sm.last = (done == static_cast<uint32_t>(nsplit) - 1u) ? 1u : 0u;
    }
    __syncthreads();
    if (sm.last != 0u) {
        for (int h = w; h < NREP; h += kUnionWaves)
            combine_head<DT, D, true, true>(part + (head0 + h) * static_cast<size_t>(nsplit) * (D + 2), nsplit, O,
                                            head0 + h);
    }
}

// Positions per thread: 4, or 8 for rows longer than 64 splits of 1024
// (combine_head merges up to kCombineMax splits in one round trip).
int union_kpt(int N) { return N <= kCombineMax * kUnionWaves * 64 * 4 ? 4 : 8; }

template <int DT, int D, int NREP>
hipError_t launch_union_t(const void* Q, const void* V, const uint32_t* sel, const uint16_t* keys,
                          const uint8_t* res, long long ldsc, float eps, float* part, uint32_t* ticket,
                          void* O, int groups, int N, long long ldn, hipStream_t s) {
    const float scale = static_cast<float>(1.0 / sqrt(static_cast<double>(D)));
    const int kpt = union_kpt(N);
    const int nsplit = (N + kUnionWaves * 64 * kpt - 1) / (kUnionWaves * 64 * kpt);
    const dim3 grid(static_cast<unsigned>(nsplit * groups));
    const auto V8 = static_cast<const uint8_t*>(V);
    if (kpt == 4)
        launch_kernel(union_attn_kernel<DT, D, NREP, 4>, grid, dim3(64 * kUnionWaves), 0, s, Q, V8, sel, keys, res,
                      ldsc, eps, part, ticket, O, ldn, nsplit, scale);
    else
        launch_kernel(union_attn_kernel<DT, D, NREP, 8>, grid, dim3(64 * kUnionWaves), 0, s, Q, V8, sel, keys, res,
                      ldsc, eps, part, ticket, O, ldn, nsplit, scale);
    return hipGetLastError();
}

template <int DT, int D>
hipError_t launch_union_rep(const void* Q, const void* V, const uint32_t* sel, const uint16_t* keys,
                            const uint8_t* res, long long ldsc, float eps, float* part, uint32_t* ticket,
                            void* O, int groups, int n_rep, int N, long long ldn, hipStream_t s) {
    switch (n_rep) {
        case 1: return launch_union_t<DT, D, 1>(Q, V, sel, keys, res, ldsc, eps, part, ticket, O, groups, N, ldn, s);
        case 2: return launch_union_t<DT, D, 2>(Q, V, sel, keys, res, ldsc, eps, part, ticket, O, groups, N, ldn, s);
        case 4: return launch_union_t<DT, D, 4>(Q, V, sel, keys, res, ldsc, eps, part, ticket, O, groups, N, ldn, s);
        case 8: return launch_union_t<DT, D, 8>(Q, V, sel, keys, res, ldsc, eps, part, ticket, O, groups, N, ldn, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dense_any(const AttnArgs& a, int dtype, int D, hipStream_t s) {
#define DCR_DENSE_CASE(DTV, DV) \
    if (dtype == DTV && D == DV) return launch_dense_rep<DTV, DV>(a, s);
    DCR_DENSE_CASE(kF32, 64)
    DCR_DENSE_CASE(kF16, 64)
    DCR_DENSE_CASE(kBF16, 64)
    DCR_DENSE_CASE(kF32, 128)
    DCR_DENSE_CASE(kF16, 128)
    DCR_DENSE_CASE(kBF16, 128)
#undef DCR_DENSE_CASE
    return hipErrorInvalidValue;
}

}  // namespace

int attn_num_splits(int groups, int k) {
    const int tile = AttnGeom<kF16, 64>::TILE;  // 32 rows
    const int J = split_rows(groups, k, tile);
    const int n = (k + J - 1) / J;
    return (n + kAttnSplitsPerWg - 1) / kAttnSplitsPerWg * kAttnSplitsPerWg;
}

int dense_num_splits(int groups, int N) {
    // Rows per split: a multiple of the waves' tile stride, enough splits for
    // about two workgroups per CU.
    const int stride = kDenseWaves * AttnGeom<kF16, 64>::TILE;
    const int J = split_rows(groups, N, stride);
    return (N + J - 1) / J;
}

hipError_t launch_sparse_attn(const void* Q, const void* K, const void* V, int dtype,
                              const int32_t* idx, float* part, uint32_t* ticket, void* O, int B, int H, int Hkv,
                              int N, long long ldn, int D, int k, int nsplit, hipStream_t s) {
    const AttnArgs a{Q, K, V, idx, nullptr, nullptr, 0, 0.0f, part, ticket, O, B, H, Hkv, N, ldn, k, nsplit};
    return launch_attn_any(a, dtype, D, s);
}

hipError_t launch_scored_attn(const void* Q, const void* V, int dtype, const int32_t* idx,
                              const uint16_t* keys, const uint8_t* res, long long ldsc, float eps, float* part,
                              uint32_t* ticket, void* O, int B, int H, int Hkv, int N, long long ldn,
                              int D, int k, int nsplit, hipStream_t s) {
    if (dtype == kF32 || keys == nullptr || res == nullptr) return hipErrorInvalidValue;
    const AttnArgs a{Q, V, V, idx, keys, res, ldsc, eps, part, ticket, O, B, H, Hkv, N, ldn, k, nsplit};
    return launch_attn_any(a, dtype, D, s);
}

int union_attn_splits(int N) {
    const int S = kUnionWaves * 64 * union_kpt(N);
    return (N + S - 1) / S;
}

hipError_t launch_union_attn(const void* Q, const void* V, int dtype, const uint32_t* sel,
                             const uint16_t* keys, const uint8_t* res, long long ldsc, float eps,
                             float* part, uint32_t* ticket, void* O, int B, int H, int Hkv, int N,
                             long long ldn, int D, hipStream_t s) {
    if (sel == nullptr || keys == nullptr || res == nullptr || ticket == nullptr || H % Hkv != 0)
        return hipErrorInvalidValue;
    const int groups = B * Hkv, n_rep = H / Hkv;
    if (dtype == kF16 && D == 64)
        return launch_union_rep<kF16, 64>(Q, V, sel, keys, res, ldsc, eps, part, ticket, O, groups, n_rep, N, ldn, s);
    if (dtype == kBF16 && D == 64)
        return launch_union_rep<kBF16, 64>(Q, V, sel, keys, res, ldsc, eps, part, ticket, O, groups, n_rep, N, ldn, s);
    if (dtype == kF16 && D == 128)
        return launch_union_rep<kF16, 128>(Q, V, sel, keys, res, ldsc, eps, part, ticket, O, groups, n_rep, N, ldn, s);
    if (dtype == kBF16 && D == 128)
        return launch_union_rep<kBF16, 128>(Q, V, sel, keys, res, ldsc, eps, part, ticket, O, groups, n_rep, N, ldn,
                                            s);
    return hipErrorInvalidValue;
}

hipError_t launch_dense_attn(const void* Q, const void* K, const void* V, int dtype, float* part,
                             uint64_t* ticket, uint64_t tag, void* O, int B, int H, int Hkv, int N,
                             long long ldn, int D, int nsplit, hipStream_t s) {
    if (ticket == nullptr || tag == 0 || (tag & kTicketCountMask) != 0) return hipErrorInvalidValue;
    uint32_t* err = fused_error_word();
    if (err == nullptr) return hipErrorInvalidSymbol;
    AttnArgs a{Q, K, V, nullptr, nullptr, nullptr, 0, 0.0f, part, nullptr, O, B, H, Hkv, N, ldn, N, nsplit};
    a.dense_ticket = ticket;
    a.dense_tag = tag;
    a.err = err;
    return launch_dense_any(a, dtype, D, s);
}

hipError_t launch_combine(const float* part, void* O, int dtype, int BH, int D, int nsplit,
                          bool base2, hipStream_t s) {
    const unsigned grid = static_cast<unsigned>((BH + 3) / 4);
#define DCR_COMBINE_CASE(DTV, DV)                                          \
    if (dtype == DTV && D == DV) {                                         \
        if (base2)                                                         \
            launch_kernel(combine_kernel<DTV, DV, true>, grid, dim3(256), 0, s, part, O, BH, nsplit); \
        else                                                               \
            launch_kernel(combine_kernel<DTV, DV, false>, grid, dim3(256), 0, s, part, O, BH, nsplit); \
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
