// capi.hip -- extern "C" entry points of libdcr_sparse_decode.so.
//
// Argument validation, workspace carving and launch sequencing for the
// kernels in uq.hip, score.hip, select.hip and attn.hip.  The declarations
// (with the reference function each entry point replaces) are in
// include/dcr_sparse_decode.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <mutex>
#include <vector>

#include "dcr_common.h"
#include "dcr_kernels.h"
#include "dcr_sparse_decode.h"

namespace dcr {
LaunchEvents& launch_events() {
    thread_local LaunchEvents ev{nullptr, nullptr};
    return ev;
}
}  // namespace dcr

// Scratch of dcr_sparse_decode_static (see static_scratch below).
constexpr size_t kStaticScratchBytes = DCR_STATIC_SCRATCH_BYTES;
static_assert(kStaticScratchBytes % 256 == 0, "scratch is carved at 256-byte offsets");
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {

constexpr int kAbiVersion = 6;

thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return DCR_OK;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(DCR_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

hipStream_t as_stream(dcr_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

bool valid_dtype(int dtype) { return dtype == DCR_F32 || dtype == DCR_F16 || dtype == DCR_BF16; }

int check_heads(int B, int H, int Hkv, int N, int D, int dtype) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || N <= 0 || D <= 0)
        return fail(DCR_ERR_INVALID_ARG, "non-positive shape B=%d H=%d Hkv=%d N=%d D=%d", B, H, Hkv,
                    N, D);
    if (!valid_dtype(dtype)) return fail(DCR_ERR_INVALID_ARG, "unknown dtype code %d", dtype);
    if (H % Hkv != 0) return fail(DCR_ERR_INVALID_ARG, "H=%d not divisible by Hkv=%d", H, Hkv);
    const int rep = H / Hkv;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8)
        return fail(DCR_ERR_UNSUPPORTED, "n_rep=%d not in {1,2,4,8}", rep);
    if (D != 64 && D != 128) return fail(DCR_ERR_UNSUPPORTED, "D=%d not in {64,128}", D);
    if (B > 65535 || Hkv > 65535)
        return fail(DCR_ERR_UNSUPPORTED, "B=%d or Hkv=%d exceeds a grid dimension", B, Hkv);
    return DCR_OK;
}

int check_k(int N, int k) {
    if (k <= 0 || k >= N) return fail(DCR_ERR_INVALID_ARG, "k=%d must be in (0, N=%d)", k, N);
    if (N > dcr::kMaxTopkN)
        return fail(DCR_ERR_UNSUPPORTED, "N=%d exceeds the top-k limit %d", N, dcr::kMaxTopkN);
    return DCR_OK;
}

// ldn: rows between consecutive KV heads of K/V (N for a contiguous cache).
int check_ldn(int N, int ldn) {
    if (ldn < N) return fail(DCR_ERR_INVALID_ARG, "ldn=%d must be >= N=%d", ldn, N);
    return DCR_OK;
}

int check_ws(const void* ws, size_t have, size_t need) {
    if (need == 0) return DCR_OK;
    if (ws == nullptr || have < need)
        return fail(DCR_ERR_WORKSPACE, "workspace %zu bytes at %p, need %zu", have, ws, need);
    if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
        return fail(DCR_ERR_WORKSPACE, "workspace %p is not 256-byte aligned", ws);
    return DCR_OK;
}

#define DCR_REQUIRE(p) \
    if ((p) == nullptr) return fail(DCR_ERR_INVALID_ARG, "null pointer: %s", #p)

// K and V rows are read with 16-byte vector loads.
#define DCR_REQUIRE_ALIGNED16(p)                                                     \
    if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0)                                  \
    return fail(DCR_ERR_INVALID_ARG, "%s=%p is not 16-byte aligned", #p, (const void*)(p))

// Level-1 histogram slabs: rows x nslab x 256 16-bit counters.
size_t hist_bytes(size_t rows, int nslab) {
    return align256(rows * static_cast<size_t>(nslab) * dcr::kHist1Bins * sizeof(dcr::slab_t));
}

size_t part_bytes(size_t BH, int nsplit, int D) {
    return align256(BH * static_cast<size_t>(nsplit) * (D + 2) * sizeof(float));
}

// Workspace of dcr_qaxis_select (u | score keys | hist slabs | select
// scratch) and of dcr_sparse_decode (the same, then idx | score residual bytes (fp16
// and bf16 only) | partials | tickets).  k = 0: select only.
struct DecodeLayout {
    size_t u, scores, hist, selpart, idx, res, sel, part, ticket, total;
    int nslab, nsplit, usplit, ldsc;
};

// Internal score rows are padded to a multiple of 64 entries (128 bytes), so
// the score kernel and the select kernel use aligned vector accesses for any N.
int score_stride(int N) { return (N + 63) / 64 * 64; }

DecodeLayout decode_layout(int B, int H, int Hkv, int N, int D, int k, int dtype) {
    DecodeLayout L{};
    const size_t BH = static_cast<size_t>(B) * H;
    L.nslab = dcr::score_slabs(dtype, B, Hkv, N, D);
    L.nsplit = k > 0 ? dcr::attn_num_splits(B * Hkv, k) : 0;
    L.usplit = k > 0 && dtype != DCR_F32 ? dcr::union_attn_splits(N) : 0;
    L.u = 0;
    L.ldsc = score_stride(N);
    L.scores = L.u + align256(BH * D * sizeof(float));
    L.hist = L.scores + align256(BH * static_cast<size_t>(L.ldsc) * sizeof(uint16_t));
    L.selpart = L.hist + hist_bytes(BH, L.nslab);
    L.idx = L.selpart + align256(dcr::select_part_words(static_cast<int>(BH), N) * sizeof(uint32_t));
    L.res = L.idx + (k > 0 ? align256(BH * static_cast<size_t>(k) * sizeof(int32_t)) : 0);
    const bool scored = k > 0 && dtype != DCR_F32;
    L.sel = L.res + (scored ? align256(BH * static_cast<size_t>(L.ldsc) * sizeof(uint8_t)) : 0);
    L.part = L.sel + (scored ? align256(BH * 2 * sizeof(uint32_t)) : 0);
    L.ticket = L.part + (k > 0 ? part_bytes(BH, L.nsplit > L.usplit ? L.nsplit : L.usplit, D) : 0);
    L.total = L.ticket + (k > 0 ? align256(static_cast<size_t>(B) * Hkv * sizeof(uint32_t)) : 0);
    return L;
}

// Workspace of the one-launch path (fused.hip): score keys | residual bytes |
// level-1 and level-2 histogram records and the per-chunk sums, one per
// (row, position chunk) | the barrier control block.
struct FusedLayout {
    dcr::FusedShape f;
    size_t keys, res, hist1p, hist2p, part, ctl, total;
    int ldsc;
};

FusedLayout fused_layout(int B, int H, int Hkv, int N, int D, int k, int dtype) {
    FusedLayout L{};
    L.f = dcr::fused_shape(dtype, B, H, Hkv, N, D, k);
    if (!L.f.ok) return L;
    const size_t BH = static_cast<size_t>(B) * H;
    const size_t recs = BH * static_cast<size_t>(L.f.chunks);
    L.ldsc = score_stride(N);
    L.keys = 0;
    L.res = L.keys + align256(BH * static_cast<size_t>(L.ldsc) * sizeof(uint16_t));
    L.hist1p = L.res + align256(BH * static_cast<size_t>(L.ldsc));
    L.hist2p = L.hist1p + align256(recs * dcr::kHist1Bins * sizeof(uint32_t));
    L.part = L.hist2p + align256(recs * 260 * sizeof(uint32_t));
    L.ctl = L.part + align256(recs * static_cast<size_t>(D + 1) * sizeof(float));
    L.total = L.ctl + align256(sizeof(dcr::FusedCtl));
    return L;
}

// Which sparse decode path runs (dcr_set_sparse_path): the one-launch path
// where the shape and the device allow it, or always the three launches.
std::atomic<int> g_sparse_path{DCR_PATH_AUTO};

// Score kernel form (dcr_set_score_form): 0 MFMA where it fits, 1 VALU.
std::atomic<int> g_score_valu{0};

// The one-launch path needs its 256 workgroups resident at once, one per
// CU, 32 on each XCD: a 256-CU device (checked once per device).
bool device_runs_fused() {
    static std::mutex mu;
    static int cached[64];  // 0 unknown, 1 yes, 2 no
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    std::lock_guard<std::mutex> lock(mu);
    if (cached[dev] == 0) {
        int cus = 0;
        const bool ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                        cus == dcr::kFusedXcds * dcr::kFusedWgPerXcd;
        cached[dev] = ok ? 1 : 2;
    }
    return cached[dev] == 1;
}

// A different 64-bit value per call (the fused path's barrier tags hash it
// with a per-workspace launch counter).
uint64_t next_nonce() {
    static std::atomic<uint64_t> ctr{static_cast<uint64_t>(
        std::chrono::steady_clock::now().time_since_epoch().count()) ^ 0xD1B54A32D192ED03ull};
    uint64_t z = ctr.fetch_add(0x9E3779B97F4A7C15ull) + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// The dense kernel's merge-ticket tag: one nonzero value per process with the
// tickets' 20 count bits clear.
uint64_t ticket_tag() {
    static const uint64_t tag = [] {
        const uint64_t t = next_nonce() & ~((uint64_t{1} << 20) - 1);
        return t != 0 ? t : (uint64_t{1} << 63);
    }();
    return tag;
}

// ---- optional per-kernel event timing (dcr_profile_begin / dcr_profile_end)
struct ProfRecord {
    const char* name;
    hipEvent_t start, stop;
};
bool g_prof_on = false;
std::vector<ProfRecord> g_prof;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t pooled_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Runs `launch` (a callable returning hipError_t, making one kernel launch)
// with launch events attached when profiling is on.
template <typename F>
hipError_t timed(const char* name, hipStream_t, F&& launch) {
    if (!g_prof_on) return launch();
    ProfRecord r{name, pooled_event(), pooled_event()};
    dcr::LaunchEvents& ev = dcr::launch_events();
    ev = dcr::LaunchEvents{r.start, r.stop};
    const hipError_t e = launch();
    ev = dcr::LaunchEvents{nullptr, nullptr};
    if (r.start != nullptr && r.stop != nullptr) g_prof.push_back(r);
    return e;
}

template <typename T>
T* at(void* ws, size_t off) {
    return reinterpret_cast<T*>(static_cast<uint8_t*>(ws) + off);
}

// ---- static scratch of dcr_sparse_decode_static ---------------------------
// A file-scope device array: every GPU the library runs on holds its own copy
// (zero-initialised, .bss of the code object) until the process ends.  Host
// code never passes the array's name to a kernel or a copy -- on the host it
// is only a stand-in symbol -- but the device address hipGetSymbolAddress
// returns for the current device, looked up once per device and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int static_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return fail(DCR_ERR_UNSUPPORTED, "device %d outside the %d devices the static scratch tracks", dev,
                    kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255u) != 0)
            return fail(DCR_ERR_HIP, "static scratch of device %d at %p is not 256-byte aligned", dev, p);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DCR_OK;
}

// Argument checks of the sparse decode entry points (no device call).
int check_decode_args(const void* Q, const void* K, const void* V, const void* O, int dtype, int B,
                      int H, int Hkv, int N, int ldn, int D, int k) {
    DCR_REQUIRE(Q);
    DCR_REQUIRE(K);
    DCR_REQUIRE(V);
    DCR_REQUIRE(O);
    DCR_REQUIRE_ALIGNED16(K);
    DCR_REQUIRE_ALIGNED16(V);
    int rc = check_heads(B, H, Hkv, N, D, dtype);
    if (rc != DCR_OK) return rc;
    rc = check_ldn(N, ldn);
    if (rc != DCR_OK) return rc;
    return check_k(N, k);
}

// The sparse decode step -- one launch (fused.hip) where the shape and the
// device allow it, else the sequence score pass with u_Q and the level-1
// histogram, top-k select, gather + attention with the merge in the last
// workgroup of each GQA group -- on a workspace: the caller's (dcr_sparse_decode) or the
// static scratch (dcr_sparse_decode_static).  Nothing in it allocates:
// every buffer is carved from the workspace, and nothing must be
// zero on entry (the select kernel clears the merge tickets in-stream).
// Workspace bytes of the sparse decode entry points: enough for either path.
size_t sparse_decode_ws_bytes(int B, int H, int Hkv, int N, int D, int k, int dtype) {
    const size_t classic = decode_layout(B, H, Hkv, N, D, k, dtype).total;
    const FusedLayout F = fused_layout(B, H, Hkv, N, D, k, dtype);
    return F.f.ok && F.total > classic ? F.total : classic;
}

int sparse_decode_impl(const void* Q, const void* K, const void* V, int dtype, void* O,
                       int32_t* idx_out, int B, int H, int Hkv, int N, int ldn, int D, int k,
                       float eps, void* workspace, size_t workspace_bytes, dcr_stream_t stream) {
    int rc = check_decode_args(Q, K, V, O, dtype, B, H, Hkv, N, ldn, D, k);
    if (rc != DCR_OK) return rc;
    rc = check_ws(workspace, workspace_bytes, sparse_decode_ws_bytes(B, H, Hkv, N, D, k, dtype));
    if (rc != DCR_OK) return rc;
    hipStream_t s = as_stream(stream);
    const int path = g_sparse_path.load(std::memory_order_relaxed);
    if (path == DCR_PATH_FUSED) {
        const FusedLayout F = fused_layout(B, H, Hkv, N, D, k, dtype);
        if (F.f.ok && F.total <= workspace_bytes && device_runs_fused()) {
            const hipError_t e = timed("fused_kernel", s, [&] {
                return dcr::launch_fused_decode(
                    Q, K, V, dtype, O, idx_out, at<uint16_t>(workspace, F.keys), at<uint8_t>(workspace, F.res),
                    at<uint32_t>(workspace, F.hist1p), at<uint32_t>(workspace, F.hist2p),
                    at<float>(workspace, F.part), at<dcr::FusedCtl>(workspace, F.ctl), next_nonce(), eps, B, H,
                    Hkv, N, ldn, F.ldsc, D, k, F.f, s);
            });
            return e == hipSuccess ? ok() : hip_fail(e, "fused_kernel");
        }
    }
    const DecodeLayout L = decode_layout(B, H, Hkv, N, D, k, dtype);
    const size_t BH = static_cast<size_t>(B) * H;
    float* u = at<float>(workspace, L.u);
    uint16_t* keys = at<uint16_t>(workspace, L.scores);
    dcr::slab_t* hist = at<dcr::slab_t>(workspace, L.hist);
    int32_t* idx = idx_out != nullptr ? idx_out : at<int32_t>(workspace, L.idx);
    // fp16/bf16: the score pass also keeps one residual byte per score, from
    // which (with the key) the attention rebuilds the selected positions' fp32
    // dot products as its logits, so it gathers V rows only; fp32 gathers K
    // as well (its tolerance is tighter than the rebuilt logits' 2^-15).
    uint8_t* res = dtype == DCR_F32 ? nullptr : at<uint8_t>(workspace, L.res);
    float* part = at<float>(workspace, L.part);
    uint32_t* ticket = at<uint32_t>(workspace, L.ticket);

    hipError_t e = timed("score_kernel", s, [&] {
        return dcr::launch_score_fused(K, Q, dtype, eps, u, keys, res, L.ldsc, hist, B, Hkv, H / Hkv,
                                       N, D, ldn, g_score_valu.load(std::memory_order_relaxed) != 0, s);
    });
    if (e != hipSuccess) return hip_fail(e, "score_kernel");
    // DCR_PATH_UNION (fp16/bf16): the select kernel hands the attention each
    // row's selection in closed form (threshold key, last selected tie), and
    // the union-gather attention reads every V row a group selected once; the
    // index list is written only when the caller asks for it.  Otherwise the
    // attention walks the index lists.
    const bool union_gather = res != nullptr && path == DCR_PATH_UNION;
    uint32_t* sel = union_gather ? at<uint32_t>(workspace, L.sel) : nullptr;
    e = timed("select_kernel", s, [&] {
        return dcr::launch_select_keys(keys, L.ldsc, hist, L.nslab, union_gather ? idx_out : idx, sel, ticket,
                                       H / Hkv, static_cast<int>(BH), N, k, at<uint32_t>(workspace, L.selpart), s);
    });
    if (e != hipSuccess) return hip_fail(e, "select_kernel");
    if (union_gather) {
        e = timed("union_attn_kernel", s, [&] {
            return dcr::launch_union_attn(Q, V, dtype, sel, keys, res, L.ldsc, eps, part, ticket, O, B, H, Hkv, N,
                                          ldn, D, s);
        });
        return e == hipSuccess ? ok() : hip_fail(e, "union_attn_kernel");
    }
    e = timed("attn_kernel", s, [&] {
        if (res != nullptr)
            return dcr::launch_scored_attn(Q, V, dtype, idx, keys, res, L.ldsc, eps, part, ticket, O, B, H,
                                           Hkv, N, ldn, D, k, L.nsplit, s);
        return dcr::launch_sparse_attn(Q, K, V, dtype, idx, part, ticket, O, B, H, Hkv, N, ldn, D, k,
                                       L.nsplit, s);
    });
    return e == hipSuccess ? ok() : hip_fail(e, "attn_kernel");
}

}  // namespace

extern "C" {

int dcr_abi_version(void) { return kAbiVersion; }

const char* dcr_status_string(int status) {
    switch (status) {
        case DCR_OK: return "ok";
        case DCR_ERR_INVALID_ARG: return "invalid argument";
        case DCR_ERR_UNSUPPORTED: return "unsupported shape";
        case DCR_ERR_WORKSPACE: return "workspace too small";
        case DCR_ERR_HIP: return "HIP error";
        default: return "unknown status";
    }
}

const char* dcr_last_error(void) { return g_err; }

int dcr_compute_uq(const void* Q, int dtype, float* uQ, int rows, int D, float eps,
                   dcr_stream_t stream) {
    DCR_REQUIRE(Q);
    DCR_REQUIRE(uQ);
    if (rows <= 0 || D <= 0) return fail(DCR_ERR_INVALID_ARG, "rows=%d D=%d", rows, D);
    if (!valid_dtype(dtype)) return fail(DCR_ERR_INVALID_ARG, "unknown dtype code %d", dtype);
    const hipError_t e = timed("uq_kernel", as_stream(stream), [&] {
        return dcr::launch_uq(Q, dtype, uQ, rows, D, eps, nullptr, 0, as_stream(stream));
    });
    return e == hipSuccess ? ok() : hip_fail(e, "uq_kernel");
}

int dcr_score_pass(const void* K, int dtype, const float* uQ, uint16_t* scores, int B, int Hkv,
                   int n_rep, int N, int ldn, int D, dcr_stream_t stream) {
    DCR_REQUIRE(K);
    DCR_REQUIRE(uQ);
    DCR_REQUIRE(scores);
    DCR_REQUIRE_ALIGNED16(K);
    if (n_rep <= 0) return fail(DCR_ERR_INVALID_ARG, "n_rep=%d", n_rep);
    int rc = check_heads(B, Hkv * n_rep, Hkv, N, D, dtype);
    if (rc != DCR_OK) return rc;
    rc = check_ldn(N, ldn);
    if (rc != DCR_OK) return rc;
    const hipError_t e = timed("score_kernel", as_stream(stream), [&] {
        return dcr::launch_score(K, dtype, uQ, scores, B, Hkv, n_rep, N, D, ldn, as_stream(stream));
    });
    return e == hipSuccess ? ok() : hip_fail(e, "score_kernel");
}

size_t dcr_topk_select_workspace_bytes(int rows, int N) {
    if (rows <= 0 || N <= 0) return 0;
    return hist_bytes(static_cast<size_t>(rows), dcr::hist_slabs(N)) +
           align256(dcr::select_part_words(rows, N) * sizeof(uint32_t));
}

int dcr_topk_select(const uint16_t* scores, int32_t* idx, int rows, int N, int k, void* workspace,
                    size_t workspace_bytes, dcr_stream_t stream) {
    DCR_REQUIRE(scores);
    DCR_REQUIRE(idx);
    if (rows <= 0 || N <= 0) return fail(DCR_ERR_INVALID_ARG, "rows=%d N=%d", rows, N);
    int rc = check_k(N, k);
    if (rc != DCR_OK) return rc;
    rc = check_ws(workspace, workspace_bytes, dcr_topk_select_workspace_bytes(rows, N));
    if (rc != DCR_OK) return rc;
    hipStream_t s = as_stream(stream);
    dcr::slab_t* hist = static_cast<dcr::slab_t*>(workspace);
    hipError_t e = timed("hist_kernel", s, [&] { return dcr::launch_hist(scores, hist, rows, N, s); });
    if (e != hipSuccess) return hip_fail(e, "hist_kernel");
    e = timed("select_kernel", s, [&] {
        uint32_t* part = at<uint32_t>(workspace, hist_bytes(static_cast<size_t>(rows), dcr::hist_slabs(N)));
        return dcr::launch_select(scores, N, hist, dcr::hist_slabs(N), idx, nullptr, 1, rows, N, k,
                                  part, s);
    });
    return e == hipSuccess ? ok() : hip_fail(e, "select_kernel");
}

size_t dcr_gather_attn_workspace_bytes(int B, int H, int Hkv, int D, int k) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || D <= 0 || k <= 0) return 0;
    const int nsplit = dcr::attn_num_splits(B * Hkv, k);
    return part_bytes(static_cast<size_t>(B) * H, nsplit, D);
}

int dcr_gather_attn(const void* Q, const void* K, const void* V, int dtype, const int32_t* idx,
                    void* O, int B, int H, int Hkv, int N, int ldn, int D, int k,
                    void* workspace, size_t workspace_bytes, dcr_stream_t stream) {
    DCR_REQUIRE(Q);
    DCR_REQUIRE(K);
    DCR_REQUIRE(V);
    DCR_REQUIRE(idx);
    DCR_REQUIRE(O);
    DCR_REQUIRE_ALIGNED16(K);
    DCR_REQUIRE_ALIGNED16(V);
    int rc = check_heads(B, H, Hkv, N, D, dtype);
    if (rc != DCR_OK) return rc;
    rc = check_ldn(N, ldn);
    if (rc != DCR_OK) return rc;
    if (k <= 0) return fail(DCR_ERR_INVALID_ARG, "k=%d must be positive", k);
    rc = check_ws(workspace, workspace_bytes, dcr_gather_attn_workspace_bytes(B, H, Hkv, D, k));
    if (rc != DCR_OK) return rc;
    hipStream_t s = as_stream(stream);
    const int nsplit = dcr::attn_num_splits(B * Hkv, k);
    float* part = static_cast<float*>(workspace);
    hipError_t e = timed("attn_kernel", s, [&] {
        return dcr::launch_sparse_attn(Q, K, V, dtype, idx, part, nullptr, O, B, H, Hkv, N, ldn, D,
                                       k, nsplit, s);
    });
    if (e != hipSuccess) return hip_fail(e, "attn_kernel");
    e = timed("combine_kernel", s, [&] { return dcr::launch_combine(part, O, dtype, B * H, D, nsplit, false, s); });
    return e == hipSuccess ? ok() : hip_fail(e, "combine_kernel");
}

size_t dcr_qaxis_select_workspace_bytes(int B, int H, int Hkv, int N, int D, int dtype) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || N <= 0 || D <= 0 || !valid_dtype(dtype)) return 0;
    return decode_layout(B, H, Hkv, N, D, 0, dtype).total;
}

int dcr_qaxis_select(const void* Q, const void* K, int dtype, int32_t* idx, int B, int H, int Hkv,
                     int N, int ldn, int D, int k, float eps, void* workspace,
                     size_t workspace_bytes, dcr_stream_t stream) {
    DCR_REQUIRE(Q);
    DCR_REQUIRE(K);
    DCR_REQUIRE(idx);
    DCR_REQUIRE_ALIGNED16(K);
    int rc = check_heads(B, H, Hkv, N, D, dtype);
    if (rc != DCR_OK) return rc;
    rc = check_ldn(N, ldn);
    if (rc != DCR_OK) return rc;
    rc = check_k(N, k);
    if (rc != DCR_OK) return rc;
    const DecodeLayout L = decode_layout(B, H, Hkv, N, D, 0, dtype);
    rc = check_ws(workspace, workspace_bytes, L.total);
    if (rc != DCR_OK) return rc;
    hipStream_t s = as_stream(stream);
    const size_t BH = static_cast<size_t>(B) * H;
    float* u = at<float>(workspace, L.u);
    uint16_t* keys = at<uint16_t>(workspace, L.scores);
    dcr::slab_t* hist = at<dcr::slab_t>(workspace, L.hist);
    hipError_t e = timed("score_kernel", s, [&] {
        return dcr::launch_score_fused(K, Q, dtype, eps, u, keys, nullptr, L.ldsc, hist, B, Hkv,
                                       H / Hkv, N, D, ldn, g_score_valu.load(std::memory_order_relaxed) != 0, s);
    });
    if (e != hipSuccess) return hip_fail(e, "score_kernel");
    e = timed("select_kernel", s, [&] {
        return dcr::launch_select_keys(keys, L.ldsc, hist, L.nslab, idx, nullptr, nullptr, 1,
                                       static_cast<int>(BH), N, k, at<uint32_t>(workspace, L.selpart), s);
    });
    return e == hipSuccess ? ok() : hip_fail(e, "select_kernel");
}

size_t dcr_sparse_decode_workspace_bytes(int B, int H, int Hkv, int N, int D, int k, int dtype) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || N <= 0 || D <= 0 || k <= 0 || !valid_dtype(dtype)) return 0;
    return sparse_decode_ws_bytes(B, H, Hkv, N, D, k, dtype);
}

int dcr_set_sparse_path(int path) {
    if (path != DCR_PATH_AUTO && path != DCR_PATH_CLASSIC && path != DCR_PATH_FUSED && path != DCR_PATH_UNION)
        return fail(DCR_ERR_INVALID_ARG, "unknown sparse path %d", path);
    ok();
    return g_sparse_path.exchange(path);
}

int dcr_set_score_form(int form) {
    if (form != DCR_SCORE_AUTO && form != DCR_SCORE_VALU)
        return fail(DCR_ERR_INVALID_ARG, "unknown score form %d", form);
    ok();
    return g_score_valu.exchange(form == DCR_SCORE_VALU ? 1 : 0) != 0 ? DCR_SCORE_VALU : DCR_SCORE_AUTO;
}

int dcr_sparse_decode_launches(int B, int H, int Hkv, int N, int D, int k, int dtype) {
    int rc = check_heads(B, H, Hkv, N, D, dtype);
    if (rc != DCR_OK) return rc;
    rc = check_k(N, k);
    if (rc != DCR_OK) return rc;
    ok();
    if (g_sparse_path.load(std::memory_order_relaxed) != DCR_PATH_FUSED) return 3;
    return dcr::fused_shape(dtype, B, H, Hkv, N, D, k).ok && device_runs_fused() ? 1 : 3;
}

int dcr_fused_errors(int clear, unsigned* errors) {
    if (errors == nullptr) return fail(DCR_ERR_INVALID_ARG, "null pointer: errors");
    uint32_t* w = dcr::fused_error_word();
    if (w == nullptr) return fail(DCR_ERR_HIP, "fused error word: symbol not found");
    uint32_t v = 0;
    hipError_t e = hipMemcpy(&v, w, sizeof v, hipMemcpyDeviceToHost);
    if (e == hipSuccess && clear) {
        const uint32_t zero = 0;
        e = hipMemcpy(w, &zero, sizeof zero, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) return hip_fail(e, "dcr_fused_errors");
    *errors = v;
    return ok();
}

int dcr_sparse_decode(const void* Q, const void* K, const void* V, int dtype, void* O,
                      int32_t* idx_out, int B, int H, int Hkv, int N, int ldn, int D, int k,
                      float eps, void* workspace, size_t workspace_bytes, dcr_stream_t stream) {
    return sparse_decode_impl(Q, K, V, dtype, O, idx_out, B, H, Hkv, N, ldn, D, k, eps, workspace,
                              workspace_bytes, stream);
}

int dcr_sparse_decode_static(const void* Q, const void* K, const void* V, int dtype, void* O,
                             int32_t* idx_out, int B, int H, int Hkv, int N, int ldn, int D, int k,
                             float eps, dcr_stream_t stream) {
    int rc = check_decode_args(Q, K, V, O, dtype, B, H, Hkv, N, ldn, D, k);
    if (rc != DCR_OK) return rc;
    const size_t need = sparse_decode_ws_bytes(B, H, Hkv, N, D, k, dtype);
    if (need > kStaticScratchBytes)
        return fail(DCR_ERR_WORKSPACE,
                    "B=%d H=%d Hkv=%d N=%d D=%d k=%d needs %zu bytes of scratch, more than the static "
                    "scratch's %zu (DCR_STATIC_SCRATCH_BYTES); call dcr_sparse_decode with a workspace",
                    B, H, Hkv, N, D, k, need, kStaticScratchBytes);
    void* ws = nullptr;
    rc = static_scratch(&ws);
    if (rc != DCR_OK) return rc;
    return sparse_decode_impl(Q, K, V, dtype, O, idx_out, B, H, Hkv, N, ldn, D, k, eps, ws,
                              kStaticScratchBytes, stream);
}

// Dense workspace: partials | the groups' merge tickets (64-bit words).
size_t dcr_dense_decode_workspace_bytes(int B, int H, int Hkv, int N, int D) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || N <= 0 || D <= 0) return 0;
    const int nsplit = dcr::dense_num_splits(B * Hkv, N);
    return part_bytes(static_cast<size_t>(B) * H, nsplit, D) +
           align256(static_cast<size_t>(B) * Hkv * sizeof(uint64_t));
}

int dcr_dense_decode(const void* Q, const void* K, const void* V, int dtype, void* O, int B, int H,
                     int Hkv, int N, int ldn, int D, void* workspace, size_t workspace_bytes,
                     dcr_stream_t stream) {
    DCR_REQUIRE(Q);
    DCR_REQUIRE(K);
    DCR_REQUIRE(V);
    DCR_REQUIRE(O);
    DCR_REQUIRE_ALIGNED16(K);
    DCR_REQUIRE_ALIGNED16(V);
    int rc = check_heads(B, H, Hkv, N, D, dtype);
    if (rc != DCR_OK) return rc;
    rc = check_ldn(N, ldn);
    if (rc != DCR_OK) return rc;
    rc = check_ws(workspace, workspace_bytes, dcr_dense_decode_workspace_bytes(B, H, Hkv, N, D));
    if (rc != DCR_OK) return rc;
    hipStream_t s = as_stream(stream);
    const int nsplit = dcr::dense_num_splits(B * Hkv, N);
    float* part = static_cast<float*>(workspace);
    uint64_t* ticket = at<uint64_t>(workspace, part_bytes(static_cast<size_t>(B) * H, nsplit, D));
    const hipError_t e = timed("dense_attn_kernel", s, [&] {
        return dcr::launch_dense_attn(Q, K, V, dtype, part, ticket, ticket_tag(), O, B, H, Hkv, N, ldn, D, nsplit,
                                      s);
    });
    return e == hipSuccess ? ok() : hip_fail(e, "attn_kernel(dense)");
}

int dcr_rank_local_fwd(const void* Q, const void* K_sorted, const void* V_sorted, int dtype,
                       const int32_t* r_center, void* O, float* lse, int BH, int Nq, int Nkv,
                       int D, int k_window, float scale, dcr_stream_t stream) {
    DCR_REQUIRE(Q);
    DCR_REQUIRE(K_sorted);
    DCR_REQUIRE(V_sorted);
    DCR_REQUIRE(r_center);
    DCR_REQUIRE(O);
    DCR_REQUIRE(lse);
    DCR_REQUIRE_ALIGNED16(K_sorted);
    DCR_REQUIRE_ALIGNED16(V_sorted);
    if (BH <= 0 || Nq <= 0 || Nkv <= 0 || D <= 0)
        return fail(DCR_ERR_INVALID_ARG, "non-positive shape BH=%d Nq=%d Nkv=%d D=%d", BH, Nq, Nkv, D);
    if (!valid_dtype(dtype)) return fail(DCR_ERR_INVALID_ARG, "unknown dtype code %d", dtype);
    if (k_window < 0) return fail(DCR_ERR_INVALID_ARG, "k_window=%d must be >= 0", k_window);
    if (D != 32 && D != 64 && D != 128) return fail(DCR_ERR_UNSUPPORTED, "D=%d not in {32,64,128}", D);
    if (BH > 65535) return fail(DCR_ERR_UNSUPPORTED, "BH=%d exceeds a grid dimension", BH);
    // The kernels form r +- half_k in 64 bits, so half_k is passed as given.
    const int half_k = k_window / 2;
    hipStream_t s = as_stream(stream);
    const hipError_t e = timed("rank_local_kernel", s, [&] {
        return dcr::launch_rank_local(Q, K_sorted, V_sorted, dtype, r_center, O, lse, BH, Nq, Nkv, D,
                                      half_k, scale, nullptr, Nkv, 1, 1, s);
    });
    return e == hipSuccess ? ok() : hip_fail(e, "rank_local_kernel");
}

int dcr_rank_local_fwd_gather(const void* Q, const void* K, const void* V, int dtype,
                              const int32_t* perm, const int32_t* r_center, void* O, float* lse, int B,
                              int H, int Hkv, int Nq, int Nkv, int ldn, int D, int k_window, float scale,
                              dcr_stream_t stream) {
    DCR_REQUIRE(Q);
    DCR_REQUIRE(K);
    DCR_REQUIRE(V);
    DCR_REQUIRE(perm);
    DCR_REQUIRE(r_center);
    DCR_REQUIRE(O);
    DCR_REQUIRE(lse);
    DCR_REQUIRE_ALIGNED16(K);
    DCR_REQUIRE_ALIGNED16(V);
    if (B <= 0 || H <= 0 || Hkv <= 0 || Nq <= 0 || Nkv <= 0 || D <= 0)
        return fail(DCR_ERR_INVALID_ARG, "non-positive shape B=%d H=%d Hkv=%d Nq=%d Nkv=%d D=%d", B, H, Hkv, Nq,
                    Nkv, D);
    if (H % Hkv != 0) return fail(DCR_ERR_INVALID_ARG, "H=%d is not a multiple of Hkv=%d", H, Hkv);
    if (ldn < Nkv) return fail(DCR_ERR_INVALID_ARG, "ldn=%d < Nkv=%d", ldn, Nkv);
    if (!valid_dtype(dtype)) return fail(DCR_ERR_INVALID_ARG, "unknown dtype code %d", dtype);
    if (k_window < 0) return fail(DCR_ERR_INVALID_ARG, "k_window=%d must be >= 0", k_window);
    if (D != 32 && D != 64 && D != 128) return fail(DCR_ERR_UNSUPPORTED, "D=%d not in {32,64,128}", D);
    const long long BH = static_cast<long long>(B) * H;
    if (BH > 65535) return fail(DCR_ERR_UNSUPPORTED, "B*H=%lld exceeds a grid dimension", BH);
    const int half_k = k_window / 2;
    hipStream_t s = as_stream(stream);
    const hipError_t e = timed("rank_local_kernel", s, [&] {
        return dcr::launch_rank_local(Q, K, V, dtype, r_center, O, lse, static_cast<int>(BH), Nq, Nkv, D, half_k,
                                      scale, perm, ldn, H, H / Hkv, s);
    });
    return e == hipSuccess ? ok() : hip_fail(e, "rank_local_kernel");
}

int dcr_profile_begin(void) {
    if (g_prof_on) return fail(DCR_ERR_INVALID_ARG, "profiling already enabled");
    g_prof.clear();
    g_prof_on = true;
    return ok();
}

int dcr_profile_end(const char** names, double* total_us, int* launches, int max) {
    if (!g_prof_on) return fail(DCR_ERR_INVALID_ARG, "profiling not enabled");
    g_prof_on = false;
    int n = 0;
    int rc = DCR_OK;
    for (const ProfRecord& r : g_prof) {
        float ms = 0.0f;
        hipError_t e = hipEventSynchronize(r.stop);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.start, r.stop);
        if (e != hipSuccess) rc = hip_fail(e, "dcr_profile_end");
        int slot = -1;
        for (int i = 0; i < n; ++i)
            if (strcmp(names[i], r.name) == 0) slot = i;
        if (slot < 0 && n < max) {
            slot = n++;
            names[slot] = r.name;
            total_us[slot] = 0.0;
            launches[slot] = 0;
        }
        if (slot >= 0) {
            total_us[slot] += 1000.0 * static_cast<double>(ms);
            launches[slot] += 1;
        }
        g_event_pool.push_back(r.start);
        g_event_pool.push_back(r.stop);
    }
    g_prof.clear();
    if (rc != DCR_OK) return rc;
    ok();
    return n;
}

}  // extern "C"
