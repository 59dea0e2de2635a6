// wf_abi.cpp -- extern "C" entry points of libwayfinder_hip.so (declared in
// include/wayfinder_hip.h): argument validation, workspace sizing, kernel dispatch and
// error reporting. Validation runs before any HIP call, so contract errors surface as
// status codes on machines without a GPU too.
#include "wayfinder_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "wf_internal.h"

namespace wf {

namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];
}  // namespace

int device_cu_count()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;   // MI355X; only the dispatch order depends on it
    g_cu_count[dev].store(n, std::memory_order_relaxed);
    return n;
}

int64_t resident_workgroups(const void* kernel, int block)
{
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    return int64_t(per_cu) * device_cu_count();
}

}  // namespace wf

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok()
{
    g_last_error.clear();
    return WF_OK;
}

size_t elem_size(int dtype) { return dtype == WF_DTYPE_F32 ? 4 : 2; }

bool valid_dtype(int dtype)
{
    return dtype == WF_DTYPE_F32 || dtype == WF_DTYPE_F16 || dtype == WF_DTYPE_BF16;
}

// 16-byte vector access is legal for every row when the innermost stride is 1, the row
// length is a multiple of 8 elements and every other stride and the base keep 16-byte
// alignment.
bool vec_ok(const void* base, int dtype, const int64_t* strides, int ndim, int64_t inner)
{
    const size_t es = elem_size(dtype);
    if (strides[ndim - 1] != 1 || inner % 8 != 0) return false;
    if (reinterpret_cast<uintptr_t>(base) % 16 != 0) return false;
    for (int i = 0; i < ndim - 1; ++i)
        if ((strides[i] * int64_t(es)) % 16 != 0) return false;
    return true;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int64_t gcd64(int64_t a, int64_t b)
{
    while (b) { const int64_t t = a % b; a = b; b = t; }
    return a;
}

// Speculative screening threshold of the retrieval: each row block estimates, from a strided
// sample of its key prefix, a threshold that about kSeedAlpha * k_eff keys of the prefix reach,
// screens with it, and checks every row exactly afterwards (rows that fail are screened again
// from -inf in the same workgroup). WAYFINDER_TOPK_SEED_ALPHA overrides it (0 turns the seed
// off: every row then starts at -inf, as the reference's streaming top-K does).
constexpr float kSeedAlpha = 3.0f;

float seed_alpha()   // read at every launch: a caller may change it between calls
{
    const char* e = std::getenv("WAYFINDER_TOPK_SEED_ALPHA");
    if (!e || !*e) return kSeedAlpha;
    const float v = std::strtof(e, nullptr);
    return v > 1.0f ? v : 0.0f;
}

constexpr int64_t kMaxTopK = 512;
constexpr int64_t kMaxR = 256;
constexpr int64_t kMaxD = 256;
constexpr int64_t kMaxReadoutK = 1024;

int check_topk(const void* query, const void* key, int dtype, int64_t B, int64_t T, int64_t R,
               const int64_t* qs, const int64_t* ks, int64_t top_k, const int32_t* out_idx)
{
    if (!valid_dtype(dtype)) return fail(WF_ERR_UNSUPPORTED, "causal_topk: unsupported dtype code %d", dtype);
    if (B < 0 || T < 0 || R < 1) return fail(WF_ERR_INVALID_ARGUMENT, "causal_topk: bad shape (B=%lld, T=%lld, R=%lld)", (long long)B, (long long)T, (long long)R);
    if (top_k < 0) return fail(WF_ERR_INVALID_ARGUMENT, "causal_topk: top_k must be >= 0, got %lld", (long long)top_k);
    if (T >= (int64_t(1) << 31) - 1) return fail(WF_ERR_UNSUPPORTED, "causal_topk: T=%lld does not fit int32 indices", (long long)T);
    if (R > kMaxR) return fail(WF_ERR_UNSUPPORTED, "causal_topk: address dim R=%lld > %lld", (long long)R, (long long)kMaxR);
    if (!qs || !ks) return fail(WF_ERR_INVALID_ARGUMENT, "causal_topk: stride arrays must not be NULL");
    const int64_t k_eff = std::min(top_k, T);
    if (k_eff > kMaxTopK) return fail(WF_ERR_UNSUPPORTED, "causal_topk: k_eff=%lld > %lld", (long long)k_eff, (long long)kMaxTopK);
    if (B > 0 && k_eff > 0 && (!query || !key || !out_idx))
        return fail(WF_ERR_INVALID_ARGUMENT, "causal_topk: NULL query/key/out_idx pointer");
    return WF_OK;
}

int check_readout(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H,
                  int64_t T, int64_t D, const int64_t* qs, const int64_t* ks, const int64_t* vs,
                  const int32_t* idx, const int64_t* is, int64_t K, const void* out,
                  const int64_t* os)
{
    if (!valid_dtype(dtype)) return fail(WF_ERR_UNSUPPORTED, "sparse_readout: unsupported dtype code %d", dtype);
    if (B < 0 || H < 0 || T < 0 || D < 1) return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout: bad shape (B=%lld, H=%lld, T=%lld, D=%lld)", (long long)B, (long long)H, (long long)T, (long long)D);
    if (D > kMaxD) return fail(WF_ERR_UNSUPPORTED, "sparse_readout: head_dim %lld > %lld", (long long)D, (long long)kMaxD);
    if (K < 1) return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout: K must be >= 1, got %lld", (long long)K);
    if (K > kMaxReadoutK) return fail(WF_ERR_UNSUPPORTED, "sparse_readout: K=%lld > %lld", (long long)K, (long long)kMaxReadoutK);
    if (T >= (int64_t(1) << 31) - 1) return fail(WF_ERR_UNSUPPORTED, "sparse_readout: T=%lld does not fit int32 indices", (long long)T);
    if (!qs || !ks || !vs || !is || !os) return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout: stride arrays must not be NULL");
    if (B * H * T > 0 && (!q || !k || !v || !idx || !out))
        return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout: NULL tensor pointer");
    return WF_OK;
}

int hip_fail(const char* what, hipError_t e)
{
    return fail(WF_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool topk_prepare(const void* query, const void* key, int dtype, int64_t B, int64_t T, int64_t R,
                  const int64_t* qs, const int64_t* ks, int64_t k_eff, int32_t* out_idx,
                  float* out_scores, void* ws, wf::TopkParams& p)
{
    p = wf::TopkParams{};
    p.query = query; p.key = key;
    p.qsb = qs[0]; p.qst = qs[1]; p.qsr = qs[2];
    p.ksb = ks[0]; p.kst = ks[1]; p.ksr = ks[2];
    p.B = B; p.T = T; p.R = R; p.k_eff = k_eff;
    p.out_idx = out_idx; p.out_scores = out_scores;
    p.chunk_absmax = static_cast<float*>(ws);
    p.n_chunks = cdiv(T, wf::kAbsmaxChunk);
    p.n_row_blocks = cdiv(T, 16);
    p.rb_begin = 0;
    p.rb_end = p.n_row_blocks;
    p.n_cus = wf::device_cu_count();
    p.seed_alpha = seed_alpha();
    // vector loads; key rows are addressed with 32-bit byte offsets from the batch base and
    // every 32-dim chunk the kernel reads lies inside the row (R = 32, 64, 128 or 256)
    return (R == 32 || R == 64 || R == 128 || R == 256) &&
           vec_ok(query, dtype, qs, 3, R) && vec_ok(key, dtype, ks, 3, R) &&
           ks[1] >= 0 && (T - 1) * ks[1] * int64_t(elem_size(dtype)) + R * int64_t(elem_size(dtype)) < (int64_t(1) << 32);
}

int check_topk_ws(int64_t B, int64_t T, int64_t R, int64_t top_k, void* ws, size_t ws_bytes)
{
    const size_t need = wf_causal_topk_workspace_bytes(B, T, R, top_k);
    if (!ws || ws_bytes < need)
        return fail(WF_ERR_WORKSPACE, "causal_topk: workspace of %zu bytes required, got %zu", need, ws ? ws_bytes : size_t(0));
    if (reinterpret_cast<uintptr_t>(ws) % 4 != 0) return fail(WF_ERR_INVALID_ARGUMENT, "causal_topk: workspace not 4-byte aligned");
    return WF_OK;
}

int run_topk(const void* query, const void* key, int dtype, int64_t B, int64_t T, int64_t R,
             const int64_t* qs, const int64_t* ks, int64_t top_k, int32_t* out_idx,
             float* out_scores, void* ws, size_t ws_bytes, hipStream_t stream)
{
    const int64_t k_eff = std::min(top_k, T);
    if (B == 0 || k_eff == 0) return WF_OK;
    const int rc = check_topk_ws(B, T, R, top_k, ws, ws_bytes);
    if (rc != WF_OK) return rc;
    wf::TopkParams p;
    const bool vec = topk_prepare(query, key, dtype, B, T, R, qs, ks, k_eff, out_idx, out_scores, ws, p);
    hipError_t e = wf::launch_key_absmax(dtype, vec, p, stream);
    if (e != hipSuccess) return hip_fail("causal_topk: key magnitude kernel launch", e);
    e = wf::launch_causal_topk(dtype, vec, p, stream);
    if (e != hipSuccess) return hip_fail("causal_topk: retrieval kernel launch", e);
    return WF_OK;
}

// Point a readout launch at query rows [r0, r1): split each (b, h) pair into row segments
// so that the number of virtual pairs is a multiple of the 8 XCDs. False if too large.
bool readout_rows(wf::ReadoutParams& p, int64_t r0, int64_t r1)
{
    const int64_t nbh = p.B * p.H;
    p.row_begin = r0;
    p.row_end = r1;
    p.seg_per_pair = 8 / gcd64(nbh, 8);
    p.rows_per_seg = cdiv(r1 - r0, p.seg_per_pair);
    p.vpairs = nbh * p.seg_per_pair;
    p.wg_per_vpair = cdiv(p.rows_per_seg, wf::kReadoutRowsPerWG);
    p.head_major = 0;   // the launcher decides from the kernel's occupancy
    return p.vpairs * p.wg_per_vpair < (int64_t(1) << 31);
}

// Readout parameters for query rows [row_begin, row_end); returns false if the problem is
// too large for one launch. *fast selects the aligned kernel.
bool readout_prepare(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H,
                     int64_t T, int64_t D, const int64_t* qs, const int64_t* ks, const int64_t* vs,
                     const int32_t* idx, const int64_t* is, int64_t K, float scale, unsigned flags,
                     void* out, const int64_t* os, float* lse2, wf::ReadoutParams& p, bool* vec,
                     bool* fast)
{
    p = wf::ReadoutParams{};
    p.q = q; p.k = k; p.v = v; p.out = out; p.idx = idx; p.lse2 = lse2;
    for (int i = 0; i < 4; ++i) { p.qs[i] = qs[i]; p.ks[i] = ks[i]; p.vs[i] = vs[i]; p.os[i] = os[i]; }
    for (int i = 0; i < 3; ++i) p.is[i] = is[i];
    p.B = B; p.H = H; p.T = T; p.D = D; p.K = K;
    p.scale = scale; p.flags = flags;
    *vec = vec_ok(q, dtype, qs, 4, D) && vec_ok(k, dtype, ks, 4, D) && vec_ok(v, dtype, vs, 4, D) &&
           vec_ok(out, dtype, os, 4, D);
    // fast path: 32-bit byte offsets cover each (b, h) span of q/k/v/out, contiguous index
    // rows, non-negative row strides
    const int64_t es = int64_t(elem_size(dtype));
    auto span_ok = [&](const int64_t* st) {
        return st[2] >= 0 && (T - 1) * st[2] * es + D * es < (int64_t(1) << 32);
    };
    // the fast kernel forms row offsets with 24-bit multiplies
    const bool mul24 = T <= (int64_t(1) << 24) && ks[2] * es < (int64_t(1) << 24) && vs[2] * es < (int64_t(1) << 24);
    *fast = *vec && is[2] == 1 && span_ok(qs) && span_ok(ks) && span_ok(vs) && span_ok(os) && mul24;
    return readout_rows(p, 0, T);
}

// Dropout parameters for probability p (0 < p < 1) and a 64-bit seed: keep iff hash >= thresh,
// thresh = round(p * 2^32), so P(keep) = 1 - thresh / 2^32.
wf::DropoutParams make_dropout(float prob, uint64_t seed)
{
    wf::DropoutParams d{};
    const double t = std::floor(double(prob) * 4294967296.0 + 0.5);
    d.thresh = uint32_t(std::min(t, 4294967295.0));
    d.k0 = uint32_t(seed);
    d.k1 = uint32_t(seed >> 32);
    d.scale = 1.0f / (1.0f - prob);
    return d;
}

int run_readout(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H,
                int64_t T, int64_t D, const int64_t* qs, const int64_t* ks, const int64_t* vs,
                const int32_t* idx, const int64_t* is, int64_t K, float scale, unsigned flags,
                void* out, const int64_t* os, float* lse2, hipStream_t stream,
                const wf::DropoutParams* drop = nullptr)
{
    if (B * H * T == 0) return WF_OK;
    wf::ReadoutParams p;
    bool vec, fast;
    if (!readout_prepare(q, k, v, dtype, B, H, T, D, qs, ks, vs, idx, is, K, scale, flags, out, os,
                         lse2, p, &vec, &fast))
        return fail(WF_ERR_UNSUPPORTED, "sparse_readout: problem too large for one launch");
    if (drop) {
        p.drop_on = 1;
        p.drop = *drop;
    }
    const hipError_t e = wf::launch_sparse_readout(dtype, vec, fast, p, stream);
    if (e != hipSuccess) return hip_fail("sparse_readout: kernel launch", e);
    return WF_OK;
}

// ---- scratch of the entry point that allocates nothing (wf_fused_topk_sparse_fwd_noalloc)
// The fused forward's only scratch is the retrieval's per-chunk key magnitude bounds:
// B * ceil(T / 256) floats, every one written by the magnitude kernel before the retrieval
// reads it, so nothing needs clearing. Each device holds its own copy of this array until
// the process ends; calls that overlap on one device share it and race.
constexpr size_t kScratchBytes = size_t(1) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
void* g_scratch_ptr[kMaxScratchDevices];
hipError_t g_scratch_err[kMaxScratchDevices];
std::once_flag g_scratch_once[kMaxScratchDevices];

// Device address of `scratch` on the current device, looked up once per device with that
// device current. The array's name is only a host-side handle; kernels get this address.
int scratch_for_current_device(void** out)
{
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail("fused_noalloc: hipGetDevice", e);
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(WF_ERR_UNSUPPORTED, "fused_noalloc: device %d beyond the %d supported", dev, kMaxScratchDevices);
    std::call_once(g_scratch_once[dev], [dev] {
        void* ptr = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? ptr : nullptr;
    });
    if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev])
        return hip_fail("fused_noalloc: hipGetSymbolAddress(scratch)", g_scratch_err[dev]);
    *out = g_scratch_ptr[dev];
    return WF_OK;
}

// Whether the fused forward takes the single-pass kernel where it applies and no flag forces
// a mode (measured against the split path at configs 3, 4 and 5).
constexpr bool kSinglePassDefault = false;

// Validation and launches of the fused forward with the workspace `ws` (the caller's, or
// the library's own scratch for the entry point that allocates nothing).
int fused_run(const wf_fused_args* a, void* ws, size_t ws_bytes, hipStream_t s)
{
    if (!a) return fail(WF_ERR_INVALID_ARGUMENT, "fused: NULL argument struct");
    int rc = check_topk(a->q_search, a->k_search, a->search_dtype, a->B, a->T, a->R,
                        a->qs_strides, a->ks_strides, a->top_k, a->out_idx);
    if (rc != WF_OK) return rc;
    const int64_t B = a->B, T = a->T, H = a->H;
    const int64_t k_eff = std::min(a->top_k, T);
    if (k_eff < 1 && B * T > 0)
        return fail(WF_ERR_INVALID_ARGUMENT, "fused: top_k must be >= 1 (empty selections have no readout)");
    const int64_t is[3] = {T * k_eff, k_eff, 1};
    rc = check_readout(a->q, a->k, a->v, a->dtype, B, H, T, a->D, a->q_strides,
                       a->k_strides, a->v_strides, a->out_idx, is, k_eff > 0 ? k_eff : 1, a->out,
                       a->out_strides);
    if (rc != WF_OK) return rc;
    if (B * T == 0) return WF_OK;
    rc = check_topk_ws(B, T, a->R, a->top_k, ws, ws_bytes);
    if (rc != WF_OK) return rc;

    wf::TopkParams tp;
    const bool tvec = topk_prepare(a->q_search, a->k_search, a->search_dtype, B, T, a->R, a->qs_strides,
                                   a->ks_strides, k_eff, a->out_idx, a->out_scores, ws, tp);
    // the readout's indices are written by the retrieval just before: all in [0, T)
    wf::ReadoutParams rp;
    bool rvec = false, rfast = false;
    if (H > 0 && !readout_prepare(a->q, a->k, a->v, a->dtype, B, H, T, a->D, a->q_strides, a->k_strides,
                                  a->v_strides, a->out_idx, is, k_eff, a->scale,
                                  (a->flags & WF_FLAG_MASK_PADS) | wf::kFlagTrustedIndices, a->out,
                                  a->out_strides, nullptr, rp, &rvec, &rfast))
        return fail(WF_ERR_UNSUPPORTED, "fused: problem too large for one launch");

    // single pass (one kernel: retrieval, then the block's rows read out for every head) or
    // split (retrieval kernel, then readout kernel); WF_FLAG_SPLIT_PASS / WF_FLAG_SINGLE_PASS
    // force one, otherwise kSinglePassDefault decides where both apply
    wf::FusedReadoutParams fr{};
    fr.q = a->q; fr.k = a->k; fr.v = a->v; fr.out = a->out;
    for (int i = 0; i < 4; ++i) {
        fr.qs[i] = a->q_strides[i]; fr.ks[i] = a->k_strides[i];
        fr.vs[i] = a->v_strides[i]; fr.os[i] = a->out_strides[i];
    }
    fr.H = H; fr.D = a->D; fr.scale = a->scale; fr.flags = a->flags & WF_FLAG_MASK_PADS;
    const bool single_ok = H > 0 && a->dtype == a->search_dtype && rvec &&
                           wf::fused_single_pass_supported(a->dtype, tvec, tp, fr);
    const unsigned mode = a->flags & (WF_FLAG_SPLIT_PASS | WF_FLAG_SINGLE_PASS);
    if (mode == (WF_FLAG_SPLIT_PASS | WF_FLAG_SINGLE_PASS))
        return fail(WF_ERR_INVALID_ARGUMENT, "fused: WF_FLAG_SPLIT_PASS and WF_FLAG_SINGLE_PASS are exclusive");
    if (mode == WF_FLAG_SINGLE_PASS && !single_ok)
        return fail(WF_ERR_UNSUPPORTED, "fused: the single-pass kernel needs bf16 addresses and q/k/v, R = 32, "
                                        "64 < k_eff <= 256, D in {64, 128}, H * D in {512, 1024} and 16-byte "
                                        "aligned rows with a contiguous head dim");
    const bool single = mode == WF_FLAG_SINGLE_PASS || (mode == 0 && single_ok && kSinglePassDefault);

    hipError_t e = wf::launch_key_absmax(a->search_dtype, tvec, tp, s);
    if (e != hipSuccess) return hip_fail("fused: key magnitude kernel launch", e);
    if (single) {
        e = wf::launch_fused_single_pass(a->dtype, tp, fr, s);
        if (e != hipSuccess) return hip_fail("fused: single-pass kernel launch", e);
        return WF_OK;
    }
    e = wf::launch_causal_topk(a->search_dtype, tvec, tp, s);
    if (e != hipSuccess) return hip_fail("fused: retrieval kernel launch", e);
    if (H == 0) return WF_OK;   // no heads: the indices are still the result's second half
    e = wf::launch_sparse_readout(a->dtype, rvec, rfast, rp, s);
    if (e != hipSuccess) return hip_fail("fused: readout kernel launch", e);
    return WF_OK;
}

int readout_bwd(const wf_readout_bwd_args* a, const wf::DropoutParams* drop, void* stream)
{
    if (!a) return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout_bwd: NULL argument struct");
    int rc = check_readout(a->q, a->k, a->v, a->dtype, a->B, a->H, a->T, a->D, a->q_strides,
                           a->k_strides, a->v_strides, a->indices, a->idx_strides, a->K, a->dout,
                           a->dout_strides);
    if (rc != WF_OK) return rc;
    const int64_t B = a->B, H = a->H, T = a->T, D = a->D, K = a->K;
    if (B * H * T == 0) return ok();
    if (!a->dq || !a->dk || !a->dv || !a->lse2)
        return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout_bwd: NULL dq/dk/dv/lse2 pointer");
    if (B * T * K >= (int64_t(1) << 32) - 1 || B * T >= (int64_t(1) << 32) - 1)
        return fail(WF_ERR_UNSUPPORTED, "sparse_readout_bwd: B*T*K=%lld exceeds 32-bit list offsets", (long long)(B * T * K));
    const int dt = a->dtype;
    const int64_t es = int64_t(elem_size(dt));
    auto fast_ok = [&](const void* base, const int64_t* st) {
        return vec_ok(base, dt, st, 4, D) && st[2] >= 0 && (T - 1) * st[2] * es + D * es < (int64_t(1) << 32);
    };
    if (!(fast_ok(a->q, a->q_strides) && fast_ok(a->k, a->k_strides) && fast_ok(a->v, a->v_strides) &&
          fast_ok(a->dout, a->dout_strides) && fast_ok(a->dq, a->dq_strides) &&
          fast_ok(a->dk, a->dk_strides) && fast_ok(a->dv, a->dv_strides)))
        return fail(WF_ERR_UNSUPPORTED, "sparse_readout_bwd: every (B,H,T,D) tensor needs a contiguous head dim, "
                                        "16-byte aligned rows and a per-(b,h) span below 4 GiB");
    if (a->idx_strides[2] != 1)
        return fail(WF_ERR_UNSUPPORTED, "sparse_readout_bwd: index rows must be contiguous (idx_strides[2] == 1)");
    const size_t need = wf::sparse_readout_bwd_workspace(B, H, T, K);
    if (!a->workspace || a->workspace_bytes < need)
        return fail(WF_ERR_WORKSPACE, "sparse_readout_bwd: workspace of %zu bytes required, got %zu", need,
                    a->workspace ? a->workspace_bytes : size_t(0));
    if (reinterpret_cast<uintptr_t>(a->workspace) % 256 != 0)
        return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout_bwd: workspace not 256-byte aligned");
    wf::ReadoutBwdParams p{};
    p.q = a->q; p.k = a->k; p.v = a->v; p.dout = a->dout;
    p.dq = a->dq; p.dk = a->dk; p.dv = a->dv;
    p.idx = a->indices; p.lse2 = a->lse2;
    for (int i = 0; i < 4; ++i) {
        p.qs[i] = a->q_strides[i]; p.ks[i] = a->k_strides[i]; p.vs[i] = a->v_strides[i];
        p.gs[i] = a->dout_strides[i]; p.dqs[i] = a->dq_strides[i]; p.dks[i] = a->dk_strides[i];
        p.dvs[i] = a->dv_strides[i];
    }
    for (int i = 0; i < 3; ++i) p.is[i] = a->idx_strides[i];
    p.B = B; p.H = H; p.T = T; p.D = D; p.K = K;
    p.scale = a->scale; p.flags = a->flags & WF_FLAG_MASK_PADS;
    const int64_t nbh = B * H;
    p.row_begin = 0;
    p.row_end = T;
    p.seg_per_pair = 8 / gcd64(nbh, 8);
    p.rows_per_seg = cdiv(T, p.seg_per_pair);
    p.vpairs = nbh * p.seg_per_pair;
    p.wg_per_vpair = cdiv(p.rows_per_seg, wf::kReadoutRowsPerWG);
    if (p.vpairs * p.wg_per_vpair >= (int64_t(1) << 31))
        return fail(WF_ERR_UNSUPPORTED, "sparse_readout_bwd: problem too large for one launch");
    if (drop) {
        p.drop_on = 1;
        p.drop = *drop;
    }
    const hipError_t e = wf::launch_sparse_readout_bwd(dt, p, a->workspace, a->workspace_bytes,
                                                       static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("sparse_readout_bwd: launch", e);
    return ok();
}

}  // namespace

extern "C" {

int wf_abi_version(void) { return WF_ABI_VERSION; }

const char* wf_last_error(void) { return g_last_error.c_str(); }

size_t wf_causal_topk_workspace_bytes(int64_t B, int64_t T, int64_t R, int64_t top_k)
{
    (void)R;
    (void)top_k;
    if (B <= 0 || T <= 0) return 0;
    return align256(size_t(B) * size_t(cdiv(T, wf::kAbsmaxChunk)) * sizeof(float));
}

size_t wf_fused_workspace_bytes(int64_t B, int64_t T, int64_t R, int64_t top_k)
{
    return wf_causal_topk_workspace_bytes(B, T, R, top_k);
}

int wf_causal_topk_fwd(const void* query, const void* key, int dtype, int64_t B, int64_t T,
                       int64_t R, const int64_t* q_strides, const int64_t* k_strides,
                       int64_t top_k, int32_t* out_idx, float* out_scores, void* workspace,
                       size_t workspace_bytes, void* stream)
{
    int rc = check_topk(query, key, dtype, B, T, R, q_strides, k_strides, top_k, out_idx);
    if (rc != WF_OK) return rc;
    rc = run_topk(query, key, dtype, B, T, R, q_strides, k_strides, top_k, out_idx, out_scores,
                  workspace, workspace_bytes, static_cast<hipStream_t>(stream));
    return rc == WF_OK ? ok() : rc;
}

int wf_sparse_readout_fwd(const void* q, const void* k, const void* v, int dtype, int64_t B,
                          int64_t H, int64_t T, int64_t D, const int64_t* q_strides,
                          const int64_t* k_strides, const int64_t* v_strides,
                          const int32_t* indices, const int64_t* idx_strides, int64_t K,
                          float scale, unsigned flags, void* out, const int64_t* out_strides,
                          void* stream)
{
    int rc = check_readout(q, k, v, dtype, B, H, T, D, q_strides, k_strides, v_strides, indices,
                           idx_strides, K, out, out_strides);
    if (rc != WF_OK) return rc;
    rc = run_readout(q, k, v, dtype, B, H, T, D, q_strides, k_strides, v_strides, indices,
                     idx_strides, K, scale, flags & WF_FLAG_MASK_PADS, out, out_strides, nullptr,
                     static_cast<hipStream_t>(stream));
    return rc == WF_OK ? ok() : rc;
}

int wf_sparse_readout_fwd_lse(const void* q, const void* k, const void* v, int dtype, int64_t B,
                              int64_t H, int64_t T, int64_t D, const int64_t* q_strides,
                              const int64_t* k_strides, const int64_t* v_strides,
                              const int32_t* indices, const int64_t* idx_strides, int64_t K,
                              float scale, unsigned flags, void* out, const int64_t* out_strides,
                              float* lse2, void* stream)
{
    int rc = check_readout(q, k, v, dtype, B, H, T, D, q_strides, k_strides, v_strides, indices,
                           idx_strides, K, out, out_strides);
    if (rc != WF_OK) return rc;
    if (!lse2 && B * H * T > 0) return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout_fwd_lse: NULL lse2");
    rc = run_readout(q, k, v, dtype, B, H, T, D, q_strides, k_strides, v_strides, indices,
                     idx_strides, K, scale, flags & WF_FLAG_MASK_PADS, out, out_strides, lse2,
                     static_cast<hipStream_t>(stream));
    return rc == WF_OK ? ok() : rc;
}

int wf_sparse_readout_fwd_dropout(const void* q, const void* k, const void* v, int dtype, int64_t B,
                                  int64_t H, int64_t T, int64_t D, const int64_t* q_strides,
                                  const int64_t* k_strides, const int64_t* v_strides,
                                  const int32_t* indices, const int64_t* idx_strides, int64_t K,
                                  float scale, unsigned flags, float dropout_p, uint64_t seed,
                                  void* out, const int64_t* out_strides, float* lse2, void* stream)
{
    int rc = check_readout(q, k, v, dtype, B, H, T, D, q_strides, k_strides, v_strides, indices,
                           idx_strides, K, out, out_strides);
    if (rc != WF_OK) return rc;
    if (!(dropout_p >= 0.0f && dropout_p < 1.0f))
        return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout_fwd_dropout: dropout_p=%g not in [0, 1)", double(dropout_p));
    if (!lse2 && B * H * T > 0) return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout_fwd_dropout: NULL lse2");
    const wf::DropoutParams d = make_dropout(dropout_p, seed);
    rc = run_readout(q, k, v, dtype, B, H, T, D, q_strides, k_strides, v_strides, indices,
                     idx_strides, K, scale, flags & WF_FLAG_MASK_PADS, out, out_strides, lse2,
                     static_cast<hipStream_t>(stream), dropout_p > 0.0f ? &d : nullptr);
    return rc == WF_OK ? ok() : rc;
}

size_t wf_sparse_readout_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t K)
{
    if (B <= 0 || H <= 0 || T <= 0 || K <= 0) return 0;
    return wf::sparse_readout_bwd_workspace(B, H, T, K);
}


int wf_sparse_readout_bwd(const wf_readout_bwd_args* a, void* stream)
{
    return readout_bwd(a, nullptr, stream);
}

int wf_sparse_readout_bwd_dropout(const wf_readout_bwd_args* a, float dropout_p, uint64_t seed, void* stream)
{
    if (!(dropout_p >= 0.0f && dropout_p < 1.0f))
        return fail(WF_ERR_INVALID_ARGUMENT, "sparse_readout_bwd_dropout: dropout_p=%g not in [0, 1)", double(dropout_p));
    const wf::DropoutParams d = make_dropout(dropout_p, seed);
    return readout_bwd(a, dropout_p > 0.0f ? &d : nullptr, stream);
}

int wf_address_project_fwd(const void* x, int dtype, int64_t B, int64_t T, int64_t d_model,
                           const int64_t* x_strides, const void* wq, const void* bq,
                           const void* wk, const void* bk, int64_t w_stride, int64_t R,
                           int normalize, void* out_q, const int64_t* oq_strides,
                           void* out_k, const int64_t* ok_strides, void* stream)
{
    if (!valid_dtype(dtype)) return fail(WF_ERR_UNSUPPORTED, "address_project: unsupported dtype code %d", dtype);
    if (B < 0 || T < 0 || d_model < 1 || R < 1)
        return fail(WF_ERR_INVALID_ARGUMENT, "address_project: bad shape (B=%lld, T=%lld, d_model=%lld, R=%lld)",
                    (long long)B, (long long)T, (long long)d_model, (long long)R);
    if (R > 32) return fail(WF_ERR_UNSUPPORTED, "address_project: address dim R=%lld > 32", (long long)R);
    if (d_model % 8 != 0) return fail(WF_ERR_UNSUPPORTED, "address_project: d_model=%lld not a multiple of 8", (long long)d_model);
    if (!x_strides || !oq_strides || (wk && !ok_strides))
        return fail(WF_ERR_INVALID_ARGUMENT, "address_project: stride arrays must not be NULL");
    if (B * T == 0) return ok();
    if (!x || !wq || !out_q || (wk && !out_k))
        return fail(WF_ERR_INVALID_ARGUMENT, "address_project: NULL x/wq/out pointer");
    const int64_t es = int64_t(elem_size(dtype));
    auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (x_strides[2] != 1 || !a16(x) || (x_strides[0] * es) % 16 || (x_strides[1] * es) % 16)
        return fail(WF_ERR_UNSUPPORTED, "address_project: x needs a contiguous last dim and 16-byte aligned rows");
    if (!a16(wq) || (wk && !a16(wk)) || (w_stride * es) % 16 || w_stride < d_model)
        return fail(WF_ERR_UNSUPPORTED, "address_project: weights need 16-byte aligned rows of at least d_model");
    wf::AddressParams p{};
    p.x = x; p.wq = wq; p.bq = bq; p.wk = wk; p.bk = bk; p.out_q = out_q; p.out_k = wk ? out_k : nullptr;
    p.xs[0] = x_strides[0]; p.xs[1] = x_strides[1];
    for (int i = 0; i < 3; ++i) { p.oqs[i] = oq_strides[i]; p.oks[i] = wk ? ok_strides[i] : 0; }
    p.w_stride = w_stride;
    p.B = B; p.T = T; p.d_model = d_model; p.R = R; p.n_tokens = B * T;
    p.normalize = normalize ? 1 : 0;
    const hipError_t e = wf::launch_address_project(dtype, p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("address_project: kernel launch", e);
    return ok();
}

int wf_residual_layernorm_fwd(const void* x, const void* delta, int dtype, int64_t rows, int64_t n,
                              int64_t x_stride, int64_t delta_stride, const void* weight,
                              const void* bias, float eps, void* sum_out, int64_t sum_stride,
                              void* y, int64_t y_stride, void* stream)
{
    if (!valid_dtype(dtype)) return fail(WF_ERR_UNSUPPORTED, "residual_layernorm: unsupported dtype code %d", dtype);
    if (rows < 0 || n < 1)
        return fail(WF_ERR_INVALID_ARGUMENT, "residual_layernorm: bad shape (rows=%lld, n=%lld)",
                    (long long)rows, (long long)n);
    if (n % 8 != 0 || n > 1024)
        return fail(WF_ERR_UNSUPPORTED, "residual_layernorm: n=%lld (needs a multiple of 8, at most 1024)", (long long)n);
    if (!(eps >= 0.0f)) return fail(WF_ERR_INVALID_ARGUMENT, "residual_layernorm: eps=%g", double(eps));
    if (rows == 0) return ok();
    if (!x || !y) return fail(WF_ERR_INVALID_ARGUMENT, "residual_layernorm: NULL x or y");
    const int64_t es = int64_t(elem_size(dtype));
    auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    auto rows_ok = [&](const void* p, int64_t stride) {
        return p == nullptr || (a16(p) && stride >= n && (stride * es) % 16 == 0);
    };
    if (!rows_ok(x, x_stride) || !rows_ok(delta, delta_stride) || !rows_ok(sum_out, sum_stride) ||
        !rows_ok(y, y_stride) || (weight && !a16(weight)) || (bias && !a16(bias)))
        return fail(WF_ERR_UNSUPPORTED, "residual_layernorm: rows and parameters need 16-byte alignment "
                                        "and strides of at least n");
    wf::LayerNormParams p{};
    p.x = x; p.delta = delta; p.weight = weight; p.bias = bias; p.sum_out = sum_out; p.y = y;
    p.x_stride = x_stride; p.delta_stride = delta_stride; p.sum_stride = sum_stride; p.y_stride = y_stride;
    p.rows = rows; p.n = n; p.eps = eps;
    const hipError_t e = wf::launch_residual_layernorm(dtype, p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("residual_layernorm: kernel launch", e);
    return ok();
}

size_t wf_probe_gather_sink_bytes(int64_t B, int64_t H, int64_t T)
{
    if (B <= 0 || H <= 0 || T <= 0) return 0;
    wf::ReadoutParams p{};
    p.B = B; p.H = H; p.T = T;
    if (!readout_rows(p, 0, T)) return 0;
    return size_t(8 * (p.vpairs / 8) * p.wg_per_vpair) * 256u * sizeof(uint32_t);
}

int wf_probe_gather(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t T,
                    int64_t D, const int64_t* k_strides, const int64_t* v_strides,
                    const int32_t* indices, const int64_t* idx_strides, int64_t K,
                    uint32_t* sink, size_t sink_bytes, void* stream)
{
    if (dtype != WF_DTYPE_BF16 && dtype != WF_DTYPE_F16)
        return fail(WF_ERR_UNSUPPORTED, "probe_gather: 16-bit types only");
    if (B < 1 || H < 1 || T < 1 || (D != 32 && D != 64 && D != 128))
        return fail(WF_ERR_INVALID_ARGUMENT, "probe_gather: bad shape");
    if (K < 4 || K % 4 != 0 || K > kMaxReadoutK)
        return fail(WF_ERR_UNSUPPORTED, "probe_gather: K must be a multiple of 4 in [4, %lld]", (long long)kMaxReadoutK);
    if (!k || !v || !indices || !sink || !k_strides || !v_strides || !idx_strides)
        return fail(WF_ERR_INVALID_ARGUMENT, "probe_gather: NULL pointer");
    const int64_t es = 2;
    auto span_ok = [&](const int64_t* st) {
        return st[2] >= 0 && (T - 1) * st[2] * es + D * es < (int64_t(1) << 32) && st[2] * es < (int64_t(1) << 24);
    };
    if (!vec_ok(k, dtype, k_strides, 4, D) || !vec_ok(v, dtype, v_strides, 4, D) || !span_ok(k_strides) ||
        !span_ok(v_strides) || T > (int64_t(1) << 24) || idx_strides[2] != 1 ||
        reinterpret_cast<uintptr_t>(indices) % 16 != 0 || idx_strides[0] % 4 != 0 || idx_strides[1] % 4 != 0)
        return fail(WF_ERR_UNSUPPORTED, "probe_gather: needs the readout's fast layout");
    if (sink_bytes < wf_probe_gather_sink_bytes(B, H, T))
        return fail(WF_ERR_WORKSPACE, "probe_gather: sink of %zu bytes required", wf_probe_gather_sink_bytes(B, H, T));
    wf::ReadoutParams p{};
    p.k = k; p.v = v; p.idx = indices;
    for (int i = 0; i < 4; ++i) { p.ks[i] = k_strides[i]; p.vs[i] = v_strides[i]; }
    for (int i = 0; i < 3; ++i) p.is[i] = idx_strides[i];
    p.B = B; p.H = H; p.T = T; p.D = D; p.K = K;
    if (!readout_rows(p, 0, T)) return fail(WF_ERR_UNSUPPORTED, "probe_gather: problem too large");
    const hipError_t e = wf::launch_gather_probe(dtype, p, sink, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail("probe_gather: kernel launch", e);
    return ok();
}

int wf_fused_topk_sparse_fwd(const wf_fused_args* a, void* stream)
{
    const int rc = fused_run(a, a ? a->workspace : nullptr, a ? a->workspace_bytes : 0,
                             static_cast<hipStream_t>(stream));
    return rc == WF_OK ? ok() : rc;
}

size_t wf_fused_noalloc_scratch_limit(void) { return kScratchBytes; }

int wf_fused_topk_sparse_fwd_noalloc(const wf_fused_args* a, void* stream)
{
    if (!a) return fail(WF_ERR_INVALID_ARGUMENT, "fused_noalloc: NULL argument struct");
    const size_t need = wf_fused_workspace_bytes(a->B, a->T, a->R, a->top_k);
    if (need > kScratchBytes)
        return fail(WF_ERR_UNSUPPORTED, "fused_noalloc: this shape needs %zu bytes of scratch; the library's "
                                        "scratch holds %zu (B * ceil(T / 256) <= %zu); use "
                                        "wf_fused_topk_sparse_fwd with a workspace instead",
                    need, kScratchBytes, kScratchBytes / sizeof(float));
    void* ws = nullptr;
    if (need > 0) {
        const int rc = scratch_for_current_device(&ws);
        if (rc != WF_OK) return rc;
    }
    const int rc = fused_run(a, ws, kScratchBytes, static_cast<hipStream_t>(stream));
    return rc == WF_OK ? ok() : rc;
}

}  // extern "C"
