// wf_internal.h -- device helpers and launcher declarations shared by the gfx950 kernels
// of libwayfinder_hip.so. Not part of the public ABI (include/wayfinder_hip.h is).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wf {

// ---------------------------------------------------------------- element types
// bf16 is carried as its raw 16-bit pattern; f16 as _Float16; f32 as float.
struct bf16_t { uint16_t bits; };

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(uint32_t(x.bits) << 16); }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(float x) { return x; }

// round-to-nearest-even fp32 -> storage type (NaN kept quiet)
__device__ __forceinline__ void from_f32(float x, bf16_t& y)
{
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) { y.bits = uint16_t((u >> 16) | 0x40u); return; }
    u += 0x7fffu + ((u >> 16) & 1u);
    y.bits = uint16_t(u >> 16);
}
__device__ __forceinline__ void from_f32(float x, _Float16& y) { y = (_Float16)x; }
__device__ __forceinline__ void from_f32(float x, float& y) { y = x; }

// Raw 16-byte chunk <-> eight fp32 values (bf16 / f16: one chunk = 8 elements).
__device__ __forceinline__ void unpack8(const uint4& u, bf16_t, float* f)
{
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(w[i] << 16);
        f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ void unpack8(const uint4& u, _Float16, float* f)
{
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        _Float16 lo = __builtin_bit_cast(_Float16, uint16_t(w[i] & 0xffffu));
        _Float16 hi = __builtin_bit_cast(_Float16, uint16_t(w[i] >> 16));
        f[2 * i] = (float)lo;
        f[2 * i + 1] = (float)hi;
    }
}

// ---------------------------------------------------------------- wave helpers (wave64)
__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ float wave_max(float x)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t y = __shfl_xor(x, o, 64);
        x = y < x ? y : x;
    }
    return x;
}
// sum over lanes with index > lane (exclusive suffix sum)
__device__ __forceinline__ int wave_suffix_excl(int x)
{
    const int lane = lane_id();
    int s = x;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_down(s, o, 64);
        if (lane + o < 64) s += y;
    }
    return s - x;
}

// order-preserving map fp32 -> uint32 (larger float -> larger uint); -0 is folded to +0
__device__ __forceinline__ uint32_t ord_f32(float s)
{
    uint32_t u = __float_as_uint(s + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unord_f32(uint32_t o)
{
    uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
    return __uint_as_float(u);
}

// ---------------------------------------------------------------- launch parameter blocks
struct TopkParams {
    const void* query;
    const void* key;
    int64_t qsb, qst, qsr;   // element strides of query (B, T, R)
    int64_t ksb, kst, ksr;   // element strides of key
    int64_t B, T, R, k_eff;
    int32_t* out_idx;        // (B, T, k_eff) contiguous
    float* out_scores;       // optional
    float* chunk_absmax;     // (B, n_chunks) workspace
    int64_t n_chunks;
    int64_t n_row_blocks;    // ceil(T / 16)
    int64_t rb_begin, rb_end;  // row blocks [rb_begin, rb_end) of this launch
    int64_t n_cus;           // compute units of the device (dispatch order of the row blocks)
    float seed_alpha;        // speculative screening threshold: ~seed_alpha * k_eff keys pass
                             // it (0: off, every row starts at -inf)
};

// Unsigned 32-bit division by a divisor fixed per launch (Granlund-Montgomery, round-up
// multiplier): l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, and for every 32-bit x
// x / d = (t + ((x - t) >> 1)) >> (l - 1) with t = umulhi(x, m); d = 1 is the identity.
struct FastDiv {
    uint32_t m, l;
};

inline FastDiv make_fastdiv(uint32_t d)
{
    FastDiv f{0, 0};
    if (d <= 1) return f;
    while ((uint64_t(1) << f.l) < d) ++f.l;
    f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << f.l) - d)) / d + 1);
    return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t x, FastDiv f)
{
    if (f.l == 0) return x;
    const uint32_t t = __umulhi(x, f.m);
    return (t + ((x - t) >> 1)) >> (f.l - 1);
}

// Dropout on the readout's attention weights. Slot s of query row t of head h in batch b is
// kept when keep_hash(row_key(k, ((b*H + h)*T + t)), s) >= thresh, a Bernoulli(1 - p) draw for
// thresh = round(p * 2^32); kept weights are scaled by 1 / (1 - p). The hash is the "lowbias32"
// integer mixer (C. Wellons, hash-prospector, public domain) chained over the 64-bit row id and
// the two halves of the 64-bit seed, then once more over the slot; the CPU oracle restates it.
struct DropoutParams {
    uint32_t thresh;   // keep iff hash >= thresh
    uint32_t k0, k1;   // low and high words of the seed
    float scale;       // 1 / (1 - p)
};

__host__ __device__ __forceinline__ uint32_t drop_mix32(uint32_t x)
{
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

__host__ __device__ __forceinline__ uint32_t drop_row_key(const DropoutParams& d, uint64_t row_id)
{
    return drop_mix32(drop_mix32(uint32_t(row_id) ^ d.k0) ^ uint32_t(row_id >> 32) ^ d.k1);
}

__host__ __device__ __forceinline__ bool drop_keep(const DropoutParams& d, uint32_t row_key, uint32_t slot)
{
    return drop_mix32(row_key ^ slot) >= d.thresh;
}

struct ReadoutParams {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    const int32_t* idx;
    int64_t qs[4], ks[4], vs[4], os[4];  // element strides (B, H, T, D)
    int64_t is[3];                       // index strides (B, T, K)
    int64_t B, H, T, D, K;
    float scale;
    unsigned flags;
    float* lse2;            // optional (B, H, T) contiguous: log2 of the softmax denominator
                            // in the kernels' base-2 domain (see wf_sparse_readout_fwd_lse)
    int64_t row_begin, row_end;  // query rows [row_begin, row_end) of this launch
    int64_t seg_per_pair;   // row segments per (b,h) pair (XCD balance)
    int64_t rows_per_seg;
    int64_t vpairs;         // B*H*seg_per_pair virtual pairs
    int64_t wg_per_vpair;   // workgroups per virtual pair
    int head_major;         // workgroup order: 1 = virtual pair by virtual pair (grids larger
                            // than one residency wave), 0 = pair blockIdx % 8 (one wave);
                            // set by the launcher from the kernel's occupancy
    int drop_on;            // dropout on the attention weights (then lse2 is set)
    DropoutParams drop;
};

// Readout stage of the single-pass fused kernel (wf_fused.hip): the block's rows for all
// heads, right after their retrieval.
struct FusedReadoutParams {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    int64_t qs[4], ks[4], vs[4], os[4];   // element strides (B, H, T, D); stride of D is 1
    int64_t H, D;
    float scale;
    unsigned flags;                        // bit 0: mask the pad slots
};

// Backward of the readout (fixed indices). Both passes pair blockIdx % 8 with a fixed set of
// (b, h) pairs at every grid size (the row pass over query rows t, the key pass over key rows
// j): chunk-major order starts the key pass's long early-key lists of every pair first, which
// measured 27 % faster than running the pairs one after another.
struct ReadoutBwdParams {
    const void* q;
    const void* k;
    const void* v;
    const void* dout;
    void* dq;
    void* dk;
    void* dv;
    const int32_t* idx;
    const float* lse2;       // (B, H, T) from the forward
    float2* row_stats;       // (B, H, T) workspace, row pass -> key pass: (lse2, delta) with
                             // delta = sum_s p_s (dout . v_s); one 8-byte load per list entry
    const uint32_t* off;     // (B*T + 1) start of each key's list in `rows`
    const uint32_t* rows;    // slots t*K + s referencing each key, grouped by key, t ascending
    int64_t qs[4], ks[4], vs[4], gs[4], dqs[4], dks[4], dvs[4];  // element strides (B, H, T, D)
    int64_t is[3];
    int64_t B, H, T, D, K;
    float scale;
    unsigned flags;
    int64_t row_begin, row_end;                                 // as in ReadoutParams
    int64_t seg_per_pair, rows_per_seg, vpairs, wg_per_vpair;
    FastDiv divK;            // t = slot / K in the key pass
    int drop_on;             // dropout on the attention weights, as in the forward
    DropoutParams drop;
};

// Learned-address projection + normalisation (wf_address.hip).
struct AddressParams {
    const void* x;           // (B, T, d_model), contiguous last dim
    const void* wq;          // (R, d_model) rows at stride w_stride
    const void* bq;          // (R) or null
    const void* wk;          // null: symmetric (only q is written)
    const void* bk;
    void* out_q;             // (B, T, R)
    void* out_k;             // null when symmetric
    int64_t xs[2];           // element strides of x over (B, T)
    int64_t oqs[3], oks[3];  // element strides of the outputs
    int64_t w_stride;
    int64_t B, T, d_model, R, n_tokens;
    int normalize;
};

// ReadoutParams.flags bit set by the fused entry point: the indices were written by this
// library's retrieval, so every entry lies in [0, T) and needs no wrap or clamp.
constexpr unsigned kFlagTrustedIndices = 0x80000000u;

// Key-magnitude chunk size of the screening bound (keys per chunk).
constexpr int kAbsmaxChunk = 256;
// Query rows per readout workgroup (4 waves x 4 consecutive rows).
constexpr int kReadoutRowsPerWG = 16;
// Compute units of the current device, read once per device (hipDeviceGetAttribute) and
// cached; thread-safe. Only scheduling decisions depend on it, never results.
int device_cu_count();

// Workgroups of `kernel` (block of `block` threads, no dynamic LDS) resident at once on the
// current device: CUs x the kernel's occupancy per CU. The caller caches it per device.
int64_t resident_workgroups(const void* kernel, int block);

// launchers (return hipError_t of the launch)
hipError_t launch_key_absmax(int dtype, bool vec, const TopkParams& p, hipStream_t s);
hipError_t launch_causal_topk(int dtype, bool vec, const TopkParams& p, hipStream_t s);
hipError_t launch_causal_topk_bf16(bool vec, const TopkParams& p, hipStream_t s);
hipError_t launch_causal_topk_f16(bool vec, const TopkParams& p, hipStream_t s);
hipError_t launch_causal_topk_f32(bool vec, const TopkParams& p, hipStream_t s);
hipError_t launch_sparse_readout(int dtype, bool vec, bool fast, const ReadoutParams& p, hipStream_t s);
// device workspace of the backward for this shape (index transpose arrays, radix histograms,
// per-row statistics); a function of the shape only
size_t sparse_readout_bwd_workspace(int64_t B, int64_t H, int64_t T, int64_t K);
hipError_t launch_sparse_readout_bwd(int dtype, ReadoutBwdParams p, void* ws, size_t ws_bytes, hipStream_t s);
hipError_t launch_address_project(int dtype, const AddressParams& p, hipStream_t s);

// residual add + LayerNorm over the last dim (wf_layernorm.hip)
struct LayerNormParams {
    const void* x;           // (rows, n) at row stride x_stride, contiguous rows
    const void* delta;       // same shape at delta_stride, or null (LayerNorm of x alone)
    const void* weight;      // (n) or null
    const void* bias;        // (n) or null
    void* sum_out;           // x + delta (rows, n) at sum_stride, or null (not written)
    void* y;                 // LayerNorm(x + delta) (rows, n) at y_stride
    int64_t x_stride, delta_stride, sum_stride, y_stride;
    int64_t rows, n;         // n % 8 == 0, n <= 1024
    float eps;
};
hipError_t launch_residual_layernorm(int dtype, const LayerNormParams& p, hipStream_t s);
// single-pass fused forward (wf_fused.hip): retrieval and all-heads readout in one kernel.
// True if the shape and layout qualify (16-bit types, R = 32 on the aligned path,
// 64 < k_eff <= 256, D / 8 lanes per head with H * D / 8 in {64, 128}).
bool fused_single_pass_supported(int dtype, bool topk_vec, const TopkParams& tp, const FusedReadoutParams& fr);
hipError_t launch_fused_single_pass(int dtype, const TopkParams& tp, const FusedReadoutParams& fr, hipStream_t s);
// measurement aid (wf_probe.hip): the readout's gathers without its arithmetic, 16-bit types
hipError_t launch_gather_probe(int dtype, const ReadoutParams& p, uint32_t* sink, hipStream_t s);

}  // namespace wf
