// wf_address.hip -- learned-address projection + L2 normalisation in one pass (gfx950).
//
// Replaces LearnedAddressModule.forward_query_key (routing_attention/models/
// learned_address.py:39-46): q = normalize(x W_q^T + b_q), k = normalize(x W_k^T + b_k),
// which PyTorch runs as two GEMMs and, per output, a norm reduction, a clamp and a division
// (six launches and three passes over the (B, T, R) tensors per layer). Here one workgroup
// takes 64 tokens: the token tile and the (up to 64-row) stacked weight tile go through LDS
// in 256-column chunks, each thread accumulates a 4 token x 4 output block with dot2
// (bf16 / f16) or FMA (fp32) in fp32, and the normalisation is an 8-lane shuffle reduction.
//
// Rounding follows the PyTorch ops it replaces, so 16-bit results match them to the GEMM's
// accumulation order: the linear output is rounded to the storage type (bias added in fp32
// first), the norm of the rounded values is accumulated in fp32 and rounded, clamped to
// eps = 1e-12, and the quotient is computed in fp32 and rounded once.
#include "wf_internal.h"

namespace wf {
namespace {

constexpr int kTPT = 2;           // tokens per thread
constexpr int kTok = 16 * kTPT;   // tokens per workgroup (512 workgroups at 16384 tokens)
constexpr int kOut = 64;          // output rows per workgroup: q in rows 0..31, k in 32..63
constexpr int kChunk = 256;       // d_model columns staged per LDS round
constexpr int kPitch = kChunk + 8;  // LDS row pitch in elements (16 B pad: conflict-free rows)

template <typename DT> struct Raw;
template <> struct Raw<bf16_t> { typedef uint16_t T; };
template <> struct Raw<_Float16> { typedef uint16_t T; };
template <> struct Raw<float> { typedef float T; };

template <typename DT>
__device__ __forceinline__ float round_to(float x)
{
    if constexpr (sizeof(DT) == 4) {
        return x;
    } else {
        DT y;
        from_f32(x, y);
        return to_f32(y);
    }
}

// sum over 8 consecutive lanes (xor 1, 2, 4)
__device__ __forceinline__ float sum8(float x)
{
    x += __shfl_xor(x, 1, 64);
    x += __shfl_xor(x, 2, 64);
    x += __shfl_xor(x, 4, 64);
    return x;
}

template <typename DT>
__device__ __forceinline__ float dot_chunk(const uint4& a, const uint4& b)
{
    if constexpr (__is_same(DT, bf16_t)) {
        typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 v2;
        float d = 0.0f;
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a.x), __builtin_bit_cast(v2, b.x), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a.y), __builtin_bit_cast(v2, b.y), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a.z), __builtin_bit_cast(v2, b.z), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a.w), __builtin_bit_cast(v2, b.w), d, false);
        return d;
    } else if constexpr (__is_same(DT, _Float16)) {
        typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 v2;
        float d = 0.0f;
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a.x), __builtin_bit_cast(v2, b.x), d, false);
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a.y), __builtin_bit_cast(v2, b.y), d, false);
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a.z), __builtin_bit_cast(v2, b.z), d, false);
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a.w), __builtin_bit_cast(v2, b.w), d, false);
        return d;
    } else {
        float d = __uint_as_float(a.x) * __uint_as_float(b.x);
        d = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), d);
        d = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), d);
        d = fmaf(__uint_as_float(a.w), __uint_as_float(b.w), d);
        return d;
    }
}

// Thread layout: tb = tid / 16 picks tokens kTPT*tb.., ob = tid % 16 picks output rows
// 4ob..4ob+3; lanes 0-7 of each 16-lane group hold q rows, lanes 8-15 k rows, so one
// 8-lane shuffle reduction gives a token's squared norm.
template <typename DT>
__global__ __launch_bounds__(256) void address_project_kernel(AddressParams p)
{
    typedef typename Raw<DT>::T RT;
    constexpr int EPC = 16 / sizeof(DT);        // elements per 16-byte chunk
    __shared__ __align__(16) RT xs[kTok * kPitch];
    __shared__ __align__(16) RT ws[kOut * kPitch];
    const int tid = threadIdx.x;
    const int tb = tid >> 4, ob = tid & 15;
    const int64_t tok0 = int64_t(blockIdx.x) * kTok;
    const int D = int(p.d_model);
    const DT* x = static_cast<const DT*>(p.x);
    float acc[kTPT][4] = {};

    // staging: every thread issues all of its 16-byte loads of a round (token tile, then the
    // weight tile) before the first LDS store, so a round waits on memory once
    constexpr int NCH = kChunk / EPC;                     // 16-byte chunks per full row
    constexpr int kXPer = kTok * NCH / 256;              // loads per thread and tile
    constexpr int kWPer = kOut * NCH / 256;
    // element offset of each token row of the tile (one 64-bit division per row, by kTok
    // threads, instead of one per load)
    __shared__ int64_t row_off[kTok];
    __shared__ int64_t row_b[kTok], row_t[kTok];
    if (tid < kTok) {
        const int64_t n = min(tok0 + tid, p.n_tokens - 1);
        const int64_t b = n / p.T, t = n % p.T;
        row_off[tid] = b * p.xs[0] + t * p.xs[1];
        row_b[tid] = b;
        row_t[tid] = t;
    }
    __syncthreads();
    for (int c0 = 0; c0 < D; c0 += kChunk) {
        const int cw = min(kChunk, D - c0);       // multiple of 8 (checked by the entry point)
        const int nch = cw / EPC;                 // 16-byte chunks per row in this round
        uint4 xv[kXPer], wv[kWPer];
#pragma unroll
        for (int k = 0; k < kXPer; ++k) {
            const int i = tid + 256 * k;
            const int r = i / NCH, c = i % NCH;   // compile-time divisor
            xv[k] = make_uint4(0, 0, 0, 0);
            if (c < nch && tok0 + r < p.n_tokens)
                xv[k] = *reinterpret_cast<const uint4*>(x + row_off[r & (kTok - 1)] + c0 + c * EPC);
        }
#pragma unroll
        for (int k = 0; k < kWPer; ++k) {
            const int i = tid + 256 * k;
            const int r = i / NCH, c = i % NCH;
            const int half = r / 32, o = r % 32;
            const DT* w = half == 0 ? static_cast<const DT*>(p.wq) : static_cast<const DT*>(p.wk);
            wv[k] = make_uint4(0, 0, 0, 0);
            if (c < nch && o < p.R && w != nullptr)
                wv[k] = *reinterpret_cast<const uint4*>(w + int64_t(o) * p.w_stride + c0 + c * EPC);
        }
        __syncthreads();   // the previous round's tiles are consumed
#pragma unroll
        for (int k = 0; k < kXPer; ++k) {
            const int i = tid + 256 * k;
            if (i % NCH < nch) *reinterpret_cast<uint4*>(&xs[(i / NCH) * kPitch + (i % NCH) * EPC]) = xv[k];
        }
#pragma unroll
        for (int k = 0; k < kWPer; ++k) {
            const int i = tid + 256 * k;
            if (i % NCH < nch) *reinterpret_cast<uint4*>(&ws[(i / NCH) * kPitch + (i % NCH) * EPC]) = wv[k];
        }
        __syncthreads();
        for (int c = 0; c < nch; ++c) {
            uint4 xv[kTPT], wv[4];
#pragma unroll
            for (int i = 0; i < kTPT; ++i) xv[i] = *reinterpret_cast<const uint4*>(&xs[(tb * kTPT + i) * kPitch + c * EPC]);
#pragma unroll
            for (int i = 0; i < 4; ++i) wv[i] = *reinterpret_cast<const uint4*>(&ws[(ob * 4 + i) * kPitch + c * EPC]);
#pragma unroll
            for (int i = 0; i < kTPT; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += dot_chunk<DT>(xv[i], wv[j]);
        }
    }

    // epilogue: bias, rounding, norm, store
    const int half = ob >> 3;                     // 0: q rows, 1: k rows
    const int o0 = (ob & 7) * 4;                  // first output of this thread within its half
    const DT* bias = half == 0 ? static_cast<const DT*>(p.bq) : static_cast<const DT*>(p.bk);
    float bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        bv[j] = 0.0f;
        if (bias != nullptr && o0 + j < p.R) {
            const DT bj = bias[o0 + j];
            bv[j] = to_f32(bj);
        }
    }
    DT* out = static_cast<DT*>(half == 0 ? p.out_q : p.out_k);
    const int64_t* os = half == 0 ? p.oqs : p.oks;
#pragma unroll
    for (int i = 0; i < kTPT; ++i) {
        float y[4], ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            y[j] = o0 + j < p.R ? round_to<DT>(acc[i][j] + bv[j]) : 0.0f;
            ss = fmaf(y[j], y[j], ss);
        }
        ss = sum8(ss);
        const float den = fmaxf(round_to<DT>(sqrtf(ss)), 1e-12f);   // norm(...).clamp_min(eps)
        const int64_t n = tok0 + tb * kTPT + i;
        if (n < p.n_tokens && out != nullptr) {
            DT* orow = out + row_b[tb * kTPT + i] * os[0] + row_t[tb * kTPT + i] * os[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (o0 + j < p.R) {
                    DT v;
                    from_f32(p.normalize ? y[j] / den : y[j], v);
                    orow[(o0 + j) * os[2]] = v;
                }
            }
        }
    }
}

}  // namespace

hipError_t launch_address_project(int dtype, const AddressParams& p, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>((p.n_tokens + kTok - 1) / kTok)), block(256);
    if (dtype == 2) address_project_kernel<bf16_t><<<grid, block, 0, s>>>(p);
    else if (dtype == 1) address_project_kernel<_Float16><<<grid, block, 0, s>>>(p);
    else address_project_kernel<float><<<grid, block, 0, s>>>(p);
    return hipGetLastError();
}

}  // namespace wf
