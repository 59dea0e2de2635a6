// wf_address.hip -- learned-address projection + L2 normalisation in one pass (gfx950).
//
// Replaces LearnedAddressModule.forward_query_key (routing_attention/models/
// learned_address.py:39-46): q = normalize(x W_q^T + b_q), k = normalize(x W_k^T + b_k),
// which PyTorch runs as two GEMMs and, per output, a norm reduction, a clamp and a division
// (six launches and three passes over the (B, T, R) tensors per layer). 16-bit inputs run
// on the matrix cores: one wave takes 16 tokens and computes their q and k outputs as four
// 16 x 16 tiles of v_mfma_f32_16x16x32_{bf16,f16} (tokens = A rows straight from x, outputs
// = B columns straight from the weight rows, no LDS), with eight 32-dim steps of loads in
// flight, and the normalisation is a 16-lane DPP reduction over each tile's outputs. fp32
// inputs keep a VALU kernel: one workgroup takes 32 tokens, the token tile and the stacked
// (up to 64-row) weight tile go through LDS in 256-column chunks, each thread accumulates a
// 2 token x 4 output block with FMA, and the norm is an 8-lane shuffle reduction.
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

// four fp32 products of a 16-byte chunk, accumulated in fp32
__device__ __forceinline__ float dot_chunk(const uint4& a, const uint4& b)
{
    float d = __uint_as_float(a.x) * __uint_as_float(b.x);
    d = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), d);
    d = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), d);
    d = fmaf(__uint_as_float(a.w), __uint_as_float(b.w), d);
    return d;
}

// fp32 inputs. Thread layout: tb = tid / 16 picks tokens kTPT*tb.., ob = tid % 16 picks
// output rows 4ob..4ob+3; lanes 0-7 of each 16-lane group hold q rows, lanes 8-15 k rows, so
// one 8-lane shuffle reduction gives a token's squared norm.
__global__ __launch_bounds__(256) void address_project_kernel(AddressParams p)
{
    typedef float DT;
    constexpr int EPC = 4;                      // elements per 16-byte chunk
    __shared__ __align__(16) float xs[kTok * kPitch];
    __shared__ __align__(16) float ws[kOut * kPitch];
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
                for (int j = 0; j < 4; ++j) acc[i][j] += dot_chunk(xv[i], wv[j]);
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
            y[j] = o0 + j < p.R ? acc[i][j] + bv[j] : 0.0f;
            ss = fmaf(y[j], y[j], ss);
        }
        ss = sum8(ss);
        const float den = fmaxf(sqrtf(ss), 1e-12f);   // norm(...).clamp_min(eps)
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

// sum over the 16 lanes of a DPP row (row_ror 8, 4, 2, 1)
__device__ __forceinline__ float row_sum16f(float x)
{
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x122, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x121, 0xf, 0xf, false));
    return x;
}

template <typename DT>
__device__ __forceinline__ f32x4_t mfma16x16x32(const uint4& a, const uint4& b, f32x4_t acc)
{
    if constexpr (__is_same(DT, bf16_t))
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), acc, 0, 0, 0);
}

// 16-bit inputs: one wave = 16 tokens tok0..tok0+15. Tile c of the output holds q outputs
// 16c..16c+15 (c = 0, 1) or k outputs 16(c-2).. (c = 2, 3). MFMA operands: A = x (lane l:
// token tok0 + l%16, dims 8(l/16)..+7 of the 32-dim step), B = W^T (lane l: output l%16 of
// the tile, the same dims); the result puts tokens 4(l/16)..+3 (elements r) of output
// l%16 in lane l, so each token's squared norm over a tile is a sum over one DPP row.
template <typename DT>
__global__ __launch_bounds__(64) void address_project_mfma_kernel(AddressParams p)
{
    constexpr int KG = 8;   // 32-dim steps whose loads are in flight together
    const int lane = threadIdx.x;
    const int n = lane & 15, g = lane >> 4;
    const int64_t tok0 = int64_t(blockIdx.x) * 16;
    const int D = int(p.d_model), R = int(p.R);
    // batch and position of token tok0 (wave-uniform); a later token of the wave steps on
    // from it, wrapping into the next batch rows
    const int64_t b0 = tok0 / p.T, t0 = tok0 % p.T;
    auto locate = [&](int j, int64_t& b, int64_t& t) {
        b = b0;
        t = t0 + j;
        while (t >= p.T) { t -= p.T; ++b; }
    };
    int64_t xb, xt;
    locate(int(min(int64_t(n), p.n_tokens - 1 - tok0)), xb, xt);   // rows past the end repeat the last
    const DT* xrow = static_cast<const DT*>(p.x) + xb * p.xs[0] + xt * p.xs[1];
    const DT* wrow[4];
    bool wok[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int o = 16 * (c & 1) + n;
        const DT* w = static_cast<const DT*>(c < 2 ? p.wq : p.wk);
        wok[c] = w != nullptr && o < R;
        wrow[c] = wok[c] ? w + int64_t(o) * p.w_stride : static_cast<const DT*>(p.wq);
    }
    f32x4_t acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < D; k0 += 32 * KG) {
        uint4 xa[KG], wb[KG][4];
#pragma unroll
        for (int kk = 0; kk < KG; ++kk) {
            // D is a multiple of 8: a chunk is all in or all out. Every load is issued (chunks
            // past D read chunk 0, rows past R read W_q row 0) and masked afterwards, so the
            // wave issues them back to back without a branch per load.
            const int d = k0 + 32 * kk + 8 * g;
            const bool in = d < D;
            const int dl = in ? d : 8 * g;
            xa[kk] = *reinterpret_cast<const uint4*>(xrow + dl);
#pragma unroll
            for (int c = 0; c < 4; ++c) wb[kk][c] = *reinterpret_cast<const uint4*>(wrow[c] + dl);
            if (!in) xa[kk] = make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (!(in && wok[c])) wb[kk][c] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int kk = 0; kk < KG; ++kk)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = mfma16x16x32<DT>(xa[kk], wb[kk][c], acc[c]);
    }

    // epilogue: bias, rounding, norm over the row's outputs, store
    float y[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int o = 16 * (c & 1) + n;
        const DT* bias = static_cast<const DT*>(c < 2 ? p.bq : p.bk);
        const float bv = bias != nullptr && wok[c] ? to_f32(bias[o]) : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) y[c][r] = wok[c] ? round_to<DT>(acc[c][r] + bv) : 0.0f;
    }
    float den[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float ss = fmaf(y[2 * h][r], y[2 * h][r], y[2 * h + 1][r] * y[2 * h + 1][r]);
            ss = row_sum16f(ss);
            den[h][r] = fmaxf(round_to<DT>(sqrtf(ss)), 1e-12f);   // norm(...).clamp_min(eps)
        }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int j = 4 * g + r;
        if (tok0 + j >= p.n_tokens) continue;
        int64_t b, t;
        locate(j, b, t);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            DT* out = static_cast<DT*>(c < 2 ? p.out_q : p.out_k);
            if (out == nullptr || !wok[c]) continue;
            const int64_t* os = c < 2 ? p.oqs : p.oks;
            DT v;
            from_f32(p.normalize ? y[c][r] / den[c >> 1][r] : y[c][r], v);
            out[b * os[0] + t * os[1] + (16 * (c & 1) + n) * os[2]] = v;
        }
    }
}

}  // namespace

hipError_t launch_address_project(int dtype, const AddressParams& p, hipStream_t s)
{
    if (dtype == 2 || dtype == 1) {
        const dim3 grid(static_cast<unsigned>((p.n_tokens + 15) / 16)), block(64);
        if (dtype == 2) address_project_mfma_kernel<bf16_t><<<grid, block, 0, s>>>(p);
        else address_project_mfma_kernel<_Float16><<<grid, block, 0, s>>>(p);
        return hipGetLastError();
    }
    const dim3 grid(static_cast<unsigned>((p.n_tokens + kTok - 1) / kTok)), block(256);
    address_project_kernel<<<grid, block, 0, s>>>(p);
    return hipGetLastError();
}

}  // namespace wf
