// wf_readout_dev.h -- device helpers shared by the readout kernels (forward in
// wf_readout.hip, backward in wf_readout_bwd.hip): constants, 16-byte row loads and
// stores, lane-group reductions (DPP within a 16-lane row, shuffles across rows) and the
// 8-element dot product / p.v update on packed 16-bit or fp32 data.
#pragma once

#include "wf_internal.h"

namespace wf {
namespace {

constexpr int kWaves = 4;        // waves per workgroup
constexpr int kRowsPerWave = kReadoutRowsPerWG / kWaves;  // consecutive query rows per wave
constexpr float kLog2e = 1.4426950408889634f;

template <typename DT, bool VEC>
__device__ __forceinline__ void load_row8(const DT* p, int64_t sd, uint4& lo, uint4& hi)
{
    if constexpr (VEC) {
        lo = *reinterpret_cast<const uint4*>(p);
        if constexpr (sizeof(DT) == 4) hi = *reinterpret_cast<const uint4*>(p + 4);
        else hi = make_uint4(0, 0, 0, 0);
    } else {
        if constexpr (sizeof(DT) == 2) {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                w[e >> 1] |= uint32_t(*reinterpret_cast<const uint16_t*>(p + e * sd)) << (16 * (e & 1));
            lo = make_uint4(w[0], w[1], w[2], w[3]);
            hi = make_uint4(0, 0, 0, 0);
        } else {
            uint32_t w[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) w[e] = __float_as_uint(*reinterpret_cast<const float*>(p + e * sd));
            lo = make_uint4(w[0], w[1], w[2], w[3]);
            hi = make_uint4(w[4], w[5], w[6], w[7]);
        }
    }
}

// Elements [0, n) of an 8-element slice at element stride sd (n < 8: the head dim ends
// inside the slice); the rest read as zero. For layouts without 16-byte vector access.
template <typename DT>
__device__ __forceinline__ void load_row8_part(const DT* p, int64_t sd, int n, uint4& lo, uint4& hi)
{
    uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if constexpr (sizeof(DT) == 2) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (e < n) w[e >> 1] |= uint32_t(*reinterpret_cast<const uint16_t*>(p + e * sd)) << (16 * (e & 1));
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (e < n) w[e] = __float_as_uint(*reinterpret_cast<const float*>(p + e * sd));
    }
    lo = make_uint4(w[0], w[1], w[2], w[3]);
    hi = sizeof(DT) == 4 ? make_uint4(w[4], w[5], w[6], w[7]) : make_uint4(0, 0, 0, 0);
}

// Elements [0, n) of an 8-element slice written from f at element stride sd.
template <typename DT>
__device__ __forceinline__ void store_row8_part(DT* p, int64_t sd, int n, const float* f)
{
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if (e < n) {
            DT v;
            from_f32(f[e], v);
            p[e * sd] = v;
        }
    }
}

template <typename DT>
__device__ __forceinline__ void cvt8(const uint4& lo, const uint4& hi, float* f)
{
    if constexpr (sizeof(DT) == 2) {
        unpack8(lo, DT{}, f);
    } else {
        f[0] = __uint_as_float(lo.x); f[1] = __uint_as_float(lo.y);
        f[2] = __uint_as_float(lo.z); f[3] = __uint_as_float(lo.w);
        f[4] = __uint_as_float(hi.x); f[5] = __uint_as_float(hi.y);
        f[6] = __uint_as_float(hi.z); f[7] = __uint_as_float(hi.w);
    }
}

template <typename DT, bool VEC>
__device__ __forceinline__ void store_row8(DT* p, int64_t sd, const float* f)
{
    DT v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) from_f32(f[e], v[e]);
    if constexpr (VEC) {
        if constexpr (sizeof(DT) == 2) {
            *reinterpret_cast<uint4*>(p) = __builtin_bit_cast(uint4, v);
        } else {
            *reinterpret_cast<float4*>(p) = make_float4(f[0], f[1], f[2], f[3]);
            *reinterpret_cast<float4*>(p + 4) = make_float4(f[4], f[5], f[6], f[7]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) p[e * sd] = v[e];
    }
}

// ---------------------------------------------------------------- reductions
// Sum over the LPN lanes that share one neighbour (LPN in {4, 8, 16, 32}), with DPP: quad_perm
// xor 1 and xor 2 sum each quad; row_half_mirror then adds the other quad of the 8-lane
// group and row_mirror the other half of the 16-lane row; for 32 lanes one shuffle adds the
// other row. Every DPP pattern reads a valid lane, so bound_ctrl changes nothing; written as
// update_dpp(0, x, ...) the compiler folds each move into the add (one v_add_f32_dpp per
// level).
template <int CTRL>
__device__ __forceinline__ float dpp(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

template <int LPN>
__device__ __forceinline__ float group_sum(float x)
{
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    if constexpr (LPN >= 8) x += dpp<0x141>(x);
    if constexpr (LPN >= 16) x += dpp<0x140>(x);
    if constexpr (LPN >= 32) x += __shfl_xor(x, 16, 64);
    return x;
}

// Reduce over the 64/LPN neighbour groups of the wave (lanes that differ in bits >= LPN).
template <int LPN, bool MAX>
__device__ __forceinline__ float across_groups(float x)
{
#pragma unroll
    for (int o = LPN; o < 64; o <<= 1) {
        const float y = __shfl_xor(x, o, 64);
        x = MAX ? fmaxf(x, y) : x + y;
    }
    return x;
}

// Dot product of 8 query dims with 8 key dims (raw 16-byte words; fp32 uses lo and hi).
template <typename DT>
__device__ __forceinline__ float dot8(const uint4& qlo, const uint4& qhi, const uint4& klo,
                                      const uint4& khi)
{
    if constexpr (__is_same(DT, bf16_t)) {
        typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 v2;
        float d = 0.0f;
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, qlo.x), __builtin_bit_cast(v2, klo.x), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, qlo.y), __builtin_bit_cast(v2, klo.y), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, qlo.z), __builtin_bit_cast(v2, klo.z), d, false);
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, qlo.w), __builtin_bit_cast(v2, klo.w), d, false);
        return d;
    } else if constexpr (__is_same(DT, _Float16)) {
        typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 v2;
        float d = 0.0f;
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, qlo.x), __builtin_bit_cast(v2, klo.x), d, false);
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, qlo.y), __builtin_bit_cast(v2, klo.y), d, false);
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, qlo.z), __builtin_bit_cast(v2, klo.z), d, false);
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, qlo.w), __builtin_bit_cast(v2, klo.w), d, false);
        return d;
    } else {
        float q[8], k[8];
        cvt8<float>(qlo, qhi, q);
        cvt8<float>(klo, khi, k);
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = fmaf(q[e], k[e], d);
        return d;
    }
}

template <int N>   // rotate right by N lanes within each 16-lane row
__device__ __forceinline__ float dpp_ror(float x)
{
    return dpp<0x120 + N>(x);
}

// op over the lane groups of the wave (groups = lanes with equal bits below LPN): DPP
// row_ror inside each 16-lane row, then xor-16 / xor-32 shuffles across rows (xor-32 only
// for 32-lane groups). (The gfx950 v_permlane{16,32}_swap builtins would avoid the shuffles,
// but this toolchain folds their two results into one when both feed the same expression.)
template <int LPN, bool MAX>
__device__ __forceinline__ float group_allreduce(float x)
{
    if constexpr (LPN <= 4) { const float y = dpp_ror<4>(x); x = MAX ? fmaxf(x, y) : x + y; }
    if constexpr (LPN <= 8) { const float y = dpp_ror<8>(x); x = MAX ? fmaxf(x, y) : x + y; }
#pragma unroll
    for (int o = LPN > 16 ? LPN : 16; o < 64; o <<= 1) {
        const float y = __shfl_xor(x, o, 64);
        x = MAX ? fmaxf(x, y) : x + y;
    }
    return x;
}

template <typename DT>
__device__ __forceinline__ void ld16(const char* base, uint32_t off, uint4& lo, uint4& hi)
{
    lo = *reinterpret_cast<const uint4*>(base + off);
    if constexpr (sizeof(DT) == 4) hi = *reinterpret_cast<const uint4*>(base + off + 16u);
    else hi = make_uint4(0, 0, 0, 0);
}

// acc[0..7] += pa * va[0..7] + pb * vb[0..7]  (two neighbours of one lane group)
template <typename DT>
__device__ __forceinline__ void pv2(float* acc, float pa, float pb, const uint4& valo, const uint4& vahi,
                                    const uint4& vblo, const uint4& vbhi)
{
    if constexpr (__is_same(DT, bf16_t)) {
        typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 v2;
        const v2 pp = {(__bf16)pa, (__bf16)pb};
        const uint32_t a[4] = {valo.x, valo.y, valo.z, valo.w};
        const uint32_t b[4] = {vblo.x, vblo.y, vblo.z, vblo.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t lo = __builtin_amdgcn_perm(b[w], a[w], 0x05040100u);   // (a.lo, b.lo)
            const uint32_t hi = __builtin_amdgcn_perm(b[w], a[w], 0x07060302u);   // (a.hi, b.hi)
            acc[2 * w] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, lo), pp, acc[2 * w], false);
            acc[2 * w + 1] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, hi), pp, acc[2 * w + 1], false);
        }
    } else if constexpr (__is_same(DT, _Float16)) {
        typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 v2;
        const v2 pp = {(_Float16)pa, (_Float16)pb};
        const uint32_t a[4] = {valo.x, valo.y, valo.z, valo.w};
        const uint32_t b[4] = {vblo.x, vblo.y, vblo.z, vblo.w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t lo = __builtin_amdgcn_perm(b[w], a[w], 0x05040100u);
            const uint32_t hi = __builtin_amdgcn_perm(b[w], a[w], 0x07060302u);
            acc[2 * w] = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, lo), pp, acc[2 * w], false);
            acc[2 * w + 1] = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, hi), pp, acc[2 * w + 1], false);
        }
    } else {
        float fa[8], fb[8];
        cvt8<float>(valo, vahi, fa);
        cvt8<float>(vblo, vbhi, fb);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(pb, fb[e], fmaf(pa, fa[e], acc[e]));
    }
}

}  // namespace
}  // namespace wf
