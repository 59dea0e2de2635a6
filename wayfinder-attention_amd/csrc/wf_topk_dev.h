// wf_topk_dev.h -- device code of the causal top-K retrieval (gfx950), shared by the
// retrieval kernels (wf_topk.hip) and the single-pass fused kernel (wf_fused.hip).
//
//
// Replaces routing_attention/kernels/causal_topk.py:132-171 (_causal_topk_row_blocked) and
// :37-57 (_finalize_causal_topk). Where the reference writes a (B, block_m, i1) fp32 score
// block to HBM per row block and runs torch.topk over it, this kernel never materialises
// scores outside LDS. One workgroup = 4 waves = one block of 16 query rows:
//
//  1. screen   The 4 waves split the block's causal key prefix into 16-key steps (wave w
//              takes steps w, w+4, ...). One v_mfma_f32_16x16x32_{bf16,f16} (eight
//              16x16x4 f32 for fp32 inputs) per 32 address dims scores a 16 keys x 16 rows
//              tile. A key becomes a candidate of a row when its MFMA score reaches the
//              row's screening threshold; candidates (MFMA score, key) are appended with
//              LDS atomics to the row's pool, shared by the 4 waves.
//  2. prune    When a pool is nearly full (checked at a workgroup barrier after every
//              step), all 16 rows are pruned in parallel, 16 lanes per row: a 128-bin
//              histogram of the pool's MFMA scores gives a value theta' with at least K
//              entries above it; entries below theta' - 2 eps are dropped and the row's
//              threshold becomes theta' - 2 eps. eps bounds |MFMA score - exact score|.
//  3. exact    At the end (or when near-ties keep a pool from shrinking) the pool is
//              rescored exactly -- fp32 fma chain over the address dims in ascending
//              order, the oracle's definition of the score -- and the K best under
//              (score desc, index asc) are radix-selected from the 64-bit keys.
//  4. emit     The K winners are bitonic-sorted into canonical order and written with
//              the reference's pad indices for rows that have fewer than K causal keys.
//              For 64 < K <= 128 with at most 144 entries left after the final prune,
//              and for 128 < K <= 256 with at most 320, the selection of step 3 and this
//              sort are one network (emit_row_merge).
//
// Exactness: let E be the exact top-K of the keys seen so far and s_K its K-th score. The
// pool always contains E: a pool holding K entries with MFMA score >= theta' has exact
// K-th score >= theta' - eps, so s_K >= theta' - eps and every key that can still enter E
// (exact score >= s_K, ties included since waves see keys out of index order) has MFMA
// score >= theta' - 2 eps = the threshold. The final choice uses exact scores only.
#pragma once

#include <type_traits>

#include "wf_internal.h"

namespace wf {
namespace {

#ifndef WF_TOPK_WAVES
#define WF_TOPK_WAVES 4
#endif

constexpr int kRows = 16;                              // query rows per workgroup (MFMA N)
constexpr int kTopkWaves = WF_TOPK_WAVES;                  // waves per workgroup (split the keys)
constexpr int kSeedSteps = 128;                        // sampled key steps of a seed, at most
constexpr int kMaxStretch = 8;                         // pool check interval of a seeded pass 0, at most x
constexpr int kBins = 128;                             // pruning histogram bins per row
constexpr int kPD = 4;                                 // key steps each wave keeps in flight (2 for R > 128)
constexpr int kStepMax = 16 * kTopkWaves;                  // appends per row in one key step of every wave, at most
// |MFMA score - exact score| <= 2 * n * 2^-24 * sum_d |q_d k_d| for n accumulated terms with
// round-to-nearest in both (2^-23 per term with truncating adds); the bound used is 2^-20
// per term: 8x the round-to-nearest bound, 4x the truncating one
constexpr float kEpsPerTerm = 1.0f / 1048576.0f;
constexpr float kTiny = 7.888609052210118e-31f;        // 2^-100: covers denormal flushing

// ------------------------------------------------------------------ operand loads
// Eight consecutive address dims [d0, d0+8) of one row as raw bits: lo holds them for
// 16-bit types; lo,hi for fp32. Dims >= R read as zero.
template <typename DT, bool VEC>
__device__ __forceinline__ void load8(const DT* row, int64_t sr, int d0, int R, uint4& lo, uint4& hi)
{
    lo = make_uint4(0, 0, 0, 0);
    hi = make_uint4(0, 0, 0, 0);
    if constexpr (sizeof(DT) == 2) {
        if constexpr (VEC) {
            if (d0 < R) lo = *reinterpret_cast<const uint4*>(row + d0);
        } else {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = d0 + e;
                uint16_t v = 0;
                if (d < R) v = *reinterpret_cast<const uint16_t*>(row + d * sr);
                w[e >> 1] |= uint32_t(v) << (16 * (e & 1));
            }
            lo = make_uint4(w[0], w[1], w[2], w[3]);
        }
    } else {
        if constexpr (VEC) {
            if (d0 < R) {
                lo = *reinterpret_cast<const uint4*>(row + d0);
                hi = *reinterpret_cast<const uint4*>(row + d0 + 4);
            }
        } else {
            uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = d0 + e;
                if (d < R) w[e] = __float_as_uint(*reinterpret_cast<const float*>(row + d * sr));
            }
            lo = make_uint4(w[0], w[1], w[2], w[3]);
            hi = make_uint4(w[4], w[5], w[6], w[7]);
        }
    }
}

template <typename DT>
__device__ __forceinline__ void to_f32x8(const uint4& lo, const uint4& hi, float* f)
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

// One 32-dim chunk of the 16x16 score tile. A = keys (M = 16 keys, lane l: key l%16, dims
// 8*(l/16)..+7), B = queries (N = 16 rows, lane l: row l%16, same dims). A and B use the
// same (lane group, element) -> dim map, so the contraction covers each dim exactly once.
template <typename DT>
__device__ __forceinline__ f32x4_t mfma_chunk(const uint4& alo, const uint4& ahi,
                                              const uint4& blo, const uint4& bhi, f32x4_t acc)
{
    if constexpr (__is_same(DT, bf16_t)) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, alo),
                                                       __builtin_bit_cast(bf16x8_t, blo), acc, 0, 0, 0);
    } else if constexpr (__is_same(DT, _Float16)) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, alo),
                                                      __builtin_bit_cast(f16x8_t, blo), acc, 0, 0, 0);
    } else {
        // fp32: eight K=4 steps; step s feeds dim 8*(l/16)+s of lane group l/16 as k=l/16.
        float a[8], b[8];
        to_f32x8<float>(alo, ahi, a);
        to_f32x8<float>(blo, bhi, b);
#pragma unroll
        for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
        return acc;
    }
}

// Exact score: acc = fmaf(q[d], k[d], acc) for d = 0..R-1 from acc = 0 (q in LDS as fp32).
// RP (a multiple of 32) bounds R; every key chunk is loaded before the chain starts.
template <typename DT, bool VEC, int RP>
__device__ __forceinline__ float exact_score(const float* q, const DT* krow, int64_t sr, int R)
{
    float acc = 0.0f;
    if constexpr (VEC) {
        constexpr int NC = RP / 8;
        uint4 lo[NC], hi[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            lo[c] = make_uint4(0, 0, 0, 0);
            hi[c] = lo[c];
            if (8 * c < R) load8<DT, true>(krow, 1, 8 * c, R, lo[c], hi[c]);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (8 * c >= R) break;
            float kf[8];
            to_f32x8<DT>(lo[c], hi[c], kf);
            const float4 qa = *reinterpret_cast<const float4*>(q + 8 * c);
            const float4 qb = *reinterpret_cast<const float4*>(q + 8 * c + 4);
            acc = fmaf(qa.x, kf[0], acc); acc = fmaf(qa.y, kf[1], acc);
            acc = fmaf(qa.z, kf[2], acc); acc = fmaf(qa.w, kf[3], acc);
            acc = fmaf(qb.x, kf[4], acc); acc = fmaf(qb.y, kf[5], acc);
            acc = fmaf(qb.z, kf[6], acc); acc = fmaf(qb.w, kf[7], acc);
        }
    } else {
        for (int d = 0; d < R; ++d) acc = fmaf(q[d], to_f32(krow[d * sr]), acc);
    }
    return acc;
}

__device__ __forceinline__ uint64_t make_key(float s, uint32_t j)
{
    return (uint64_t(ord_f32(s)) << 32) | uint64_t(0xffffffffu - j);
}

// ------------------------------------------------------------------ 16-lane row groups
// In the row-parallel phases query row r of the block is owned by lanes 16*(r%4)..+15 of
// wave r/4, i.e. by one 16-lane DPP row, so every cross-lane step is a DPP move (no LDS
// round trip): row_ror rotations for all-reduces, row_shl shifts for suffix scans.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t x)
{
    return uint32_t(__builtin_amdgcn_mov_dpp(int(x), CTRL, 0xf, 0xf, false));
}
template <int CTRL>   // shifted-in lanes read 0
__device__ __forceinline__ uint32_t dpp32z(uint32_t x)
{
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(x), CTRL, 0xf, 0xf, true));
}
constexpr int kRor8 = 0x128, kRor4 = 0x124, kRor2 = 0x122, kRor1 = 0x121;

__device__ __forceinline__ float row_max16(float x)
{
    x = fmaxf(x, __uint_as_float(dpp32<kRor8>(__float_as_uint(x))));
    x = fmaxf(x, __uint_as_float(dpp32<kRor4>(__float_as_uint(x))));
    x = fmaxf(x, __uint_as_float(dpp32<kRor2>(__float_as_uint(x))));
    x = fmaxf(x, __uint_as_float(dpp32<kRor1>(__float_as_uint(x))));
    return x;
}
__device__ __forceinline__ float row_min16(float x)
{
    x = fminf(x, __uint_as_float(dpp32<kRor8>(__float_as_uint(x))));
    x = fminf(x, __uint_as_float(dpp32<kRor4>(__float_as_uint(x))));
    x = fminf(x, __uint_as_float(dpp32<kRor2>(__float_as_uint(x))));
    x = fminf(x, __uint_as_float(dpp32<kRor1>(__float_as_uint(x))));
    return x;
}
__device__ __forceinline__ int row_max16_i32(int x)
{
    x = max(x, int(dpp32<kRor8>(uint32_t(x))));
    x = max(x, int(dpp32<kRor4>(uint32_t(x))));
    x = max(x, int(dpp32<kRor2>(uint32_t(x))));
    x = max(x, int(dpp32<kRor1>(uint32_t(x))));
    return x;
}
__device__ __forceinline__ int row_sum16_i32(int x)
{
    x += int(dpp32<kRor8>(uint32_t(x)));
    x += int(dpp32<kRor4>(uint32_t(x)));
    x += int(dpp32<kRor2>(uint32_t(x)));
    x += int(dpp32<kRor1>(uint32_t(x)));
    return x;
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t x)
{
    return (uint64_t(dpp32<CTRL>(uint32_t(x >> 32))) << 32) | dpp32<CTRL>(uint32_t(x));
}
__device__ __forceinline__ uint64_t row_max16_u64(uint64_t x)
{
    uint64_t y;
    y = dpp64<kRor8>(x); x = y > x ? y : x;
    y = dpp64<kRor4>(x); x = y > x ? y : x;
    y = dpp64<kRor2>(x); x = y > x ? y : x;
    y = dpp64<kRor1>(x); x = y > x ? y : x;
    return x;
}
__device__ __forceinline__ uint64_t row_min16_u64(uint64_t x)
{
    uint64_t y;
    y = dpp64<kRor8>(x); x = y < x ? y : x;
    y = dpp64<kRor4>(x); x = y < x ? y : x;
    y = dpp64<kRor2>(x); x = y < x ? y : x;
    y = dpp64<kRor1>(x); x = y < x ? y : x;
    return x;
}
// sum of x over the lanes of the row with a higher sub-lane index (row_shl:n brings lane
// i+n to lane i, zero past the end of the row)
__device__ __forceinline__ int row_suffix_excl16(int x)
{
    uint32_t s = uint32_t(x);
    s += dpp32z<0x101>(s);
    s += dpp32z<0x102>(s);
    s += dpp32z<0x104>(s);
    s += dpp32z<0x108>(s);
    return int(s) - x;
}
__device__ __forceinline__ uint32_t row_bits16(uint64_t ballot)
{
    return uint32_t(ballot >> (lane_id() & 48)) & 0xffffu;
}
// value of lane u ^ LX within the 16-lane row (LX in {1, 2, 4, 8})
template <int LX>
__device__ __forceinline__ uint64_t xor16_u64(uint64_t x, int u)
{
    if constexpr (LX == 1) return dpp64<0xB1>(x);       // quad_perm [1,0,3,2]
    else if constexpr (LX == 2) return dpp64<0x4E>(x);  // quad_perm [2,3,0,1]
    else if constexpr (LX == 8) return dpp64<kRor8>(x);
    else {                                              // row_ror:4 / :12, by lane
        const uint64_t a = dpp64<kRor4>(x), b = dpp64<0x12C>(x);
        return (u & 4) ? a : b;
    }
}

// value of lane u ^ lx within the 16-lane row, lx in {1, 2, 3, 4, 7, 8, 15} (a compile-time
// constant once the caller's loops unroll)
__device__ __forceinline__ uint64_t lane_xor16_u64(uint64_t x, int lx, int u)
{
    switch (lx) {
    case 1: return xor16_u64<1>(x, u);
    case 2: return xor16_u64<2>(x, u);
    case 3: return dpp64<0x1B>(x);       // quad_perm [3,2,1,0]
    case 4: return xor16_u64<4>(x, u);
    case 7: return dpp64<0x141>(x);      // row_half_mirror
    case 8: return xor16_u64<8>(x, u);
    default: return dpp64<0x140>(x);     // row_mirror: lane 15 - u
    }
}

struct Entry {
    float s;      // MFMA score while pending, exact score after rescoring
    uint32_t j;   // key index
};

template <int RP, int POOL>
struct TopkSmem {
    float q[kRows][RP];            // fp32 query rows (exact rescoring)
    // candidate pool per row + 20 dummy slots (sinks of masked writes: POOL + g for appends,
    // POOL + 4 + u for prune lanes); a row stride of 1064 dwords spreads rows over the banks
    Entry pool[kRows][POOL + 20];
    // per-row histogram (pruning, radix select) + one dummy bin per lane (kBins + u): a masked
    // atomic lands on its own bank instead of serialising on a shared address
    uint32_t hist[kRows][kBins + 16];
    int cnt[kRows];                // pool fill
    float thr[kRows];              // screening threshold (-inf until K candidates are known)
    float eps[kRows];              // |MFMA score - exact score| bound of the row
    float seed[kRows];             // speculative screening threshold (-inf: none)
    int fail[kRows];               // the row's seed was too high: screen it again from -inf
};

// Largest bin b (of the row's kBins-bin histogram) whose suffix count C(b) reaches `need`;
// also C(b+1) (entries strictly above) and the count of bin b. Exactly one lane of the row
// holds the crossing; its values reach the other lanes through row maxima.
__device__ __forceinline__ void find_boundary(const uint32_t* hist, int u, int need, int& b,
                                              int& gt, int& eq)
{
    const uint4 h0 = reinterpret_cast<const uint4*>(hist)[2 * u];
    const uint4 h1 = reinterpret_cast<const uint4*>(hist)[2 * u + 1];
    const int h[8] = {int(h0.x), int(h0.y), int(h0.z), int(h0.w),
                      int(h1.x), int(h1.y), int(h1.z), int(h1.w)};
    int tot = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) tot += h[k];
    const int above = row_suffix_excl16(tot);
    const bool has = above < need && above + tot >= need;
    int cum = above, bb = -1, g = 0, e = 0;
#pragma unroll
    for (int k = 7; k >= 0; --k) {
        if (bb < 0 && cum + h[k] >= need) { bb = 8 * u + k; g = cum; e = h[k]; }
        cum += h[k];
    }
    b = row_max16_i32(has ? bb : -1);
    gt = row_max16_i32(has ? g : -1);
    eq = row_max16_i32(has ? e : -1);
}

// Entry <-> 64-bit selection key: (order-preserving score bits, complemented index), so a
// larger key is a better entry under (score desc, index asc).
__device__ __forceinline__ Entry key_entry(uint64_t k)
{
    return Entry{unord_f32(uint32_t(k >> 32)), 0xffffffffu - uint32_t(k)};
}

// Histogram pruning of a row whose pool holds c > K entries. Returns false when the scores
// are too close together to separate (the caller then rescores exactly); otherwise the
// pool is cut to the entries >= theta' - 2 eps, c_out is the new count (uniform over the
// row's lanes) and, from lane u == 0, cnt / thr are stored for the other waves. Each lane
// reads EPR slots (c <= 16 EPR).
template <int EPR, int POOL>
__device__ bool prune_row(Entry* pool, uint32_t* hist, int c, int& c_out, int& cnt,
                          float& thr, float eps, int K, int u)
{
    c_out = c;
    // every slot is read unconditionally (slots >= c hold stale data and are masked below), so
    // the reads issue back to back and the row waits on LDS once
    uint2 ent[EPR];
#pragma unroll
    for (int m = 0; m < EPR; ++m) ent[m] = reinterpret_cast<const uint2*>(pool)[u + 16 * m];
    // masked slots become NaN: every comparison below is false for them (and for NaN scores)
    float s[EPR];
    float lo = __builtin_inff(), hi = -__builtin_inff();
#pragma unroll
    for (int m = 0; m < EPR; ++m) {
        s[m] = u + 16 * m < c ? __uint_as_float(ent[m].x) : __builtin_nanf("");
        lo = fminf(lo, s[m]);   // minNum / maxNum: NaN entries leave the bound unchanged
        hi = fmaxf(hi, s[m]);
    }
    lo = row_min16(lo);
    hi = row_max16(hi);
    const float span = hi - lo;
    if (!(span > 0.0009765625f * fmaxf(fabsf(hi), fabsf(lo))) || !(span < 3.0e38f)) return false;
    const float inv = float(kBins) / span;
    reinterpret_cast<uint4*>(hist)[2 * u] = make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(hist)[2 * u + 1] = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int m = 0; m < EPR; ++m) {   // masked entries count in the lane's dummy bin
        int bin = int((s[m] - lo) * inv);
        bin = bin < 0 ? 0 : (bin > kBins - 1 ? kBins - 1 : bin);
        atomicAdd(&hist[s[m] >= lo ? bin : kBins + u], 1u);
    }
    int b, gt, eq;
    find_boundary(hist, u, K, b, gt, eq);
    // one bin of slack absorbs the rounding of the bin computation
    float theta = b >= 1 ? lo + float(b - 1) * (span / float(kBins)) : lo;
    int keep_lane = 0;   // this lane's survivors of the linear cut, reused by the compaction
#pragma unroll
    for (int m = 0; m < EPR; ++m) keep_lane += s[m] >= theta - 2.0f * eps ? 1 : 0;
    const int keep_lin = row_sum16_i32(keep_lane);
    bool raised = false;   // uniform over the row
    if (keep_lin > K + K / 4) {
        // the cut would keep too much: heavy-tailed scores, whose few large values stretch
        // [lo, hi] and crowd the rest into the lowest bins. Second histogram in the
        // order-preserving integer image of the scores (2^sh consecutive images per bin:
        // relative resolution); integer arithmetic makes its bin edges exact, so an entry in
        // bin >= b2 has score >= theta2
        const uint32_t olo = ord_f32(lo), ohi = ord_f32(hi);
        const int sh = max(0, 32 - __clz(int(ohi - olo)) - 7);
        reinterpret_cast<uint4*>(hist)[2 * u] = make_uint4(0, 0, 0, 0);
        reinterpret_cast<uint4*>(hist)[2 * u + 1] = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int m = 0; m < EPR; ++m) {
            const uint32_t bin = (ord_f32(s[m]) - olo) >> sh;
            atomicAdd(&hist[s[m] >= lo ? bin : uint32_t(kBins + u)], 1u);
        }
        int b2, gt2, eq2;
        find_boundary(hist, u, K, b2, gt2, eq2);
        const float theta2 = unord_f32(olo + (uint32_t(b2) << sh));
        if (theta2 > theta) {
            theta = theta2;
            raised = true;
        }
    }
    const float kappa = theta - 2.0f * eps;
    // compaction: each lane's survivors go, in order, after those of the higher lanes of the
    // row (all entries are in registers, so the in-place writes cannot clobber unread ones);
    // dropped entries are written to the lane's dummy slot
    int mine = keep_lane;
    if (raised) {
        mine = 0;
#pragma unroll
        for (int m = 0; m < EPR; ++m) mine += s[m] >= kappa ? 1 : 0;
    }
    int pos = row_suffix_excl16(mine);
    const int total = row_max16_i32(pos + mine);
#pragma unroll
    for (int m = 0; m < EPR; ++m) {
        const bool sel = s[m] >= kappa;
        reinterpret_cast<uint2*>(pool)[sel ? pos : POOL + 4 + u] = ent[m];
        pos += sel ? 1 : 0;
    }
    c_out = total;
    if (u == 0) { cnt = total; thr = kappa; }
    return true;
}

// prune_row sized to the fullest pool among the wave's four rows (cw, wave-uniform, so the
// wave takes one branch): a final prune sees ~220 entries and an in-loop one 385-450, and
// every slot read costs the histogram, count and compaction work of an entry (config 4:
// final prune 3.6 -> 2.7 us per block). SIZED = false reads the whole pool: the K = 256
// kernels, where the extra variants push the register allocator into scratch spills
// (88 bytes per lane, config 5 1.5x slower).
template <bool SIZED, int POOL>
__device__ bool prune_sized(Entry* pool, uint32_t* hist, int c, int cw, int& c_out, int& cnt,
                            float& thr, float eps, int K, int u)
{
    if constexpr (SIZED) {
        if (POOL / 16 > 16 && cw <= 16 * 16) return prune_row<16, POOL>(pool, hist, c, c_out, cnt, thr, eps, K, u);
        if (POOL / 16 > 24 && cw <= 16 * 24) return prune_row<24, POOL>(pool, hist, c, c_out, cnt, thr, eps, K, u);
        if (POOL / 16 > 28 && cw <= 16 * 28) return prune_row<28, POOL>(pool, hist, c, c_out, cnt, thr, eps, K, u);
    }
    return prune_row<POOL / 16, POOL>(pool, hist, c, c_out, cnt, thr, eps, K, u);
}

// largest value of v over the wave's four 16-lane rows (v uniform within each row)
__device__ __forceinline__ int wave_max_of_rows(int v)
{
    const int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
    const int c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
    return max(max(a, b), max(c, d));
}

// Exact rescoring of a row's c pool entries: pool[e].s becomes the exact score. The VEC
// path keeps NBR key rows per lane in flight at once (the chains wait on one round trip per
// batch) and walks the address dims in ascending order, one 8-dim chunk of q at a time, for
// all NBR chains together.
template <typename DT, bool VEC, int RP>
__device__ void rescore_row(Entry* pool, int c, const float* q, const DT* kb, int64_t kst,
                            int64_t ksr, int R, int u)
{
    if constexpr (VEC) {   // R == RP: every chunk lies inside the row
        constexpr int NC = RP / 8;
        // chunks loaded at once: all of them up to R = 128, else groups of 16 (the chain then
        // continues over the next group, so the dims are still summed in ascending order)
        constexpr int NCG = NC < 16 ? NC : 16;
        constexpr int U4 = NCG * (sizeof(DT) == 4 ? 2 : 1);   // 16-byte loads per key row and group
        // key rows in flight per lane: 2 for 16-bit keys at R = 32 (measured faster than 4:
        // the phase is bound by its VALU work, not by load round trips), else 16 / U4
        constexpr int NBR = U4 >= 16 ? 1 : (U4 == 4 ? 2 : 16 / U4);
        for (int e0 = 0; e0 < c; e0 += 16 * NBR) {
            const DT* krow[NBR];
#pragma unroll
            for (int m = 0; m < NBR; ++m) {
                const int e = e0 + u + 16 * m;
                const uint32_t jr = pool[min(e, c - 1)].j;   // unconditional read: no LDS wait per entry
                krow[m] = kb + int64_t(e < c ? jr : 0u) * kst;
            }
            float acc[NBR];
#pragma unroll
            for (int m = 0; m < NBR; ++m) acc[m] = 0.0f;
#pragma unroll
            for (int c0 = 0; c0 < NC; c0 += NCG) {
                uint4 lo[NBR][NCG], hi[NBR][NCG];
#pragma unroll
                for (int m = 0; m < NBR; ++m) {
#pragma unroll
                    for (int cc = 0; cc < NCG; ++cc) {
                        lo[m][cc] = *reinterpret_cast<const uint4*>(krow[m] + 8 * (c0 + cc));
                        if constexpr (sizeof(DT) == 4) hi[m][cc] = *reinterpret_cast<const uint4*>(krow[m] + 8 * (c0 + cc) + 4);
                        else hi[m][cc] = make_uint4(0, 0, 0, 0);
                    }
                }
#pragma unroll
                for (int cc = 0; cc < NCG; ++cc) {
                    const float4 qa = *reinterpret_cast<const float4*>(q + 8 * (c0 + cc));
                    const float4 qb = *reinterpret_cast<const float4*>(q + 8 * (c0 + cc) + 4);
#pragma unroll
                    for (int m = 0; m < NBR; ++m) {
                        float kf[8];
                        to_f32x8<DT>(lo[m][cc], hi[m][cc], kf);
                        float a = acc[m];
                        a = fmaf(qa.x, kf[0], a); a = fmaf(qa.y, kf[1], a);
                        a = fmaf(qa.z, kf[2], a); a = fmaf(qa.w, kf[3], a);
                        a = fmaf(qb.x, kf[4], a); a = fmaf(qb.y, kf[5], a);
                        a = fmaf(qb.z, kf[6], a); a = fmaf(qb.w, kf[7], a);
                        acc[m] = a;
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < NBR; ++m) {
                const int e = e0 + u + 16 * m;
                if (e < c) pool[e].s = acc[m];
            }
        }
    } else {
        for (int e = u; e < c; e += 32) {   // two independent chains per iteration
            const bool two = e + 16 < c;
            const uint32_t j0 = pool[e].j;
            const uint32_t j1 = two ? pool[e + 16].j : j0;
            const float s0 = exact_score<DT, VEC, RP>(q, kb + int64_t(j0) * kst, ksr, R);
            const float s1 = exact_score<DT, VEC, RP>(q, kb + int64_t(j1) * kst, ksr, R);
            pool[e].s = s0;
            if (two) pool[e + 16].s = s1;
        }
    }
}

// Exact selection of the min(K, c) best of a row's c exactly scored entries by (score desc,
// index asc), radix-selected on the 64-bit keys (EPR >= ceil(c / 16) entries per lane); the
// winners end up in pool[0..kept). Returns kept (uniform over the row); lane u == 0 stores
// cnt and the exact threshold s_K - eps.
template <int EPR>
__device__ int select_row(Entry* pool, uint32_t* hist, int c, int& cnt, float& thr, float eps,
                          int K, int u)
{
    uint64_t key[EPR];
#pragma unroll
    for (int m = 0; m < EPR; ++m) {   // unconditional reads, masked: one LDS wait for the row
        const uint2 en = reinterpret_cast<const uint2*>(pool)[u + 16 * m];
        key[m] = u + 16 * m < c ? make_key(__uint_as_float(en.x), en.y) : 0ull;   // real keys are > 0
    }
    uint64_t prefix = 0, pmask = 0;
    if (c > K) {
        uint64_t kmax = 0, kmin = ~0ull;
#pragma unroll
        for (int m = 0; m < EPR; ++m)
            if (u + 16 * m < c) { kmax = key[m] > kmax ? key[m] : kmax; kmin = key[m] < kmin ? key[m] : kmin; }
        kmax = row_max16_u64(kmax);
        kmin = row_min16_u64(kmin);
        const int top = 63 - __clzll((long long)(kmax ^ kmin));   // keys are distinct
        pmask = top >= 63 ? 0ull : ~((2ull << top) - 1ull);
        prefix = kmax & pmask;
        int need = K;
        for (int shift = top - 6; shift > -7; shift -= 7) {
            reinterpret_cast<uint4*>(hist)[2 * u] = make_uint4(0, 0, 0, 0);
            reinterpret_cast<uint4*>(hist)[2 * u + 1] = make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int m = 0; m < EPR; ++m) {   // entries off the prefix count in a dummy bin
                const uint32_t d = shift >= 0 ? uint32_t(key[m] >> shift) & 127u
                                              : uint32_t(key[m] << (-shift)) & 127u;
                const bool in = u + 16 * m < c && (key[m] & pmask) == prefix;
                atomicAdd(&hist[in ? d : uint32_t(kBins + u)], 1u);
            }
            int d, gt, eq;
            find_boundary(hist, u, need, d, gt, eq);
            need -= gt;
            prefix |= shift >= 0 ? (uint64_t(d) << shift) : (uint64_t(d) >> (-shift));
            pmask |= shift >= 0 ? (127ull << shift) : (127ull >> (-shift));
            if (eq == need) break;
        }
    }
    int base = 0;
    uint64_t kmin_sel = ~0ull;
    const uint32_t lt = (1u << u) - 1u;
#pragma unroll
    for (int m = 0; m < EPR; ++m) {
        const bool sel = u + 16 * m < c && (key[m] & pmask) >= prefix;
        const uint32_t bits = row_bits16(__ballot(sel));
        if (sel) {
            pool[base + __popc(bits & lt)] = key_entry(key[m]);
            kmin_sel = key[m] < kmin_sel ? key[m] : kmin_sel;
        }
        base += __popc(bits);
    }
    kmin_sel = row_min16_u64(kmin_sel);
    if (u == 0) {
        cnt = base;
        thr = base >= K ? key_entry(kmin_sel).s - eps : -__builtin_inff();
    }
    return base;
}

// Exact rescoring of a row's c pool entries and exact selection of its min(K, c) best by
// (score desc, index asc); the winners end up in pool[0..kept) with exact scores. Returns
// kept (uniform over the row); lane u == 0 stores cnt and the exact threshold s_K - eps.
// The selection reads ceil(cw / 16) entries per lane, cw >= c being the fullest pool among
// the wave's rows (wave-uniform, so the wave takes one branch): after a final prune a
// K = 128 pool holds ~135 entries. SIZED adds the 9-entry variant (K <= 128 kernels); the
// K = 256 kernels read 20 entries per lane when the wave's pools hold at most 320 (a final
// K = 256 pool holds ~290 entries).
template <typename DT, bool VEC, int RP, int POOL, bool SIZED>
__device__ int exact_row(Entry* pool, uint32_t* hist, int c, int cw, int& cnt, float& thr,
                         float eps, const float* q, const DT* kb, int64_t kst, int64_t ksr, int R,
                         int K, int u)
{
    rescore_row<DT, VEC, RP>(pool, c, q, kb, kst, ksr, R, u);
    if constexpr (SIZED) {
        if (cw <= 16 * 9) return select_row<9>(pool, hist, c, cnt, thr, eps, K, u);
    } else {
        if (cw <= 16 * 20) return select_row<20>(pool, hist, c, cnt, thr, eps, K, u);
    }
    if (cw <= 16 * 12) return select_row<12>(pool, hist, c, cnt, thr, eps, K, u);
    return select_row<POOL / 16>(pool, hist, c, cnt, thr, eps, K, u);
}

// Bitonic network in which every compare-exchange has the same direction: the first step of
// each merge pairs element i with its mirror i ^ (kk - 1) inside the 2S-block, the following
// steps pair i with i ^ jj; the lower element index keeps the larger key. Element i sits in
// lane u = i / EPL, register m = i % EPL. Partners inside the lane are registers; across
// lanes they are one DPP move (mirror: lane u ^ 1/3/7/15 and element EPL-1-m; xor: u ^
// 1/2/4/8). x = partner distance (i ^ x), kk = merge block (mirror steps only).
template <int EPL>
__device__ __forceinline__ void bitonic_stage(uint64_t (&key)[EPL], int kk, int x, bool mirror, int u)
{
    if (x < EPL) {
#pragma unroll
        for (int m = 0; m < EPL; ++m) {
            const int m2 = m ^ x;
            if (m2 <= m) continue;
            const uint64_t a = key[m], b = key[m2];
            const bool gt = a > b;
            key[m] = gt ? a : b;
            key[m2] = gt ? b : a;
        }
    } else {
        const int lx = x / EPL;                           // partner lane = u ^ lx
        const int hb = mirror ? (kk / EPL) >> 1 : lx;     // lane bit of the pair's top index bit
        const bool keep_max = (u & hb) == 0;
        uint64_t other[EPL];
#pragma unroll
        for (int m = 0; m < EPL; ++m) other[m] = lane_xor16_u64(key[mirror ? EPL - 1 - m : m], lx, u);
#pragma unroll
        for (int m = 0; m < EPL; ++m) {
            const bool gt = key[m] > other[m];
            key[m] = gt == keep_max ? key[m] : other[m];
        }
    }
}

// sorts every group of N consecutive elements (N / EPL lanes) into descending order
template <int EPL, int N>
__device__ __forceinline__ void bitonic_sort(uint64_t (&key)[EPL], int u)
{
#pragma unroll
    for (int kk = 2; kk <= N; kk <<= 1) {
#pragma unroll
        for (int jj = kk >> 1; jj > 0; jj >>= 1) {
            const bool mirror = jj == (kk >> 1);
            bitonic_stage<EPL>(key, kk, mirror ? kk - 1 : jj, mirror, u);
        }
    }
}

// sorts a bitonic group of N elements (descending, then ascending) into descending order
template <int EPL, int N>
__device__ __forceinline__ void bitonic_merge(uint64_t (&key)[EPL], int u)
{
#pragma unroll
    for (int jj = N >> 1; jj > 0; jj >>= 1) bitonic_stage<EPL>(key, N, jj, false, u);
}

template <int KP2>
__device__ void write_row(const uint64_t (&key)[KP2 / 16], int kept, int64_t row, int64_t T,
                          int64_t k_eff, int32_t* out_idx, float* out_scores, int32_t* lidx, int u);

// Element i (row-uniform) of a row's sorted keys, in every lane of the row: element i sits
// in lane i / EPL, register i % EPL.
template <int EPL>
__device__ __forceinline__ uint64_t row_element(const uint64_t (&key)[EPL], int i, int u)
{
    uint64_t v = 0;
#pragma unroll
    for (int m = 0; m < EPL; ++m) v = m == i % EPL ? key[m] : v;
    return row_max16_u64(u == i / EPL ? v : 0ull);
}

// lidx if the row's k_eff-th key (0: fewer were kept) has a score >= lidx_min, else null
__device__ __forceinline__ int32_t* lidx_gate(int32_t* lidx, uint64_t kth, float lidx_min)
{
    if (!lidx || lidx_min == -__builtin_inff()) return lidx;
    return kth != 0ull && key_entry(kth).s >= lidx_min ? lidx : nullptr;
}

// Sort row r's (exactly scored) winners into canonical order and write them plus pads.
// `row` is the query position t in its batch; out_idx/out_scores point at the batch; lidx,
// if not null, receives a copy of the index row in LDS (the row's own pool, already read).
// Returns the row's k_eff-th key in canonical order (0 if fewer than k_eff were kept); the
// LDS copy goes to lidx only if that key's score reaches lidx_min.
template <int KP2, int POOL>
__device__ uint64_t emit_row(const Entry* pool, int kept, int64_t row, int64_t T,
                             int64_t k_eff, int32_t* out_idx, float* out_scores, int32_t* lidx,
                             float lidx_min, int u)
{
    constexpr int EPL = KP2 / 16;   // elements per lane; element i = u * EPL + m
    uint64_t key[EPL];
#pragma unroll
    for (int m = 0; m < EPL; ++m) {
        const int i = u * EPL + m;   // < KP2 < POOL: read unconditionally, masked
        const uint2 en = reinterpret_cast<const uint2*>(pool)[i];
        key[m] = i < kept ? make_key(__uint_as_float(en.x), en.y) : 0ull;
    }
    bitonic_sort<EPL, KP2>(key, u);
    const uint64_t kth = row_element<EPL>(key, int(k_eff) - 1, u);
    write_row<KP2>(key, kept, row, T, k_eff, out_idx, out_scores, lidx_gate(lidx, kth, lidx_min), u);
    return kth;
}

// Exact selection fused into the sort, for c <= KP2 + NB exactly scored entries (after the
// final prune a K = 128 pool holds ~135, a K = 256 pool ~290): A = slots 0..KP2-1 is sorted
// descending and B = slots KP2..c-1 (at most NB, in the last NB / EPL lanes) descending;
// then C[i] = max(A[i], B[KP2-1 - i]) holds the KP2 largest of A and B as a bitonic
// sequence (A falls, the reversed B rises), and one bitonic merge sorts it. This replaces
// the radix select's histogram rounds with an NB-element sort, one exchange and log2(KP2)
// merge steps. B[KP2-1 - i] for element i = EPL u + m of a B lane is register EPL-1 - m of
// lane u ^ LXB (KP2 = 128, NB = 16: lanes 14, 15 and LXB = 1; KP2 = 256, NB = 64: lanes
// 12..15 and LXB = 3); the other lanes pair with lanes whose B keys are 0.
// Returns the row's k_eff-th key in canonical order (0 if fewer than k_eff were kept); the
// LDS copy goes to lidx only if that key's score reaches lidx_min.
template <int KP2, int NB, int LXB, int POOL>
__device__ uint64_t emit_row_merge(const Entry* pool, int c, int64_t row, int64_t T, int64_t k_eff,
                                   int32_t* out_idx, float* out_scores, int32_t* lidx,
                                   float lidx_min, int u)
{
    constexpr int EPL = KP2 / 16;
    static_assert(POOL >= KP2 + NB, "pool too small");
    static_assert((KP2 == 128 && NB == 16 && LXB == 1) || (KP2 == 256 && NB == 64 && LXB == 3),
                  "lane pairing of the reversed B");
    uint64_t key[EPL], bkey[EPL];
#pragma unroll
    for (int m = 0; m < EPL; ++m) {
        const int i = u * EPL + m;   // reads are unconditional (slots < KP2 + NB <= POOL), masked
        const uint2 ea = reinterpret_cast<const uint2*>(pool)[i];
        key[m] = i < c ? make_key(__uint_as_float(ea.x), ea.y) : 0ull;
        const int jb = i - (KP2 - NB);   // B entry of element i of the B lanes
        const int sb = KP2 + (jb < 0 ? 0 : jb);
        const uint2 eb = reinterpret_cast<const uint2*>(pool)[sb];
        bkey[m] = jb >= 0 && sb < c ? make_key(__uint_as_float(eb.x), eb.y) : 0ull;
    }
    bitonic_sort<EPL, KP2>(key, u);
    bitonic_sort<EPL, NB>(bkey, u);   // the B lanes hold B sorted; the other lanes hold 0
#pragma unroll
    for (int m = 0; m < EPL; ++m) {
        const uint64_t o = lane_xor16_u64(bkey[EPL - 1 - m], LXB, u);
        key[m] = o > key[m] ? o : key[m];
    }
    bitonic_merge<EPL, KP2>(key, u);
    const uint64_t kth = row_element<EPL>(key, int(k_eff) - 1, u);
    write_row<KP2>(key, c < KP2 ? c : KP2, row, T, k_eff, out_idx, out_scores,
                   lidx_gate(lidx, kth, lidx_min), u);
    return kth;
}

// Write a row's sorted keys (the first `kept` are winners) and the pads after them; with
// lidx, the same int32 row into LDS too. The keys were read from the row's pool before the
// sort, and every value written depends on them, so lidx may alias that pool.
template <int KP2>
__device__ void write_row(const uint64_t (&key)[KP2 / 16], int kept, int64_t row, int64_t T,
                          int64_t k_eff, int32_t* out_idx, float* out_scores, int32_t* lidx, int u)
{
    constexpr int EPL = KP2 / 16;
    int32_t* oi = out_idx + row * k_eff;
    float* os = out_scores ? out_scores + row * k_eff : nullptr;
    if (kept == KP2 && k_eff == KP2 && !os && (reinterpret_cast<uintptr_t>(oi) & 15u) == 0) {
        // a full row without scores: each lane's EPL consecutive slots leave as 16-byte stores
        uint32_t v[EPL];
#pragma unroll
        for (int m = 0; m < EPL; ++m) v[m] = 0xffffffffu - uint32_t(key[m]);
        uint4* o4 = reinterpret_cast<uint4*>(oi + u * EPL);
#pragma unroll
        for (int m = 0; m < EPL / 4; ++m) o4[m] = make_uint4(v[4 * m], v[4 * m + 1], v[4 * m + 2], v[4 * m + 3]);
        if (lidx) {
            uint4* l4 = reinterpret_cast<uint4*>(lidx + u * EPL);
#pragma unroll
            for (int m = 0; m < EPL / 4; ++m) l4[m] = make_uint4(v[4 * m], v[4 * m + 1], v[4 * m + 2], v[4 * m + 3]);
        }
        return;
    }
#pragma unroll
    for (int m = 0; m < EPL; ++m) {
        const int64_t i = u * EPL + m;
        if (i >= k_eff) continue;
        int32_t j;
        if (i < kept) {
            j = int32_t(0xffffffffu - uint32_t(key[m]));
            if (os) os[i] = unord_f32(uint32_t(key[m] >> 32));
        } else {
            j = int32_t((uint32_t(row) + uint32_t(k_eff) + uint32_t(i) + 1u) % uint32_t(T));   // < 2^32: T < 2^31
            if (os) os[i] = -__builtin_inff();
        }
        oi[i] = j;
        if (lidx) lidx[i] = j;
    }
}

// Speculative seed of one row (16 lanes u): a value that at least rk of the row's m sampled
// values (group maxima, at sv[0..m), m <= 16 NV) reach, found by bisection of [min, max] and
// accepted once between rk and ~1.25 rk of them reach it. Any value is safe as a seed: the
// row is checked exactly after its screen. Non-finite samples end the search early (the
// check then fails, or the seed is -inf).
template <int NV>
__device__ float seed_select(const float* sv, int m, int rk, int u)
{
    float v[NV];
    float lo = __builtin_inff(), hi = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        v[i] = u + 16 * i < m ? sv[u + 16 * i] : -__builtin_inff();
        if (u + 16 * i < m) { lo = fminf(lo, v[i]); hi = fmaxf(hi, v[i]); }
    }
    lo = row_min16(lo);
    hi = row_max16(hi);
    const int accept = rk + (rk >> 2) + 2;
    for (int it = 0; it < 20; ++it) {   // every value reaches lo
        const float mid = 0.5f * lo + 0.5f * hi;
        if (!(mid > lo && mid < hi)) break;
        int c = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i) c += int(v[i] >= mid);
        c = row_sum16_i32(c);
        if (c >= rk) {
            lo = mid;
            if (c <= accept) break;
        } else {
            hi = mid;
        }
    }
    return lo;
}

// The retrieval kernel variant of (RC, KP2): two workgroups per CU up to R = 64 and K = 256,
// else one (the wide kernel: its LDS and registers exceed the two-per-CU budget).
template <int RC, int KP2>
constexpr bool kWideTopk = RC > 2 || KP2 > 256;

// No stage after the retrieval (the retrieval kernels). A tail type with kActive = true runs
// its run(...) once every row of the block has been emitted, with each emitted index row
// (k_eff int32) at the start of that row's pool in LDS (the single-pass fused kernel).
struct NoTail {
    static constexpr bool kActive = false;
};

template <typename DT, bool VEC, int RC, int KP2, class Tail = NoTail>
__device__ __forceinline__ void causal_topk_body(const TopkParams& p, const Tail& tail = Tail{})
{
    constexpr int RP = RC * 32;
    // pool entries per row: two workgroups (<= 80 KiB of LDS each) per CU for RC <= 2; the
    // wide variant runs one workgroup per CU (register-bound) and has LDS to spare
    constexpr int POOL = KP2 > 256 ? 768 : 512;
    constexpr int PD = RC >= 8 ? 2 : kPD;   // key steps in flight per wave (operand registers)
    // pool checks every CG key steps: every step for K > 128, whose pruned pools keep so many
    // entries that the room a check interval must reserve decides how often they are pruned
    // (config 5: 18.5 -> 11.3 prunes per block, 2.20 -> 2.04 ms), every 2 steps otherwise
    // (fewer barriers; config 4 is 1-2 % faster that way)
    constexpr int CG = KP2 >= 256 ? 1 : 2;
    constexpr int LIMIT = POOL - CG * kStepMax;  // a pool above this is pruned at the next check
    constexpr int HEADROOM = 64;                 // a prune must leave this much room
    static_assert(LIMIT - HEADROOM > KP2 + 32, "pool too small for K");
    static_assert(sizeof(TopkSmem<RP, POOL>) <= (kWideTopk<RC, KP2> ? 160 : 80) * 1024, "LDS per workgroup");
    __shared__ TopkSmem<RP, POOL> sm;

    const int lane = lane_id();
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    // screening layout: MFMA column n = query row, lane group g = dims 8g..8g+7 / keys 4g..4g+3
    const int n = lane & 15;
    const int g = lane >> 4;
    // row-parallel layout: row rr owned by the 16 lanes u = 0..15 of DPP row (lane >> 4)
    const int rr = 4 * w + (lane >> 4);
    const int u = lane & 15;

    const int64_t T = p.T;
    // Workgroups take (batch, row block) pairs longest causal prefix first, except that the
    // second half of the first residency wave runs in reverse: the two workgroups that start
    // on one CU (c and c + n_cus, two retrieval workgroups fit a CU) then hold positions c and
    // 2 n_cus - 1 - c, whose prefix lengths sum to the same total on every CU (config 4:
    // 0.157 -> 0.150 ms). Any order is a permutation of the same blocks, so results do not
    // depend on it.
    int64_t pos = blockIdx.x;
    const int64_t ncu = p.n_cus;
    if (p.B * (p.rb_end - p.rb_begin) >= 2 * ncu && pos >= ncu && pos < 2 * ncu)
        pos = 3 * ncu - 1 - pos;
    const int64_t b = pos % p.B;
    const int64_t rb = p.rb_end - 1 - pos / p.B;
    const int64_t r0 = rb * kRows;
    const int64_t row = r0 + n;
    const bool row_ok = row < T;
    const int64_t last = min(r0 + kRows - 1, T - 1);
    const int R = int(p.R);
    const int K = int(p.k_eff);
    const DT* qb = static_cast<const DT*>(p.query) + b * p.qsb;
    const DT* kb = static_cast<const DT*>(p.key) + b * p.ksb;

    // query operands (B of the MFMA) in every wave; fp32 rows in LDS from wave 0
    uint4 qlo[RC], qhi[RC];
    const DT* qrow = qb + (row_ok ? row : 0) * p.qst;
#pragma unroll
    for (int c = 0; c < RC; ++c) {
        load8<DT, VEC>(qrow, p.qsr, 32 * c + 8 * g, R, qlo[c], qhi[c]);
        if (!row_ok) { qlo[c] = make_uint4(0, 0, 0, 0); qhi[c] = qlo[c]; }
        if (w == 0) {
            float f[8];
            to_f32x8<DT>(qlo[c], qhi[c], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) sm.q[n][32 * c + 8 * g + e] = f[e];
        }
    }
    if (threadIdx.x < kRows) {
        sm.cnt[threadIdx.x] = 0;
        sm.thr[threadIdx.x] = -__builtin_inff();
        sm.seed[threadIdx.x] = -__builtin_inff();
        sm.fail[threadIdx.x] = 0;
    }
    float mk = 0.0f;
    const int64_t nch = last / kAbsmaxChunk + 1;
    for (int64_t c = lane; c < nch; c += 64) mk = fmaxf(mk, p.chunk_absmax[b * p.n_chunks + c]);
    mk = wave_max(mk);
    __syncthreads();
    if (threadIdx.x < kRows) {
        float l1 = 0.0f;
        for (int d = 0; d < RP; ++d) l1 += fabsf(sm.q[threadIdx.x][d]);
        sm.eps[threadIdx.x] = kEpsPerTerm * float(RP) * (l1 * 1.0001f) * (mk + kTiny) + kTiny;
    }
    __syncthreads();

#ifdef WF_TOPK_TIMING
    // Measurement build only (build.py --timing; bench.py --leg topk-phases reads it): the
    // retrieval runs unchanged, but out_scores carries 8 uint64 per workgroup instead of
    // scores (index = the workgroup's dispatch position), in wall-clock ticks (100 MHz):
    // [0] after set-up, [1] end of the screen, [2] end of the block, [3] row block |
    // in-loop prunes << 16 | their ticks << 32, [4] after the final prune, [5] after exact
    // rescoring and selection, [6] after the seed, [7] pool count before the final prune |
    // passes << 24 | overflowed rows << 28 | count after it << 32.
    uint64_t tm0 = wall_clock64();
    uint64_t tcomp = 0, ncomp = 0;
    uint64_t tm1 = 0, tmA = 0, tmB = 0;
    int c_in = 0, c_pr = 0, npass = 0;
#endif
    // ---- screen
    // Steps 0 .. nfull-1 hold keys below the block's first row r0, so they need neither a
    // causal mask nor clamping; step nfull (the diagonal, keys r0 .. r0+15) is taken once,
    // after the loop, by wave nfull % kTopkWaves. The loop keeps kPD key loads in flight per wave
    // in distinct registers (the unrolled v) and never waits for more than the oldest.
    const int Ti = int(T);
    const int rowi = int(row);
    const int r0i = int(r0);
    const int nsteps = int(last / 16) + 1;
    const int nfull = nsteps - 1;
    const int iters = (nfull + kTopkWaves - 1) / kTopkWaves;   // equal in every wave: barriers match
    // key rows are read at 32-bit byte offsets from the batch base (VEC layouts only)
    const char* kbytes = reinterpret_cast<const char*>(kb);
    const uint32_t krow = uint32_t(p.kst) * uint32_t(sizeof(DT));
    const uint32_t lane_off = uint32_t(n) * krow + uint32_t(8 * g) * uint32_t(sizeof(DT));
    // keys j0 + n of one step; VEC requires R % 32 == 0, so every lane's dims are inside R
    auto load_step = [&](int j0, uint4 (&lo)[RC], uint4 (&hi)[RC]) {
#pragma unroll
        for (int c = 0; c < RC; ++c) {
            if constexpr (VEC) {
                const uint32_t off = uint32_t(j0) * krow + lane_off + uint32_t(32 * c * sizeof(DT));
                lo[c] = *reinterpret_cast<const uint4*>(kbytes + off);
                if constexpr (sizeof(DT) == 4) hi[c] = *reinterpret_cast<const uint4*>(kbytes + off + 16u);
                else hi[c] = make_uint4(0, 0, 0, 0);
            } else {
                const int j = min(j0 + n, Ti - 1);
                load8<DT, false>(kb + int64_t(j) * p.kst, p.ksr, 32 * c + 8 * g, R, lo[c], hi[c]);
            }
        }
    };
    auto score = [&](const uint4 (&alo)[RC], const uint4 (&ahi)[RC]) {
        f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < RC; ++c) acc = mfma_chunk<DT>(alo[c], ahi[c], qlo[c], qhi[c], acc);
        return acc;
    };

    // ---- seed
    // A row that starts at -inf appends every key until its pool first fills, and its
    // threshold then climbs one prune at a time (~1000 appends and 3 prunes per row at config 4).
    // Instead, the block scores ns strided 16-key steps of its full steps first and sets each
    // row's threshold (the seed) where about seed_alpha * K keys of the prefix would reach it:
    // the value that rk of the row's 4 ns group maxima (keys 4g..4g+3 of a step) reach, a
    // group of 4 independent keys reaching it with probability 1 - (1 - pf)^4. The seed is a
    // guess, and the selection stays exact by a check instead: a key the seed rejects has
    // MFMA score < seed, hence exact score < seed + eps, so it cannot be among the row's K
    // best when the row's K-th best exact score s_K0 is >= seed + eps. A row that fails the
    // check keeps its pool and screens its prefix again (pass 1, same workgroup) for the keys
    // the seed rejected that can still matter: MFMA score in [s_K0 - 2 eps, seed) when it
    // kept K (any key of the K best has exact score >= s_K0, MFMA score >= s_K0 - eps), or
    // below the seed when it kept fewer.
    // Pool checks of a seeded block in pass 0 come `stretch` times less often than the worst
    // case (every key of every wave reaching the threshold) requires: about pf of the keys
    // reach a seed, so an interval stretched by 1 / (4 pf) takes a quarter of the room it
    // reserves, on average. A pool that still overflows (clamped appends keep every write in
    // the pool) is detected by its count, and its row is screened again from -inf in pass 1,
    // whose checks reserve the worst case.
    int stretch = 1;
    if (p.seed_alpha > 0.0f && nfull >= 16) {
        const float pf = p.seed_alpha * float(K) / float(16 * nfull);   // block-uniform
        if (pf < 0.5f) {
            stretch = max(1, min(kMaxStretch, int(0.25f / pf)));
            int ns = min(max(int(ceilf(1.25f / pf)), 16), kSeedSteps);   // ~16+ maxima above the seed
            ns = min(ns, nfull);
            ns -= ns % (kTopkWaves * 4);
            const int per_w = ns / kTopkWaves;   // steps per wave, equal in every wave
            float* const samp = reinterpret_cast<float*>(sm.pool[n]);   // group maxima of row n
            for (int i0 = 0; i0 < per_w; i0 += PD) {
                uint4 slo[PD][RC], shi[PD][RC];
#pragma unroll
                for (int v = 0; v < PD; ++v) {   // step j of the sample is full step j * nfull / ns
                    const int j = w + kTopkWaves * min(i0 + v, per_w - 1);
                    load_step(16 * int((int64_t(j) * nfull) / ns), slo[v], shi[v]);
                }
#pragma unroll
                for (int v = 0; v < PD; ++v) {
                    const f32x4_t a = score(slo[v], shi[v]);
                    if (i0 + v < per_w)
                        samp[4 * (w + kTopkWaves * (i0 + v)) + g] = fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3]));
                }
            }
            __syncthreads();   // every group maximum is in LDS
            const int m = 4 * ns;
            const float q1 = (1.0f - pf) * (1.0f - pf);
            const int rk = max(1, int((1.0f - q1 * q1) * float(m) + 0.5f));
            const float* const sv = reinterpret_cast<const float*>(sm.pool[rr]);
            const float sd = m <= 16 * 16 ? seed_select<16>(sv, m, rk, u) : seed_select<kSeedSteps / 4>(sv, m, rk, u);
            if (u == 0) { sm.seed[rr] = sd; sm.thr[rr] = sd; }
            __syncthreads();   // the seeds are set before any wave screens
        }
    }
#ifdef WF_TOPK_TIMING
    const uint64_t tmS = wall_clock64();
#endif

    // one screen and finish; pass 1 (rows whose seed failed) is a second inlined copy, not a
    // loop, which would keep every loop-invariant value of the finish alive through both screens
    auto run_pass = [&](const int pass) __attribute__((always_inline)) {
#ifdef WF_TOPK_TIMING
        npass = pass + 1;
#endif
        // rows past T never take candidates; their threshold is +inf. Pass 1 takes the band
        // [thr, seed) of the rows that failed their check (the others have thr = +inf).
        float th = row_ok ? sm.thr[n] : __builtin_inff();
        const float th_hi = pass == 1 ? sm.seed[n] : __builtin_inff();
        // append the lane's candidates (keys jb .. jb+3 of row n) that reach the threshold; one
        // LDS atomic reserves their slots, the others are written to a dummy slot of the row
        // the row's pool and this lane's dummy slot as LDS pointers, formed once: an append then
        // advances one pointer instead of recomputing a slot address per entry
        Entry* const pool_row = sm.pool[n];
        Entry* const pool_dummy = pool_row + POOL + g;
        auto append = [&](const f32x4_t& acc, const bool (&pp)[4], int jb) {
            const int cntp = int(pp[0]) + int(pp[1]) + int(pp[2]) + int(pp[3]);
            // slot + cntp <= POOL unless a stretched interval overflowed the pool
            Entry* dst = pool_row + min(atomicAdd(&sm.cnt[n], cntp), POOL - cntp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                *(pp[i] ? dst : pool_dummy) = Entry{acc[i], uint32_t(jb + i)};
                dst += int(pp[i]);
            }
        };
        auto consider = [&](const f32x4_t& acc, int jb) {
            bool pp[4] = {acc[0] >= th, acc[1] >= th, acc[2] >= th, acc[3] >= th};
            if (pass == 1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) pp[i] = pp[i] && acc[i] < th_hi;
            }
            if (pp[0] || pp[1] || pp[2] || pp[3]) append(acc, pp, jb);
        };
        // budget: check intervals (CG key steps) every wave may still take before a pool could
        // overflow (a step of all waves appends at most kStepMax per row). Every wave must take
        // the same decisions at a check (the barriers must pair up), so they all decide on one
        // snapshot of the counts: a second barrier keeps every wave from appending again until
        // all of them have read it.
        // (pass 1 starts from the pools pass 0 left: at most max(K, KP2 + 16) entries a row)
        const int bmul = pass == 0 ? stretch : 1;
        int budget = bmul * max(1, (POOL - (pass == 0 ? 0 : __builtin_amdgcn_readfirstlane(
                                         row_max16_i32(lane < kRows ? sm.cnt[lane] : 0)))) / (CG * kStepMax));
        auto check = [&]() {
            __syncthreads();   // every append of the unit has landed
            int cl = lane < kRows ? sm.cnt[lane] : 0;
            if (cl > POOL) sm.fail[lane] = 2;   // overflowed: screen the row again from -inf
            __syncthreads();   // the snapshot is read in every wave before anyone appends again
            if (__ballot(cl > LIMIT)) {
#ifdef WF_TOPK_TIMING
                const uint64_t tc0 = wall_clock64();
#endif
                const int c = rr < kRows ? min(sm.cnt[rr], POOL) : 0;
                const int cw = wave_max_of_rows(c);
                if (c > K) {
                    int c2 = c;
                    const bool ok = prune_sized<(KP2 <= 128), POOL>(sm.pool[rr], sm.hist[rr], c, cw, c2, sm.cnt[rr],
                                                      sm.thr[rr], sm.eps[rr], K, u);
                    if (!ok || c2 > LIMIT - HEADROOM)
                        exact_row<DT, VEC, RP, POOL, false>(sm.pool[rr], sm.hist[rr], c2, POOL, sm.cnt[rr],
                                                     sm.thr[rr], sm.eps[rr], sm.q[rr], kb, p.kst,
                                                     p.ksr, R, K, u);
                }
                __syncthreads();   // every row is pruned
                // a prune's threshold may fall below the seed; in pass 0 the seed still holds
                th = row_ok ? (pass == 0 ? fmaxf(sm.thr[n], sm.seed[n]) : sm.thr[n]) : __builtin_inff();
                cl = lane < kRows ? sm.cnt[lane] : 0;
                __syncthreads();   // ... and read everywhere before anyone appends again
#ifdef WF_TOPK_TIMING
                tcomp += wall_clock64() - tc0;
                ++ncomp;
#endif
            }
            const int cmax = __builtin_amdgcn_readfirstlane(row_max16_i32(cl));
            budget = bmul * max(1, (POOL - cmax) / (CG * kStepMax));
        };
        if (iters > 0) {
            uint4 blo[PD][RC], bhi[PD][RC];
            // issued in buffer order (the scheduler must not reorder them): the loop then waits
            // for the two oldest loads only
#pragma unroll
            for (int v = 0; v < PD; ++v) {
                load_step(16 * min(w + kTopkWaves * v, nfull - 1), blo[v], bhi[v]);
                __builtin_amdgcn_sched_barrier(0);
            }
            for (int it0 = 0; it0 < iters; it0 += PD) {
#pragma unroll
                for (int h = 0; h < PD; h += 2) {   // one 2-step unit
                    // both MFMAs read their buffers before the refills overwrite them
                    const f32x4_t acc0 = score(blo[h], bhi[h]);
                    const f32x4_t acc1 = score(blo[h + 1], bhi[h + 1]);
                    const int st0 = w + kTopkWaves * (it0 + h);
                    const int st1 = st0 + kTopkWaves;
                    load_step(16 * min(st0 + kTopkWaves * PD, nfull - 1), blo[h], bhi[h]);
                    load_step(16 * min(st1 + kTopkWaves * PD, nfull - 1), blo[h + 1], bhi[h + 1]);
                    if (st0 < nfull) consider(acc0, st0 * 16 + 4 * g);
                    if constexpr (CG == 1) {
                        if (--budget == 0) check();
                    }
                    if (st1 < nfull) consider(acc1, st1 * 16 + 4 * g);
                    if (--budget == 0) check();
                }
            }
        }
        if (w == nfull % kTopkWaves) {   // the diagonal step: keys r0 .. r0+15, causal mask
            uint4 alo[RC], ahi[RC];
            if constexpr (VEC) {
                // the block's last rows may pass T: clamp those lanes' key to T-1 (masked below)
                const int j = min(r0i + n, Ti - 1);
#pragma unroll
                for (int c = 0; c < RC; ++c) {
                    const uint32_t off = uint32_t(j) * krow + uint32_t(8 * g + 32 * c) * uint32_t(sizeof(DT));
                    alo[c] = *reinterpret_cast<const uint4*>(kbytes + off);
                    if constexpr (sizeof(DT) == 4) ahi[c] = *reinterpret_cast<const uint4*>(kbytes + off + 16u);
                    else ahi[c] = make_uint4(0, 0, 0, 0);
                }
            } else {
                load_step(r0i, alo, ahi);
            }
            const f32x4_t acc = score(alo, ahi);
            const int jb = r0i + 4 * g;
            const bool pp[4] = {acc[0] >= th && acc[0] < th_hi && jb <= rowi,
                                acc[1] >= th && acc[1] < th_hi && jb + 1 <= rowi,
                                acc[2] >= th && acc[2] < th_hi && jb + 2 <= rowi,
                                acc[3] >= th && acc[3] < th_hi && jb + 3 <= rowi};
            if (pp[0] || pp[1] || pp[2] || pp[3]) append(acc, pp, jb);
        }
        // ---- finish: prune, rescore exactly, select, sort, write, check the seed
        __syncthreads();
#ifdef WF_TOPK_TIMING
        tm1 = wall_clock64();
#endif
        // pass 1 finishes only the rows it screened again; pass 0 leaves overflowed rows to it
        const int craw = rr < kRows && r0 + rr < T ? sm.cnt[rr] : 0;
        const bool ovf = pass == 0 && (craw > POOL || sm.fail[rr] == 2);
        if (ovf && u == 0) sm.fail[rr] = 2;
        const bool row_live = rr < kRows && r0 + rr < T && !ovf && (pass == 0 || sm.fail[rr] != 0);
        int c = row_live ? craw : 0;   // rows past T hold 0 in every lane
#ifdef WF_TOPK_TIMING
        c_in = c;
#endif
        const int cw = wave_max_of_rows(c);
        if (row_live && c > K) {
            int c2 = c;
            prune_sized<(KP2 <= 128), POOL>(sm.pool[rr], sm.hist[rr], c, cw, c2, sm.cnt[rr], sm.thr[rr], sm.eps[rr], K, u);
            c = c2;
        }
#ifdef WF_TOPK_TIMING
        tmA = wall_clock64();
        c_pr = c;
#endif
        const int cw2 = wave_max_of_rows(c);   // counts after the prune, every lane of the wave
        if (row_live) {
            int32_t* const oidx = p.out_idx + b * T * p.k_eff;
#ifdef WF_TOPK_TIMING
            float* const oscr = nullptr;   // out_scores carries the timestamps
#else
            float* const oscr = p.out_scores ? p.out_scores + b * T * p.k_eff : nullptr;
#endif
            // a seeded row's pool must outlive a failed check: its index row reaches LDS after it
            const float sd = sm.seed[rr];
            const bool checked = pass == 0 && sd > -__builtin_inff();
            int32_t* const lidx = Tail::kActive ? reinterpret_cast<int32_t*>(sm.pool[rr]) : nullptr;
            const float lidx_min = checked ? sd + sm.eps[rr] : -__builtin_inff();
            bool done = false;
            uint64_t kth = 0;   // the row's K-th best key (exact score), 0 if it kept fewer
            if constexpr (KP2 == 128 || KP2 == 256) {
                constexpr int NB = KP2 == 128 ? 16 : 64;
                if (cw2 <= KP2 + NB) {   // wave-uniform: selection fused into the sort
                    rescore_row<DT, VEC, RP>(sm.pool[rr], c, sm.q[rr], kb, p.kst, p.ksr, R, u);
#ifdef WF_TOPK_TIMING
                    tmB = wall_clock64();
#endif
                    kth = emit_row_merge<KP2, NB, KP2 == 128 ? 1 : 3, POOL>(sm.pool[rr], c, r0 + rr, T, p.k_eff,
                                                                        oidx, oscr, lidx, lidx_min, u);
                    done = true;
                }
            }
            if (!done) {
                const int kept = exact_row<DT, VEC, RP, POOL, (KP2 <= 128)>(sm.pool[rr], sm.hist[rr], c, cw2,
                                                                           sm.cnt[rr], sm.thr[rr], sm.eps[rr],
                                                                           sm.q[rr], kb, p.kst, p.ksr, R, K, u);
#ifdef WF_TOPK_TIMING
                tmB = wall_clock64();
#endif
                kth = emit_row<KP2, POOL>(sm.pool[rr], kept, r0 + rr, T, p.k_eff, oidx, oscr, lidx, lidx_min, u);
            }
            if (checked) {
                const float eps = sm.eps[rr];
                const bool good = kth != 0ull && key_entry(kth).s >= sd + eps;
                if (!good && u == 0) {
                    sm.fail[rr] = 1;
                    sm.thr[rr] = kth != 0ull ? key_entry(kth).s - 2.0f * eps : -__builtin_inff();
                }
            }
        }
    };
    run_pass(0);
    __syncthreads();   // every row's check is done
    const int fl = lane < kRows ? sm.fail[lane] : 0;
    if (__ballot(fl != 0)) {   // the same flags in every wave
        __syncthreads();   // ... read everywhere before the reset
        // rows that passed are final: they take nothing more, and with count 0 no check prunes
        // them (the single-pass kernel keeps their index rows at the start of their pools);
        // overflowed rows start again from an empty pool and take every key
        if (threadIdx.x < kRows) {
            const int f = sm.fail[threadIdx.x];
            if (f != 1) sm.cnt[threadIdx.x] = 0;
            if (f == 0) sm.thr[threadIdx.x] = __builtin_inff();
            if (f == 2) { sm.thr[threadIdx.x] = -__builtin_inff(); sm.seed[threadIdx.x] = __builtin_inff(); }
        }
        __syncthreads();
        run_pass(1);
    }
    if constexpr (Tail::kActive) {
        __syncthreads();   // every row's index list is in LDS
        tail.run(reinterpret_cast<const char*>(sm.pool), sizeof(sm.pool[0]), b, r0, T, K, w, lane);
    }
#ifdef WF_TOPK_TIMING
    __syncthreads();
    if (threadIdx.x == 0 && p.out_scores) {
        uint64_t* tm = reinterpret_cast<uint64_t*>(p.out_scores) + 8 * blockIdx.x;
        tm[0] = tm0; tm[1] = tm1; tm[2] = wall_clock64(); tm[3] = uint64_t(rb) | (ncomp << 16) | (tcomp << 32);
        tm[4] = tmA; tm[5] = tmB; tm[6] = tmS;
        int novf = 0;   // rows whose pool overflowed in pass 0
        for (int r = 0; r < kRows; ++r) novf += sm.fail[r] == 2;
        tm[7] = uint64_t(c_in) | (uint64_t(npass) << 24) | (uint64_t(min(novf, 15)) << 28) | (uint64_t(c_pr) << 32);
    }
#endif
}

}  // namespace
}  // namespace wf
