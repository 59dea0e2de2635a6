// wf_topk.hip -- causal top-K address retrieval for gfx950 (MI355X).
//
// Replaces routing_attention/kernels/causal_topk.py:132-171 (_causal_topk_row_blocked) and
// :37-57 (_finalize_causal_topk). Where the reference writes a (B, block_m, i1) fp32 score
// block to HBM per row block and runs torch.topk over it, this kernel never materialises
// scores outside LDS:
//
//  1. screen   One wave owns 16 query rows. It streams the causal key prefix 16 keys at a
//              time; one v_mfma_f32_16x16x32_{bf16,f16} (or eight 16x16x4 f32) per 32
//              address dims scores the 16x16 tile. A key is kept as a candidate of a row
//              only if its MFMA score reaches that row's threshold: the exact K-th best
//              score so far minus eps, where eps bounds |MFMA score - exact score|.
//  2. pool     Candidates are appended (LDS atomics) to a per-row pool in LDS that holds
//              the current exact top-K plus pending candidate indices.
//  3. compact  When a pool fills up, the wave rescores the pending candidates exactly
//              (fp32 fma chain over d ascending, the oracle's definition of the score),
//              radix-selects the K best under (score desc, index asc) and raises the
//              row's threshold.
//  4. emit     After the prefix is exhausted, each row's top-K is bitonic-sorted into
//              canonical order and written with the reference's pad indices.
//
// The selection is exact: a key that belongs to the final top-K has exact score > the
// current K-th score (ties lose to the lower, earlier index), so its MFMA score is at
// least threshold - eps and it reaches the pool; the final choice uses exact scores only.
#include "wf_internal.h"

namespace wf {
namespace {

constexpr int kRows = 16;                              // query rows per wave (MFMA N)
constexpr int kPrefetch = 8;                           // key steps loaded ahead
constexpr float kEpsRel = 1.0f / 4096.0f;              // 2^-12: > 20x the MFMA/FMA error bound
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
template <typename DT, bool VEC>
__device__ __forceinline__ float exact_score(const float* q, const DT* krow, int64_t sr, int R)
{
    float acc = 0.0f;
    if constexpr (VEC) {
        for (int d0 = 0; d0 < R; d0 += 8) {
            uint4 lo, hi;
            load8<DT, true>(krow, 1, d0, R, lo, hi);
            float kf[8];
            to_f32x8<DT>(lo, hi, kf);
            const float4 qa = *reinterpret_cast<const float4*>(q + d0);
            const float4 qb = *reinterpret_cast<const float4*>(q + d0 + 4);
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

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int m)
{
    const uint32_t lo = __shfl_xor(uint32_t(x), m, 64);
    const uint32_t hi = __shfl_xor(uint32_t(x >> 32), m, 64);
    return (uint64_t(hi) << 32) | lo;
}

// ------------------------------------------------------------------ LDS layout
template <int RP, int POOL>
struct TopkSmem {
    float q[kRows][RP];            // fp32 query rows (exact rescoring)
    float score[kRows][POOL];      // exact scores of kept entries / rescored pending ones
    uint32_t idx[kRows][POOL];     // key index of every pool entry
    uint32_t hist[256];            // radix-select histogram
    int cnt[kRows];                // pool fill (kept + pending)
    int kept[kRows];               // entries with exact scores that form the current top-K
    float thr[kRows];              // screening threshold (K-th exact score - eps, or -inf)
    float eps[kRows];              // |MFMA score - exact score| bound of the row
};

// Rescore row r's pending entries, keep its K best, refresh its threshold.
template <typename DT, bool VEC, int RP, int POOL>
__device__ void compact_row(TopkSmem<RP, POOL>& sm, int r, int K, const DT* kb, int64_t kst,
                            int64_t ksr, int R)
{
    constexpr int E = POOL / 64;
    const int lane = lane_id();
    const int c = sm.cnt[r];
    const int nk = sm.kept[r];

    for (int e = nk + lane; e < c; e += 64) {
        const uint32_t j = sm.idx[r][e];
        sm.score[r][e] = exact_score<DT, VEC>(sm.q[r], kb + int64_t(j) * kst, ksr, R);
    }
    __syncthreads();

    uint64_t key[E];
    float sv[E];
    uint32_t iv[E];
    bool val[E];
#pragma unroll
    for (int m = 0; m < E; ++m) {
        const int e = lane + 64 * m;
        val[m] = e < c;
        sv[m] = val[m] ? sm.score[r][e] : 0.0f;
        iv[m] = val[m] ? sm.idx[r][e] : 0u;
        key[m] = val[m] ? make_key(sv[m], iv[m]) : 0ull;
    }

    // MSD radix select of the K-th largest key (8-bit digits, early exit once the
    // boundary bucket is taken whole). Keys are unique (distinct indices).
    uint64_t prefix = 0, pmask = 0;
    if (c > K) {
        int need = K;
        for (int shift = 56; shift >= 0; shift -= 8) {
            reinterpret_cast<uint4*>(sm.hist)[lane] = make_uint4(0, 0, 0, 0);
            __syncthreads();
#pragma unroll
            for (int m = 0; m < E; ++m)
                if (val[m] && (key[m] & pmask) == prefix)
                    atomicAdd(&sm.hist[(key[m] >> shift) & 255u], 1u);
            __syncthreads();
            const uint4 h = reinterpret_cast<const uint4*>(sm.hist)[lane];
            const int s3 = int(h.w), s2 = int(h.z) + s3, s1 = int(h.y) + s2, s0 = int(h.x) + s1;
            const int above = wave_suffix_excl(s0);
            const bool has = above < need && s0 + above >= need;
            int d, gt, eq;
            if (s3 + above >= need) { d = 4 * lane + 3; gt = above; eq = int(h.w); }
            else if (s2 + above >= need) { d = 4 * lane + 2; gt = above + s3; eq = int(h.z); }
            else if (s1 + above >= need) { d = 4 * lane + 1; gt = above + s2; eq = int(h.y); }
            else { d = 4 * lane; gt = above + s1; eq = int(h.x); }
            const uint64_t hm = __ballot(has);
            const int src = __ffsll((unsigned long long)hm) - 1;
            d = __shfl(d, src, 64);
            gt = __shfl(gt, src, 64);
            eq = __shfl(eq, src, 64);
            need -= gt;
            prefix |= uint64_t(d) << shift;
            pmask |= uint64_t(0xff) << shift;
            __syncthreads();
            if (eq == need) break;
        }
    }

    // stream-compact the selected entries to the front of the pool
    int base = 0;
    uint32_t minord = 0xffffffffu;
    const uint64_t lt = (1ull << lane) - 1ull;
#pragma unroll
    for (int m = 0; m < E; ++m) {
        const bool sel = val[m] && (key[m] & pmask) >= prefix;
        const uint64_t bm = __ballot(sel);
        if (sel) {
            const int pos = base + __popcll(bm & lt);
            sm.score[r][pos] = sv[m];
            sm.idx[r][pos] = iv[m];
            const uint32_t o = uint32_t(key[m] >> 32);
            minord = o < minord ? o : minord;
        }
        base += __popcll(bm);
    }
    minord = wave_min_u32(minord);
    if (lane == 0) {
        sm.cnt[r] = base;
        sm.kept[r] = base;
        sm.thr[r] = (base >= K) ? unord_f32(minord) - sm.eps[r] : -__builtin_inff();
    }
    __syncthreads();
}

// Sort row r's kept entries into canonical order and write them (plus pads). `row` is the
// query position t within its batch; out_idx / out_scores point at that batch's (T, k_eff).
template <int KP2, int RP, int POOL>
__device__ void emit_row(TopkSmem<RP, POOL>& sm, int r, int64_t row, int64_t T, int64_t k_eff,
                         int32_t* out_idx, float* out_scores)
{
    constexpr int E2 = KP2 / 64;
    const int lane = lane_id();
    const int kept = sm.kept[r];
    uint64_t key[E2];
#pragma unroll
    for (int m = 0; m < E2; ++m) {
        const int i = 64 * m + lane;
        key[m] = i < kept ? make_key(sm.score[r][i], sm.idx[r][i]) : 0ull;
    }
    // bitonic sort, descending
#pragma unroll
    for (int kk = 2; kk <= KP2; kk <<= 1) {
#pragma unroll
        for (int jj = kk >> 1; jj > 0; jj >>= 1) {
            if (jj >= 64) {
                const int mj = jj >> 6;
#pragma unroll
                for (int m = 0; m < E2; ++m) {
                    if (m & mj) continue;
                    const int m2 = m | mj;
                    const int i = 64 * m + lane;
                    const bool desc = (i & kk) == 0;
                    const uint64_t a = key[m], b = key[m2];
                    const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
                    key[m] = desc ? hi : lo;
                    key[m2] = desc ? lo : hi;
                }
            } else {
#pragma unroll
                for (int m = 0; m < E2; ++m) {
                    const int i = 64 * m + lane;
                    const uint64_t other = shfl_xor_u64(key[m], jj);
                    const bool low = (lane & jj) == 0;
                    const bool desc = (i & kk) == 0;
                    const uint64_t hi = key[m] > other ? key[m] : other;
                    const uint64_t lo = key[m] > other ? other : key[m];
                    key[m] = (low == desc) ? hi : lo;
                }
            }
        }
    }
    int32_t* oi = out_idx + row * k_eff;
    float* os = out_scores ? out_scores + row * k_eff : nullptr;
#pragma unroll
    for (int m = 0; m < E2; ++m) {
        const int64_t i = 64 * m + lane;
        if (i >= k_eff) continue;
        if (i < kept) {
            oi[i] = int32_t(0xffffffffu - uint32_t(key[m]));
            if (os) os[i] = unord_f32(uint32_t(key[m] >> 32));
        } else {
            oi[i] = int32_t((row + k_eff + i + 1) % T);
            if (os) os[i] = -__builtin_inff();
        }
    }
}

// ------------------------------------------------------------------ kernels
template <typename DT>
__global__ __launch_bounds__(256) void key_absmax_kernel(TopkParams p)
{
    const int64_t b = blockIdx.y;
    const int64_t j0 = int64_t(blockIdx.x) * kAbsmaxChunk;
    const int64_t j1 = min(p.T, j0 + kAbsmaxChunk);
    const int64_t n = (j1 - j0) * p.R;
    const DT* kb = static_cast<const DT*>(p.key) + b * p.ksb;
    float m = 0.0f;
    for (int64_t e = threadIdx.x; e < n; e += blockDim.x) {
        const int64_t j = j0 + e / p.R, d = e % p.R;
        m = fmaxf(m, fabsf(to_f32(kb[j * p.kst + d * p.ksr])));
    }
    m = wave_max(m);
    __shared__ float part[4];
    if (lane_id() == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0)
        p.chunk_absmax[b * p.n_chunks + blockIdx.x] =
            fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
}

template <typename DT, bool VEC, int RC, int KP2>
__global__ __launch_bounds__(64) void causal_topk_kernel(TopkParams p)
{
    constexpr int RP = RC * 32;
    constexpr int POOL = KP2 + 128;
    __shared__ TopkSmem<RP, POOL> sm;

    const int lane = threadIdx.x;
    const int n = lane & 15;       // query row of this lane (MFMA column)
    const int g = lane >> 4;       // lane group: dims 8g..8g+7 of each chunk, keys 4g..4g+3
    const int64_t T = p.T;
    const int64_t b = blockIdx.x % p.B;
    const int64_t rb = p.n_row_blocks - 1 - blockIdx.x / p.B;   // longest prefixes first
    const int64_t r0 = rb * kRows;
    const int64_t row = r0 + n;
    const bool row_ok = row < T;
    const int64_t last = min(r0 + kRows - 1, T - 1);
    const int R = int(p.R);
    const int K = int(p.k_eff);
    const DT* qb = static_cast<const DT*>(p.query) + b * p.qsb;
    const DT* kb = static_cast<const DT*>(p.key) + b * p.ksb;

    // query operands (B of the MFMA) and fp32 query rows in LDS
    uint4 qlo[RC], qhi[RC];
    const DT* qrow = qb + (row_ok ? row : 0) * p.qst;
#pragma unroll
    for (int c = 0; c < RC; ++c) {
        load8<DT, VEC>(qrow, p.qsr, 32 * c + 8 * g, R, qlo[c], qhi[c]);
        if (!row_ok) { qlo[c] = make_uint4(0, 0, 0, 0); qhi[c] = qlo[c]; }
        float f[8];
        to_f32x8<DT>(qlo[c], qhi[c], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) sm.q[n][32 * c + 8 * g + e] = f[e];
    }
    if (lane < kRows) {
        sm.cnt[lane] = 0;
        sm.kept[lane] = 0;
        sm.thr[lane] = -__builtin_inff();
    }
    // bound on |key element| over the scanned prefix [0, last]
    float mk = 0.0f;
    const int64_t nch = last / kAbsmaxChunk + 1;
    for (int64_t c = lane; c < nch; c += 64) mk = fmaxf(mk, p.chunk_absmax[b * p.n_chunks + c]);
    mk = wave_max(mk);
    __syncthreads();
    if (lane < kRows) {
        float l1 = 0.0f;
        for (int d = 0; d < RP; ++d) l1 += fabsf(sm.q[lane][d]);
        sm.eps[lane] = kEpsRel * (l1 * 1.0001f) * (mk + kTiny) + kTiny;
    }
    __syncthreads();

    float th = -__builtin_inff();
    const int64_t nsteps = last / 16 + 1;
    uint4 plo[kPrefetch][RC], phi[kPrefetch][RC];
#pragma unroll
    for (int u = 0; u < kPrefetch; ++u) {
        const int64_t j = min(int64_t(u) * 16 + n, T - 1);
#pragma unroll
        for (int c = 0; c < RC; ++c) load8<DT, VEC>(kb + j * p.kst, p.ksr, 32 * c + 8 * g, R, plo[u][c], phi[u][c]);
    }

    for (int64_t s0 = 0; s0 < nsteps; s0 += kPrefetch) {
#pragma unroll
        for (int u = 0; u < kPrefetch; ++u) {
            const int64_t st = s0 + u;
            if (st >= nsteps) break;
            uint4 alo[RC], ahi[RC];
#pragma unroll
            for (int c = 0; c < RC; ++c) { alo[c] = plo[u][c]; ahi[c] = phi[u][c]; }
            {   // refill this slot with step st + kPrefetch
                const int64_t j = min((st + kPrefetch) * 16 + n, T - 1);
                if (st + kPrefetch < nsteps) {
#pragma unroll
                    for (int c = 0; c < RC; ++c)
                        load8<DT, VEC>(kb + j * p.kst, p.ksr, 32 * c + 8 * g, R, plo[u][c], phi[u][c]);
                }
            }
            f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < RC; ++c) acc = mfma_chunk<DT>(alo[c], ahi[c], qlo[c], qhi[c], acc);

            const int64_t j0 = st * 16;
            const bool diag = (j0 == r0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t j = j0 + 4 * g + i;
                const bool pass = row_ok && acc[i] >= th && (!diag || j <= row);
                if (pass) {
                    const int pos = atomicAdd(&sm.cnt[n], 1);
                    sm.idx[n][pos] = uint32_t(j);
                }
            }
            const int c = sm.cnt[n];
            uint64_t full = __ballot(lane < kRows && c > POOL - 16);
            if (full) {
                while (full) {
                    const int r = __ffsll((unsigned long long)full) - 1;
                    full &= full - 1;
                    compact_row<DT, VEC, RP, POOL>(sm, r, K, kb, p.kst, p.ksr, R);
                }
                th = sm.thr[n];
            }
        }
    }

    // finish every row: rescore what is pending, select, sort, write
    for (int r = 0; r < kRows; ++r) {
        if (r0 + r >= T) break;
        compact_row<DT, VEC, RP, POOL>(sm, r, K, kb, p.kst, p.ksr, R);
        emit_row<KP2, RP, POOL>(sm, r, r0 + r, T, p.k_eff, p.out_idx + b * T * p.k_eff,
                                p.out_scores ? p.out_scores + b * T * p.k_eff : nullptr);
    }
}

template <typename DT, bool VEC, int RC>
hipError_t launch_topk_k(const TopkParams& p, hipStream_t s)
{
    const dim3 grid(unsigned(p.B * p.n_row_blocks)), block(64);
    if (p.k_eff <= 64) causal_topk_kernel<DT, VEC, RC, 64><<<grid, block, 0, s>>>(p);
    else if (p.k_eff <= 128) causal_topk_kernel<DT, VEC, RC, 128><<<grid, block, 0, s>>>(p);
    else causal_topk_kernel<DT, VEC, RC, 256><<<grid, block, 0, s>>>(p);
    return hipGetLastError();
}

template <typename DT, bool VEC>
hipError_t launch_topk_r(const TopkParams& p, hipStream_t s)
{
    if (p.R <= 32) return launch_topk_k<DT, VEC, 1>(p, s);
    if (p.R <= 64) return launch_topk_k<DT, VEC, 2>(p, s);
    return launch_topk_k<DT, VEC, 4>(p, s);
}

template <typename DT>
hipError_t launch_topk_t(bool vec, const TopkParams& p, hipStream_t s)
{
    return vec ? launch_topk_r<DT, true>(p, s) : launch_topk_r<DT, false>(p, s);
}

}  // namespace

hipError_t launch_key_absmax(int dtype, const TopkParams& p, hipStream_t s)
{
    const dim3 grid(unsigned(p.n_chunks), unsigned(p.B)), block(256);
    if (dtype == 2) key_absmax_kernel<bf16_t><<<grid, block, 0, s>>>(p);
    else if (dtype == 1) key_absmax_kernel<_Float16><<<grid, block, 0, s>>>(p);
    else key_absmax_kernel<float><<<grid, block, 0, s>>>(p);
    return hipGetLastError();
}

hipError_t launch_causal_topk(int dtype, bool vec, const TopkParams& p, hipStream_t s)
{
    if (dtype == 2) return launch_topk_t<bf16_t>(vec, p, s);
    if (dtype == 1) return launch_topk_t<_Float16>(vec, p, s);
    return launch_topk_t<float>(vec, p, s);
}

}  // namespace wf
