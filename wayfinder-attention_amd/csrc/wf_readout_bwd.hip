// wf_readout_bwd.hip -- backward of the sparse readout with fixed indices (gfx950).
//
// Counterpart of the autograd the reference gets from its differentiable readout
// (routing_attention/models/attention.py:35-55 with _gather_kv_heads :58-69: gather,
// softmax, weighted sum), whose backward scatters (B, H, T, K, D) gradient copies back into
// k and v with index_put accumulation. With p_s the softmax weight of slot s of row t,
// dp_s = dout_t . v_{j_s} and delta_t = sum_s p_s dp_s:
//
//   dq_t = scale * (sum_s p_s dp_s k_{j_s} - delta_t * sum_s p_s k_{j_s})
//   dk_j = scale * sum_{(t,s): j_s = j} p_s (dp_s - delta_t) q_t
//   dv_j = sum_{(t,s): j_s = j} p_s dout_t
//
// With dropout on the weights (kept with mask m_s, scaled by c = 1/(1-p); the forward output
// is sum_s p_s m_s c v_s) the same formulas hold with dp_s = m_s c (dout_t . v_{j_s}) and
// dv_j = sum p_s m_s c dout_t; delta_t = sum_s p_s dp_s is still dout_t . out_t.
//
// computed without floating-point atomics, so the gradients are deterministic:
//  1. index transpose: a stable LSD radix sort (8-bit digits; per pass a workgroup
//     histogram, a per-digit scan over workgroups and a stable scatter ranked with wave
//     ballots) of (b*T + j) keys with the slot t*K + s as value groups the rows that selected
//     each key, t ascending; a binary search per key over the sorted keys gives each list's
//     offset. Masked pad slots sort past the last list. No memsets, no global atomics: every
//     count is written whole, so the backward can be captured into a HIP graph.
//  2. row pass (the forward's mapping: one wave walks 4 query rows, D/8 lanes per
//     neighbour): recomputes p from the forward's base-2 log-sum-exp and writes dq, and
//     (lse2, delta) per row for the key pass -- delta exact, from the row's own p and dp
//     rather than the rounded output;
//  3. key pass (same mapping over key rows): each key row walks its list, gathering q_t and
//     dout_t -- the forward's access pattern with the roles of query and key swapped -- and
//     recomputes p and dp for every entry. Nothing of size (B, H, T, K) is stored.
// All accumulation is fp32; each gradient element is rounded once to the input dtype.
#include "wf_readout_dev.h"

namespace wf {
namespace {

// ---------------------------------------------------------------- index transpose
constexpr int kSortThreads = 256;                      // 4 waves
constexpr int kSortItems = 16;                         // items per thread and pass
constexpr uint32_t kSortTile = kSortThreads * kSortItems;

// Input of one radix pass: the (b, t, s) slots themselves on the first pass (key b*T + j with
// j wrapped and clamped as in the forward, value t*K + s; masked pad slots -- s > t on rows
// t < K-1 with WF_FLAG_MASK_PADS -- get the key B*T, past every list), the previous pass's
// arrays after it. B*T*K < 2^32 (checked by the entry point), so slot arithmetic is 32-bit.
struct SortSrc {
    const int32_t* idx;
    int64_t is0, is1, is2;
    uint32_t B, T, K;
    FastDiv divK, divTK;    // by K and by T*K
    bool mask_pads;
    const uint32_t* keys;   // null: first pass
    const uint32_t* vals;
};

__device__ __forceinline__ uint32_t sort_key(const SortSrc& s, uint32_t e, uint32_t& val)
{
    if (s.keys) {
        val = s.vals[e];
        return s.keys[e];
    }
    const uint32_t b = fdiv(e, s.divTK);
    const uint32_t r = e - b * (s.T * s.K);
    const uint32_t t = fdiv(r, s.divK);
    const uint32_t sl = r - t * s.K;
    int j = s.idx[int64_t(b) * s.is0 + int64_t(t) * s.is1 + int64_t(sl) * s.is2];
    j += (j >> 31) & int(s.T);
    j = min(max(j, 0), int(s.T) - 1);
    val = r;   // t * K + sl
    const bool masked = s.mask_pads && t + 1 < s.K && sl > t;
    return masked ? s.B * s.T : b * s.T + uint32_t(j);
}

// Digit histogram of one tile: H[d * nblk + tile] = items of the tile with digit d.
__global__ __launch_bounds__(kSortThreads) void radix_hist(SortSrc s, uint32_t n, int shift,
                                                           uint32_t nblk, uint32_t* H)
{
    __shared__ uint32_t h[256];
    const uint32_t tid = threadIdx.x;
    h[tid] = 0;
    uint32_t key[kSortItems];   // every load issued before the first use
#pragma unroll
    for (int i = 0; i < kSortItems; ++i) {
        const uint32_t e = blockIdx.x * kSortTile + uint32_t(i) * kSortThreads + tid;
        uint32_t v;
        key[i] = e < n ? sort_key(s, e, v) : 0u;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSortItems; ++i) {
        const uint32_t e = blockIdx.x * kSortTile + uint32_t(i) * kSortThreads + tid;
        if (e < n) atomicAdd(&h[(key[i] >> shift) & 255u], 1u);
    }
    __syncthreads();
    H[tid * nblk + blockIdx.x] = h[tid];
}

// Exclusive scan of 256 values across the workgroup (one per thread); returns the exclusive
// prefix of this thread's value, and the total in *sum.
__device__ __forceinline__ uint32_t block_excl_scan256(uint32_t x, uint32_t* buf, uint32_t* sum)
{
    const uint32_t tid = threadIdx.x;
    buf[tid] = x;
    for (uint32_t o = 1; o < 256; o <<= 1) {
        __syncthreads();
        const uint32_t y = tid >= o ? buf[tid - o] : 0u;
        __syncthreads();
        buf[tid] += y;
    }
    __syncthreads();
    *sum = buf[255];
    const uint32_t incl = buf[tid];
    __syncthreads();
    return incl - x;
}

// One workgroup per digit d: H[d][*] becomes its exclusive scan over tiles, total[d] the
// digit's count.
__global__ __launch_bounds__(kSortThreads) void radix_scan(uint32_t* H, uint32_t nblk, uint32_t* total)
{
    __shared__ uint32_t buf[256];
    uint32_t* row = H + size_t(blockIdx.x) * nblk;
    const uint32_t per = (nblk + kSortThreads - 1) / kSortThreads;
    const uint32_t beg = min(threadIdx.x * per, nblk), end = min(beg + per, nblk);
    uint32_t sum = 0;
    for (uint32_t i = beg; i < end; ++i) sum += row[i];
    uint32_t all;
    uint32_t run = block_excl_scan256(sum, buf, &all);
    for (uint32_t i = beg; i < end; ++i) {
        const uint32_t v = row[i];
        row[i] = run;
        run += v;
    }
    if (threadIdx.x == 0) total[blockIdx.x] = all;
}

// Stable scatter of one tile: items are taken in order (round r, thread t -> item
// tile*kSortTile + r*256 + t); an item's place among the tile's items of its digit is the
// count in earlier rounds + in earlier waves of this round + in earlier lanes of its wave
// (lanes with the same digit found by 8 ballots). The tile is first ordered in LDS by
// (digit, place), then written out by consecutive threads, so each digit's run of the tile
// goes to global memory as one contiguous, coalesced stretch.
__global__ __launch_bounds__(kSortThreads) void radix_scatter(SortSrc s, uint32_t n, int shift,
                                                              uint32_t nblk, const uint32_t* H,
                                                              const uint32_t* total,
                                                              uint32_t* okeys, uint32_t* ovals)
{
    __shared__ uint32_t buf[256], base[256], lstart[256], run[256], wcnt[4][256];
    __shared__ uint32_t sk[kSortTile], sv[kSortTile];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, w = tid >> 6;
    const uint32_t tile0 = blockIdx.x * kSortTile;
    const uint32_t ntile = min(kSortTile, n - tile0);
    uint32_t keys[kSortItems], vals[kSortItems];   // every load issued before the rounds
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const uint32_t e = tile0 + uint32_t(r) * kSortThreads + tid;
        keys[r] = 0;
        vals[r] = 0;
        if (e < n) keys[r] = sort_key(s, e, vals[r]);
    }
    // digit d of this tile: global start base[d], start inside the tile lstart[d]
    const uint32_t hd = H[tid * nblk + blockIdx.x];
    const uint32_t mine = (blockIdx.x + 1 < nblk ? H[tid * nblk + blockIdx.x + 1] : total[tid]) - hd;
    uint32_t all;
    const uint32_t pre = block_excl_scan256(total[tid], buf, &all);
    base[tid] = pre + hd;
    lstart[tid] = block_excl_scan256(mine, buf, &all);
    run[tid] = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) wcnt[k][tid] = 0;
    __syncthreads();
    const uint64_t lt = (uint64_t(1) << lane) - 1;
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const bool valid = uint32_t(r) * kSortThreads + tid < ntile;
        const uint32_t d = (keys[r] >> shift) & 255u;
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool on = (d >> bit) & 1u;
            const uint64_t m = __ballot(on);
            peers &= on ? m : ~m;
        }
        const uint32_t rank = __popcll(peers & lt);
        if (valid && rank == 0) wcnt[w][d] = __popcll(peers);
        __syncthreads();
        if (valid) {
            uint32_t off = lstart[d] + run[d] + rank;
            for (uint32_t k = 0; k < w; ++k) off += wcnt[k][d];
            sk[off] = keys[r];
            sv[off] = vals[r];
        }
        __syncthreads();
        run[tid] += wcnt[0][tid] + wcnt[1][tid] + wcnt[2][tid] + wcnt[3][tid];
#pragma unroll
        for (int k = 0; k < 4; ++k) wcnt[k][tid] = 0;
        __syncthreads();
    }
    for (uint32_t i = tid; i < ntile; i += kSortThreads) {
        const uint32_t key = sk[i];
        const uint32_t d = (key >> shift) & 255u;
        const uint32_t g = base[d] + (i - lstart[d]);
        okeys[g] = key;
        ovals[g] = sv[i];
    }
}

// off[k] = first position of the sorted keys holding a key >= k, for k = 0 .. B*T: the start
// of key k's list (off[B*T] = the number of unmasked slots). One binary search per key.
__global__ void bwd_list_offsets(const uint32_t* sorted, uint32_t n, uint32_t nkeys, uint32_t* off)
{
    const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= nkeys) return;
    uint32_t lo = 0, hi = n;   // invariant: sorted[lo-1] < k <= sorted[hi]
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (sorted[mid] < k) lo = mid + 1;
        else hi = mid;
    }
    off[k] = lo;
}

struct Pair { int64_t b, h, r0; int n; };

// The forward's XCD-aware mapping: returns the (b, h) pair and the first of this wave's
// (up to kRowsPerWave) consecutive rows; n = 0 when the wave has no rows.
__device__ __forceinline__ Pair map_rows(const ReadoutBwdParams& p, int wave)
{
    Pair r{0, 0, 0, 0};
    const int64_t xcd = blockIdx.x & 7;
    const int64_t it = blockIdx.x >> 3;
    const int64_t vp = (it / p.wg_per_vpair) * 8 + xcd;
    if (vp >= p.vpairs) return r;
    const int64_t chunk = it % p.wg_per_vpair;
    const int64_t pair = vp / p.seg_per_pair;
    const int64_t seg = vp % p.seg_per_pair;
    r.b = pair / p.H;
    r.h = pair % p.H;
    const int64_t t0 = p.row_begin + seg * p.rows_per_seg;
    const int64_t t1 = min(p.row_end, t0 + p.rows_per_seg);
    r.r0 = t0 + (chunk * kWaves + wave) * kRowsPerWave;
    if (r.r0 < t1) r.n = int(min(int64_t(kRowsPerWave), t1 - r.r0));
    return r;
}

__device__ __forceinline__ int wrap_index(int j, int T)
{
    j += (j >> 31) & T;
    return min(max(j, 0), T - 1);
}

// Keep bits of slots slot_u (u < 2) of every lane group: lane sub < 2 of each group hashes its
// group's slot_sub, and one ballot hands each group its two bits (groups are LPN >= 4 lanes).
template <int LPN>
__device__ __forceinline__ uint32_t drop_bits2(const DropoutParams& d, uint32_t row_key0,
                                               uint32_t row_key1, uint32_t slot0, uint32_t slot1,
                                               int sub, int grp)
{
    const bool mine = sub < 2 && drop_keep(d, sub == 0 ? row_key0 : row_key1, sub == 0 ? slot0 : slot1);
    return uint32_t(__ballot(mine) >> (grp * LPN)) & 3u;
}

// Row pass: dq and delta for query rows t of one (b, h) pair.
template <typename DT, int D, bool DROP>
__global__ __launch_bounds__(64 * kWaves) void readout_bwd_rows(ReadoutBwdParams p)
{
    constexpr int LPN = D / 8;
    constexpr int NPS = 64 / LPN;
    constexpr uint32_t ES = sizeof(DT);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sub = lane % LPN;
    const int grp = lane / LPN;
    const Pair w = map_rows(p, wave);
    if (w.n == 0) return;
    const int64_t b = w.b, h = w.h, tw = w.r0;
    const int K = int(p.K);
    const int T = int(p.T);
    const bool mask_flag = (p.flags & 1u) != 0;
    const float sl2 = p.scale * kLog2e;

    const char* kb = reinterpret_cast<const char*>(static_cast<const DT*>(p.k) + b * p.ks[0] + h * p.ks[1]);
    const char* vb = reinterpret_cast<const char*>(static_cast<const DT*>(p.v) + b * p.vs[0] + h * p.vs[1]);
    const char* qb = reinterpret_cast<const char*>(static_cast<const DT*>(p.q) + b * p.qs[0] + h * p.qs[1] + tw * p.qs[2]);
    const char* gb = reinterpret_cast<const char*>(static_cast<const DT*>(p.dout) + b * p.gs[0] + h * p.gs[1] + tw * p.gs[2]);
    char* db = reinterpret_cast<char*>(static_cast<DT*>(p.dq) + b * p.dqs[0] + h * p.dqs[1] + tw * p.dqs[2]);
    const uint32_t krow = uint32_t(p.ks[2]) * ES, vrow = uint32_t(p.vs[2]) * ES;
    const uint32_t qrow = uint32_t(p.qs[2]) * ES, grow = uint32_t(p.gs[2]) * ES;
    const uint32_t drow = uint32_t(p.dqs[2]) * ES;
    // lanes past the head dim (p.D < D) read the last slice, zero their q / dout slices (no
    // contribution to any dot product) and store nothing
    const int dv = int(p.D) / 8;
    const bool lane_on = sub < dv;
    const uint32_t loff = uint32_t(min(sub, dv - 1)) * 8u * ES;
    const int32_t* ib = p.idx + b * p.is[0] + tw * p.is[1];
    const int64_t rbase = (b * p.H + h) * p.T + tw;

    for (int r = 0; r < w.n; ++r) {
        const int t = int(tw) + r;
        uint4 qlo, qhi, glo, ghi;
        ld16<DT>(qb, uint32_t(r) * qrow + loff, qlo, qhi);
        ld16<DT>(gb, uint32_t(r) * grow + loff, glo, ghi);
        if (!lane_on) { qlo = make_uint4(0, 0, 0, 0); qhi = qlo; glo = qlo; ghi = qlo; }
        const float lt2 = p.lse2[rbase + r];
        const int lim = (mask_flag && t < K - 1) ? t + 1 : K;   // slots >= lim carry no weight
        const uint32_t rkey = DROP ? drop_row_key(p.drop, uint64_t(rbase + r)) : 0u;
        const int32_t* ip = ib + r * p.is[1];
        float A[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float Bk[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float dsum = 0.0f;
        for (int s0 = 0; s0 < K; s0 += 2 * NPS) {
            const int sl[2] = {s0 + grp, s0 + NPS + grp};
            uint4 klo[2], khi[2], vlo[2], vhi[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int j = wrap_index(ip[min(sl[u], K - 1)], T);
                ld16<DT>(kb, uint32_t(j) * krow + loff, klo[u], khi[u]);
                ld16<DT>(vb, uint32_t(j) * vrow + loff, vlo[u], vhi[u]);
            }
            float pu[2], pd[2];
            const uint32_t kb2 = DROP ? drop_bits2<LPN>(p.drop, rkey, rkey, uint32_t(sl[0]), uint32_t(sl[1]), sub, grp) : 3u;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const float d = group_sum<LPN>(dot8<DT>(qlo, qhi, klo[u], khi[u]));
                float dp = group_sum<LPN>(dot8<DT>(glo, ghi, vlo[u], vhi[u]));
                if (DROP) dp = (kb2 >> u) & 1u ? dp * p.drop.scale : 0.0f;
                // v_exp_f32 directly: 2^(s - lse) <= 1; masked slots get no weight
                pu[u] = sl[u] < lim ? __builtin_amdgcn_exp2f(d * sl2 - lt2) : 0.0f;
                pd[u] = pu[u] * dp;
                dsum += pd[u];
            }
            // both neighbours at once: v_dot2 over (k_a, k_b) pairs, weights in the input dtype
            pv2<DT>(A, pd[0], pd[1], klo[0], khi[0], klo[1], khi[1]);
            pv2<DT>(Bk, pu[0], pu[1], klo[0], khi[0], klo[1], khi[1]);
        }
        const float delta = group_allreduce<LPN, false>(dsum);
        float o8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float a = group_allreduce<LPN, false>(A[e]);
            const float bk = group_allreduce<LPN, false>(Bk[e]);
            o8[e] = p.scale * (a - delta * bk);
        }
        if (grp == 0) {
            if (lane_on) store_row8<DT, true>(reinterpret_cast<DT*>(db + uint32_t(r) * drow + loff), 1, o8);
            if (sub == 0) p.row_stats[rbase + r] = make_float2(lt2, delta);
        }
    }
}

// Key pass: dk and dv for key rows j of one (b, h) pair.
template <typename DT, int D, bool DROP>
__global__ __launch_bounds__(64 * kWaves) void readout_bwd_keys(ReadoutBwdParams p)
{
    constexpr int LPN = D / 8;
    constexpr int NPS = 64 / LPN;
    constexpr uint32_t ES = sizeof(DT);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sub = lane % LPN;
    const int grp = lane / LPN;
    const Pair w = map_rows(p, wave);
    if (w.n == 0) return;
    const int64_t b = w.b, h = w.h, jw = w.r0;
    const float sl2 = p.scale * kLog2e;

    const char* qb = reinterpret_cast<const char*>(static_cast<const DT*>(p.q) + b * p.qs[0] + h * p.qs[1]);
    const char* gb = reinterpret_cast<const char*>(static_cast<const DT*>(p.dout) + b * p.gs[0] + h * p.gs[1]);
    const char* kb = reinterpret_cast<const char*>(static_cast<const DT*>(p.k) + b * p.ks[0] + h * p.ks[1] + jw * p.ks[2]);
    const char* vb = reinterpret_cast<const char*>(static_cast<const DT*>(p.v) + b * p.vs[0] + h * p.vs[1] + jw * p.vs[2]);
    char* dkb = reinterpret_cast<char*>(static_cast<DT*>(p.dk) + b * p.dks[0] + h * p.dks[1] + jw * p.dks[2]);
    char* dvb = reinterpret_cast<char*>(static_cast<DT*>(p.dv) + b * p.dvs[0] + h * p.dvs[1] + jw * p.dvs[2]);
    const uint32_t qrow = uint32_t(p.qs[2]) * ES, grow = uint32_t(p.gs[2]) * ES;
    const uint32_t krow = uint32_t(p.ks[2]) * ES, vrow = uint32_t(p.vs[2]) * ES;
    const uint32_t dkrow = uint32_t(p.dks[2]) * ES, dvrow = uint32_t(p.dvs[2]) * ES;
    const int dv = int(p.D) / 8;   // lanes past the head dim: zero k / v slices, no stores
    const bool lane_on = sub < dv;
    const uint32_t loff = uint32_t(min(sub, dv - 1)) * 8u * ES;
    const float2* rs = p.row_stats + (b * p.H + h) * p.T;
    const uint32_t* off = p.off + b * p.T + jw;

    for (int r = 0; r < w.n; ++r) {
        uint4 klo, khi, vlo, vhi;
        ld16<DT>(kb, uint32_t(r) * krow + loff, klo, khi);
        ld16<DT>(vb, uint32_t(r) * vrow + loff, vlo, vhi);
        if (!lane_on) { klo = make_uint4(0, 0, 0, 0); khi = klo; vlo = klo; vhi = klo; }
        const uint32_t e0 = off[r], e1 = off[r + 1];
        float ak[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float av[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t e = e0; e < e1; e += 2 * NPS) {
            const uint32_t en[2] = {e + uint32_t(grp), e + uint32_t(NPS + grp)};
            int t[2];
            uint32_t slot[2];
            uint4 qlo[2], qhi[2], glo[2], ghi[2];
            float2 st[2];   // (lse2, delta) of the entry's query row
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t rv = en[u] < e1 ? p.rows[en[u]] : 0u;   // t * K + s
                t[u] = int(fdiv(rv, p.divK));
                slot[u] = rv - uint32_t(t[u]) * uint32_t(p.K);
                ld16<DT>(qb, uint32_t(t[u]) * qrow + loff, qlo[u], qhi[u]);
                ld16<DT>(gb, uint32_t(t[u]) * grow + loff, glo[u], ghi[u]);
                st[u] = rs[t[u]];
            }
            uint32_t kb2 = 3u;
            if (DROP) {
                const uint64_t rb0 = uint64_t(b * p.H + h) * uint64_t(p.T);
                kb2 = drop_bits2<LPN>(p.drop, drop_row_key(p.drop, rb0 + uint64_t(t[0])),
                                      drop_row_key(p.drop, rb0 + uint64_t(t[1])), slot[0], slot[1], sub, grp);
            }
            float pu[2], ds[2], pw[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const float d = group_sum<LPN>(dot8<DT>(qlo[u], qhi[u], klo, khi));
                float dp = group_sum<LPN>(dot8<DT>(glo[u], ghi[u], vlo, vhi));
                const float mc = DROP ? ((kb2 >> u) & 1u ? p.drop.scale : 0.0f) : 1.0f;
                if (DROP) dp *= mc;
                pu[u] = en[u] < e1 ? __builtin_amdgcn_exp2f(d * sl2 - st[u].x) : 0.0f;
                ds[u] = pu[u] * (dp - st[u].y);
                pw[u] = DROP ? pu[u] * mc : pu[u];   // the weight dout_t carries into dv
            }
            pv2<DT>(ak, ds[0], ds[1], qlo[0], qhi[0], qlo[1], qhi[1]);
            pv2<DT>(av, pw[0], pw[1], glo[0], ghi[0], glo[1], ghi[1]);
        }
        float ok8[8], ov8[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            ok8[c] = p.scale * group_allreduce<LPN, false>(ak[c]);
            ov8[c] = group_allreduce<LPN, false>(av[c]);
        }
        if (grp == 0 && lane_on) {
            store_row8<DT, true>(reinterpret_cast<DT*>(dkb + uint32_t(r) * dkrow + loff), 1, ok8);
            store_row8<DT, true>(reinterpret_cast<DT*>(dvb + uint32_t(r) * dvrow + loff), 1, ov8);
        }
    }
}

// ---------------------------------------------------------------- workspace layout
size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

int key_bits(int64_t B, int64_t T)
{
    int bits = 1;
    while ((int64_t(1) << bits) <= B * T) ++bits;   // keys take values 0 .. B*T
    return bits;
}

struct BwdLayout {
    size_t off, keys, keys_out, vals, vals_out, row_stats, hist, total, total_bytes;
    uint32_t nblk;
};

BwdLayout bwd_layout(int64_t B, int64_t H, int64_t T, int64_t K)
{
    BwdLayout L{};
    const size_t nkeys = size_t(B * T) + 1;
    const size_t n = size_t(B * T * K);
    L.nblk = uint32_t((n + kSortTile - 1) / kSortTile);
    size_t o = 0;
    L.off = o;       o += a256(nkeys * 4);
    L.keys = o;      o += a256(n * 4);
    L.keys_out = o;  o += a256(n * 4);
    L.vals = o;      o += a256(n * 4);
    L.vals_out = o;  o += a256(n * 4);
    L.row_stats = o; o += a256(size_t(B * H * T) * 8);
    L.hist = o;      o += a256(size_t(256) * L.nblk * 4);
    L.total = o;     o += a256(256 * 4);
    L.total_bytes = o;
    return L;
}

template <typename DT, bool DROP>
hipError_t launch_passes(const ReadoutBwdParams& p, hipStream_t s)
{
    const int64_t grid = 8 * (p.vpairs / 8) * p.wg_per_vpair;
    const dim3 g(static_cast<unsigned>(grid)), blk(64 * kWaves);
    // lane layout: the head dim padded to 32, 64, 128 or 256 (D / 8 lanes per neighbour)
    if (p.D <= 32) {
        readout_bwd_rows<DT, 32, DROP><<<g, blk, 0, s>>>(p);
        readout_bwd_keys<DT, 32, DROP><<<g, blk, 0, s>>>(p);
    } else if (p.D <= 64) {
        readout_bwd_rows<DT, 64, DROP><<<g, blk, 0, s>>>(p);
        readout_bwd_keys<DT, 64, DROP><<<g, blk, 0, s>>>(p);
    } else if (p.D <= 128) {
        readout_bwd_rows<DT, 128, DROP><<<g, blk, 0, s>>>(p);
        readout_bwd_keys<DT, 128, DROP><<<g, blk, 0, s>>>(p);
    } else {
        readout_bwd_rows<DT, 256, DROP><<<g, blk, 0, s>>>(p);
        readout_bwd_keys<DT, 256, DROP><<<g, blk, 0, s>>>(p);
    }
    return hipGetLastError();
}

template <typename DT>
hipError_t launch_passes_t(const ReadoutBwdParams& p, hipStream_t s)
{
    return p.drop_on ? launch_passes<DT, true>(p, s) : launch_passes<DT, false>(p, s);
}

}  // namespace

size_t sparse_readout_bwd_workspace(int64_t B, int64_t H, int64_t T, int64_t K)
{
    return bwd_layout(B, H, T, K).total_bytes;
}

hipError_t launch_sparse_readout_bwd(int dtype, ReadoutBwdParams p, void* ws, size_t ws_bytes, hipStream_t s)
{
    const BwdLayout L = bwd_layout(p.B, p.H, p.T, p.K);
    if (ws_bytes < L.total_bytes) return hipErrorInvalidValue;
    char* w = static_cast<char*>(ws);
    uint32_t* off = reinterpret_cast<uint32_t*>(w + L.off);
    uint32_t* A[2] = {reinterpret_cast<uint32_t*>(w + L.keys), reinterpret_cast<uint32_t*>(w + L.vals)};
    uint32_t* Z[2] = {reinterpret_cast<uint32_t*>(w + L.keys_out), reinterpret_cast<uint32_t*>(w + L.vals_out)};
    uint32_t* hist = reinterpret_cast<uint32_t*>(w + L.hist);
    uint32_t* total = reinterpret_cast<uint32_t*>(w + L.total);
    const uint32_t nkeys = uint32_t(p.B * p.T + 1);
    const uint32_t n = uint32_t(p.B * p.T * p.K);

    if (n > 0) {
        // 8-bit digits over the key range 0 .. B*T; ping-pong so the last pass lands in Z
        const int passes = (key_bits(p.B, p.T) + 7) / 8;
        SortSrc src{p.idx, p.is[0], p.is[1], p.is[2], uint32_t(p.B), uint32_t(p.T), uint32_t(p.K),
                    make_fastdiv(uint32_t(p.K)), make_fastdiv(uint32_t(p.T * p.K)),
                    (p.flags & 1u) != 0, nullptr, nullptr};
        for (int pass = 0; pass < passes; ++pass) {
            uint32_t* const* dst = (passes - 1 - pass) % 2 == 0 ? Z : A;
            const int shift = 8 * pass;
            radix_hist<<<dim3(L.nblk), dim3(kSortThreads), 0, s>>>(src, n, shift, L.nblk, hist);
            radix_scan<<<dim3(256), dim3(kSortThreads), 0, s>>>(hist, L.nblk, total);
            radix_scatter<<<dim3(L.nblk), dim3(kSortThreads), 0, s>>>(src, n, shift, L.nblk, hist, total,
                                                                     dst[0], dst[1]);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            src.keys = dst[0];
            src.vals = dst[1];
        }
    }
    bwd_list_offsets<<<dim3((nkeys + 255) / 256), dim3(256), 0, s>>>(Z[0], n, nkeys, off);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    p.row_stats = reinterpret_cast<float2*>(w + L.row_stats);
    p.off = off;
    p.rows = Z[1];
    p.divK = make_fastdiv(uint32_t(p.K));
    if (dtype == 2) return launch_passes_t<bf16_t>(p, s);
    if (dtype == 1) return launch_passes_t<_Float16>(p, s);
    return launch_passes_t<float>(p, s);
}

}  // namespace wf
