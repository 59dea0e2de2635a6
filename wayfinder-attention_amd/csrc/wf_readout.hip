// wf_readout.hip -- sparse attention readout over indices shared across heads (gfx950).
//
// Replaces routing_attention/kernels/fused_sparse.py:97-128 (_sparse_meat_batched) and
// :80-94 (sparse_meat_attention_reference). The reference materialises k_sel/v_sel as
// (B, H, T, K, D) tensors (2 GiB each at T=16384, H=8, K=128, bf16) and runs two batched
// GEMVs; here every gathered K/V row goes straight from memory to registers:
//
//  - a wave walks 4 consecutive (b, h, t) query rows; D/8 lanes share one neighbour (8 dims,
//    one 16-byte load each), so a wave step covers 64*8/D neighbours with full 128-byte
//    lines. The rows are cut into tasks of 4 steps and software-pipelined: indices are
//    fetched two tasks ahead and the K/V rows one task ahead of the compute;
//  - q.k uses v_dot2_f32_{bf16,f16} (fp32 FMA for fp32 inputs) and a DPP reduction over the
//    D/8 lanes of a neighbour; an online softmax (exp2, log2(e) folded into the scale)
//    carries max and sum across tasks; fp32 accumulation, one rounding to the output;
//  - workgroup order keeps each L2's working set to one or two heads' K and V (2 x T x D x s
//    bytes, 4 MiB at the benchmark shape, one XCD's L2): pair by pair for grids that run in
//    several residency waves, blockIdx % 8 -> fixed pairs (one XCD each under the initial
//    round-robin dispatch) for grids that fit in one (readout_block).
#include <atomic>

#include "wf_readout_dev.h"

namespace wf {
namespace {

// Workgroup -> (virtual pair, chunk of its rows). A grid that fits in one residency wave is
// dispatched round-robin over the 8 XCDs, so pairing blockIdx % 8 with a fixed set of virtual
// pairs keeps each pair's K and V in one XCD's L2. Larger grids are refilled as workgroups
// retire, wherever a slot frees up, so there the grid runs pair by pair instead: the
// resident workgroups then share one or two pairs' K/V in every L2 (measured 4-5 % faster
// at T >= 4096 than the XCD pairing, which mixes all pairs in every L2 after the first wave).
__device__ __forceinline__ void readout_block(const ReadoutParams& p, int64_t& vp, int64_t& chunk)
{
    if (p.head_major) {
        vp = blockIdx.x / p.wg_per_vpair;
        chunk = blockIdx.x % p.wg_per_vpair;
    } else {
        const int64_t it = blockIdx.x >> 3;
        vp = (it / p.wg_per_vpair) * 8 + (blockIdx.x & 7);
        chunk = it % p.wg_per_vpair;
    }
}

// One task = NB wave steps of one query row (NB * 64/LPN neighbour slots). The stage holds
// what a task needs before its compute: key indices, validity, the query slice.
template <int NB>
struct Stage {
    int j[NB];
    bool ok[NB];
    uint4 qlo, qhi;
};

// D: the lane layout's head dim (32, 64, 128, 256); the problem's p.D is any value up to D
// (lanes holding dims past p.D read zeros and store nothing; a slice the head dim ends in is
// read and written element by element). NB: wave steps per task.
template <typename DT, bool VEC, int D, int NB, bool DROP = false>
__global__ __launch_bounds__(64 * kWaves) void sparse_readout_kernel(ReadoutParams p)
{
    static_assert(!DROP || NB <= D / 8, "dropout: one keep bit per lane");
    constexpr int LPN = D / 8;       // lanes per neighbour
    constexpr int NPS = 64 / LPN;    // neighbours per wave step
    constexpr int CH = NB * NPS;     // neighbour slots per task
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane % LPN;      // 8-dim slice of the head
    const int grp = lane / LPN;      // neighbour within a step

    // XCD-aware mapping: blockIdx % 8 is the XCD; virtual pair vp runs on XCD vp % 8.
    int64_t vp, chunk;
    readout_block(p, vp, chunk);
    if (vp >= p.vpairs) return;
    const int64_t pair = vp / p.seg_per_pair;
    const int64_t seg = vp % p.seg_per_pair;
    const int64_t b = pair / p.H, h = pair % p.H;
    const int64_t t0 = p.row_begin + seg * p.rows_per_seg;
    const int64_t t1 = min(p.row_end, t0 + p.rows_per_seg);
    const int64_t tw = t0 + (chunk * kWaves + wave) * kRowsPerWave;   // first row of this wave
    if (tw >= t1) return;
    const int nrows = int(min(int64_t(kRowsPerWave), t1 - tw));

    const int64_t T = p.T;
    const int K = int(p.K);
    const int nb = (K + CH - 1) / CH;
    const int ntask = nrows * nb;
    const bool mask_flag = (p.flags & 1u) != 0;
    const float sl2 = p.scale * kLog2e;   // scale multiplies the finished dot, as in the reference

    const int nd = min(8, int(p.D) - sub * 8);   // dims of this lane's slice (<= 0: none)
    const int sl = nd > 0 ? sub : 0;             // slice addressed (in bounds for idle lanes)
    const DT* qbase = static_cast<const DT*>(p.q) + b * p.qs[0] + h * p.qs[1] + int64_t(sl) * 8 * p.qs[3];
    const DT* kbase = static_cast<const DT*>(p.k) + b * p.ks[0] + h * p.ks[1] + int64_t(sl) * 8 * p.ks[3];
    const DT* vbase = static_cast<const DT*>(p.v) + b * p.vs[0] + h * p.vs[1] + int64_t(sl) * 8 * p.vs[3];
    const int32_t* ibase = p.idx + b * p.is[0];
    // one slice: a 16-byte vector when the layout allows and the slice is whole, else the
    // slice's first nd elements one by one; zeros for lanes past the head dim
    auto load_slice = [&](const DT* ptr, int64_t sd, uint4& lo, uint4& hi) {
        if (nd >= 8) {
            load_row8<DT, VEC>(ptr, sd, lo, hi);
        } else if (nd > 0) {
            load_row8_part<DT>(ptr, sd, nd, lo, hi);
        } else {
            lo = make_uint4(0, 0, 0, 0);
            hi = lo;
        }
    };

    auto fetch_idx = [&](int tau, Stage<NB>& st) {
        const int64_t t = tw + tau / nb;
        const int bat = tau % nb;
        const int32_t* ip = ibase + t * p.is[1];
        const bool mp = mask_flag && t < K - 1;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int slot = bat * CH + u * NPS + grp;
            const bool in = slot < K;
            st.ok[u] = in && !(mp && slot > t);
            int64_t j = in ? int64_t(ip[int64_t(slot) * p.is[2]]) : 0;
            if (j < 0) j += T;
            st.j[u] = int(j < 0 ? 0 : (j > T - 1 ? T - 1 : j));
        }
        if (bat == 0) load_slice(qbase + t * p.qs[2], p.qs[3], st.qlo, st.qhi);
    };
    auto fetch_kv = [&](const Stage<NB>& st, uint4 (&klo)[NB], uint4 (&khi)[NB], uint4 (&vlo)[NB],
                        uint4 (&vhi)[NB]) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            load_slice(kbase + int64_t(st.j[u]) * p.ks[2], p.ks[3], klo[u], khi[u]);
            load_slice(vbase + int64_t(st.j[u]) * p.vs[2], p.vs[3], vlo[u], vhi[u]);
        }
    };

    uint4 qlo = make_uint4(0, 0, 0, 0), qhi = qlo;
    float m = -__builtin_inff(), l = 0.0f;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t rkey = 0;   // dropout: the row's hash key

    auto compute = [&](int tau, const Stage<NB>& st, const uint4 (&klo)[NB], const uint4 (&khi)[NB],
                       const uint4 (&vlo)[NB], const uint4 (&vhi)[NB]) {
        const int bat = tau % nb;
        if (bat == 0) {
            qlo = st.qlo;
            qhi = st.qhi;
            m = -__builtin_inff();
            l = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
            if (DROP) rkey = drop_row_key(p.drop, uint64_t(b * p.H + h) * uint64_t(T) + uint64_t(tw + tau / nb));
        }
        // dropout keep bits of the group's slots bat*CH + u*NPS + grp: lane sub < NB hashes
        // step sub's slot and one ballot hands every group its bits
        uint32_t kbits = 0;
        if (DROP)
            kbits = uint32_t(__ballot(sub < NB && drop_keep(p.drop, rkey, uint32_t(bat * CH + sub * NPS + grp))) >>
                             (grp * LPN));
        float sc[NB];
        float bm = -__builtin_inff();
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float d = group_sum<LPN>(dot8<DT>(qlo, qhi, klo[u], khi[u]));
            sc[u] = st.ok[u] ? d * sl2 : -__builtin_inff();
            bm = fmaxf(bm, sc[u]);
        }
        bm = across_groups<LPN, true>(bm);
        const float mn = fmaxf(m, bm);
        const float alpha = (mn == -__builtin_inff()) ? 1.0f : exp2f(m - mn);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float pu = st.ok[u] ? exp2f(sc[u] - mn) : 0.0f;
            l += pu;   // the normaliser counts every weight; dropout scales the values
            const float wu = DROP ? ((kbits >> u) & 1u ? pu * p.drop.scale : 0.0f) : pu;
            float vf[8];
            cvt8<DT>(vlo[u], vhi[u], vf);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(wu, vf[e], acc[e]);
        }
        m = mn;
        if (bat == nb - 1) {
            // combine the lane groups (different neighbours, same dims) and store the row
            const float lt = across_groups<LPN, false>(l);
            float o8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o8[e] = across_groups<LPN, false>(acc[e]);
            if (grp == 0) {
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) o8[e] *= inv;
                const int64_t t = tw + tau / nb;
                DT* op = static_cast<DT*>(p.out) + b * p.os[0] + h * p.os[1] + t * p.os[2] + int64_t(sl) * 8 * p.os[3];
                if (nd >= 8) store_row8<DT, VEC>(op, p.os[3], o8);
                else if (nd > 0) store_row8_part<DT>(op, p.os[3], nd, o8);
                if (p.lse2 && sub == 0) p.lse2[(b * p.H + h) * T + t] = m + log2f(lt);
            }
        }
    };

    // two-deep software pipeline: indices two tasks ahead, K/V one task ahead
    Stage<NB> sA, sB;
    uint4 kAlo[NB], kAhi[NB], vAlo[NB], vAhi[NB], kBlo[NB], kBhi[NB], vBlo[NB], vBhi[NB];
    fetch_idx(0, sA);
    fetch_kv(sA, kAlo, kAhi, vAlo, vAhi);
    if (ntask > 1) fetch_idx(1, sB);
    for (int tau = 0; tau < ntask; tau += 2) {
        if (tau + 1 < ntask) fetch_kv(sB, kBlo, kBhi, vBlo, vBhi);
        const Stage<NB> cA = sA;
        if (tau + 2 < ntask) fetch_idx(tau + 2, sA);
        compute(tau, cA, kAlo, kAhi, vAlo, vAhi);
        if (tau + 1 < ntask) {
            if (tau + 2 < ntask) fetch_kv(sA, kAlo, kAhi, vAlo, vAhi);
            const Stage<NB> cB = sB;
            if (tau + 3 < ntask) fetch_idx(tau + 3, sB);
            compute(tau + 1, cB, kBlo, kBhi, vBlo, vBhi);
        }
    }
}

// ---------------------------------------------------------------- fast path
// Aligned (B,T,H,D)-style layouts whose per-(b,h) span fits 32-bit byte offsets: every
// gather is a global load from a uniform 64-bit base plus a 32-bit per-lane offset. Each
// lane group keeps its own online-softmax state (max, sum, 8 accumulators) across the
// row's tasks; the groups are combined once per row (DPP row_ror within 16-lane rows, two
// shuffles across rows), so the per-step work has no LDS or ds_bpermute traffic.

// NB (even): wave steps per task. For 16-bit types the allocator is held to at most 128
// registers (the kernel needs 96: 5 waves per SIMD; more gathers in flight per CU were
// measured faster at every step from 3 waves up). The query slices of a wave's 4 rows sit in
// LDS (16 KiB per workgroup) rather than in registers.
// LSE: also write the row's base-2 log-sum-exp (the training forward, 4 waves per SIMD).
// TRUST: the indices are known to lie in [0, T) (they come from this library's retrieval),
// so the wrap/clamp is skipped.
// Byte offsets of gathered rows use 24-bit multiplies (T and the row strides below 2^24,
// checked by the host).
// VI: lane group g takes the NB consecutive slots g*NB .. g*NB+NB-1 of a task, so its
// indices arrive in one 16-byte load per task instead of one 4-byte load per step (a quarter
// of the vector-memory instructions); needs
// K % 4 == 0, 16-byte aligned index rows and K >= NB (checked by the launcher).
// D: the lane layout's head dim (32, 64, 128, 256); the problem's head dim p.D may be any
// multiple of 8 up to D. Lanes past p.D / 8 load the row's last slice (so no load is
// conditional), zero their query slice (so they add nothing to any dot product) and store
// nothing.
template <typename DT, int D, int NB, bool LSE, bool TRUST, bool VI, bool DROP = false>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(sizeof(DT) == 2 && !LSE ? 4 : 1)))
void sparse_readout_fast(ReadoutParams p)
{
    static_assert(!DROP || (LSE && NB <= D / 8), "dropout: training forward, one keep bit per lane");
    static_assert(NB % 2 == 0, "steps are consumed in pairs");
    static_assert(!VI || NB == 4, "one 16-byte index load per task");
    constexpr int LPN = D / 8;
    constexpr int NPS = 64 / LPN;
    constexpr int CH = NB * NPS;
    constexpr uint32_t ES = sizeof(DT);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    const int sub = lane % LPN;
    const int grp = lane / LPN;

    int64_t vp, chunk;
    readout_block(p, vp, chunk);
    if (vp >= p.vpairs) return;
    const int64_t pair = vp / p.seg_per_pair;
    const int64_t seg = vp % p.seg_per_pair;
    const int64_t b = pair / p.H, h = pair % p.H;
    const int64_t t0 = p.row_begin + seg * p.rows_per_seg;
    const int64_t t1 = min(p.row_end, t0 + p.rows_per_seg);
    const int64_t tw = t0 + (chunk * kWaves + wave) * kRowsPerWave;
    if (tw >= t1) return;
    const int nrows = int(min(int64_t(kRowsPerWave), t1 - tw));

    const int K = int(p.K);
    const int T = int(p.T);
    const int nb = (K + CH - 1) / CH;
    const bool mask_flag = (p.flags & 1u) != 0;
    const float sl2 = p.scale * kLog2e;

    const char* kb = reinterpret_cast<const char*>(static_cast<const DT*>(p.k) + b * p.ks[0] + h * p.ks[1]);
    const char* vb = reinterpret_cast<const char*>(static_cast<const DT*>(p.v) + b * p.vs[0] + h * p.vs[1]);
    const char* qb = reinterpret_cast<const char*>(static_cast<const DT*>(p.q) + b * p.qs[0] + h * p.qs[1] + tw * p.qs[2]);
    char* ob = reinterpret_cast<char*>(static_cast<DT*>(p.out) + b * p.os[0] + h * p.os[1] + tw * p.os[2]);
    const uint32_t krow = uint32_t(p.ks[2]) * ES, vrow = uint32_t(p.vs[2]) * ES;
    const uint32_t qrow = uint32_t(p.qs[2]) * ES, orow = uint32_t(p.os[2]) * ES;
    const int dv = int(p.D) / 8;                     // active lanes per neighbour
    const bool lane_on = sub < dv;
    const uint32_t loff = uint32_t(min(sub, dv - 1)) * 8u * ES;
    const int32_t* ib = p.idx + b * p.is[0] + tw * p.is[1];
    float* lrow = LSE ? p.lse2 + (b * p.H + h) * p.T + tw : nullptr;   // wave-uniform
    const int64_t irow = p.is[1];

    // Indices are loaded one pipeline step before the K/V gathers that use them, and issued
    // ahead of the gathers of the step in between: loads return in issue order, so waiting
    // for an index load then never waits for K/V rows still in flight.
    int ri = 0, qi = 0;   // task whose indices load next
    auto load_idx = [&](int (&jn)[NB]) {   // past the last task: reloads the last row's indices
        const char* ip = reinterpret_cast<const char*>(ib + min(ri, nrows - 1) * irow);
        if constexpr (VI) {
            // slots past K (masked in the compute) read the row's last NB indices instead
            const int s0 = min(qi * CH + grp * NB, K - NB);
            const uint4 w = *reinterpret_cast<const uint4*>(ip + uint32_t(s0) * 4u);
            jn[0] = int(w.x); jn[1] = int(w.y); jn[2] = int(w.z); jn[3] = int(w.w);
        } else {
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int slot = min(qi * CH + u * NPS + grp, K - 1);
                jn[u] = *reinterpret_cast<const int*>(ip + uint32_t(slot) * 4u);
            }
        }
        if (++qi == nb) { qi = 0; ++ri; }
    };
    auto advance = [&](int& r, int& q) { if (++q == nb) { q = 0; ++r; } };

    // compute state
    uint4 qlo = make_uint4(0, 0, 0, 0), qhi = qlo;
    float m = -__builtin_inff(), l = 0.0f;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int rc = 0, qc = 0;   // task being computed
    uint32_t rkey = 0;    // dropout: the row's hash key
    const uint64_t row_id0 = uint64_t(b * p.H + h) * uint64_t(T) + uint64_t(tw);

    // the query slices of the wave's rows, loaded once ahead of the pipeline and parked in
    // LDS (otherwise unused here) rather than in registers
    constexpr int QW = sizeof(DT) == 4 ? 2 : 1;   // 16-byte words per lane and row
    __shared__ uint4 sq[kWaves][kRowsPerWave][QW][64];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        uint4 lo, hi;
        ld16<DT>(qb, uint32_t(min(r, nrows - 1)) * qrow + loff, lo, hi);
        if (!lane_on) { lo = make_uint4(0, 0, 0, 0); hi = lo; }   // past the head dim
        sq[wave][r][0][lane] = lo;
        if constexpr (QW == 2) sq[wave][r][QW - 1][lane] = hi;
    }

    auto compute = [&](const uint4 (&klo)[NB], const uint4 (&khi)[NB], const uint4 (&vlo)[NB],
                       const uint4 (&vhi)[NB]) {
        if (qc == 0) {   // the wave's own LDS slot: no barrier needed
            qlo = sq[wave][rc][0][lane];
            if constexpr (QW == 2) qhi = sq[wave][rc][QW - 1][lane];
            m = -__builtin_inff();
            l = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
            if (DROP) rkey = drop_row_key(p.drop, row_id0 + uint64_t(rc));
        }
        const int t = int(tw) + rc;
        const int slot0 = qc * CH + (VI ? grp * NB : grp);   // slot of step u: slot0 + u * SU
        constexpr int SU = VI ? 1 : NPS;
        // dropout keep bits of the group's NB slots: lane sub < NB hashes slot0 + sub * SU and
        // one ballot hands every group its bits
        uint32_t kbits = 0;
        if (DROP)
            kbits = uint32_t(__ballot(sub < NB && drop_keep(p.drop, rkey, uint32_t(slot0 + sub * SU))) >>
                             (grp * LPN));
        const int lim = (mask_flag && t < K - 1) ? t + 1 : K;   // slots >= lim carry no weight
        float sc[NB];
        float bm = -__builtin_inff();
        if (lim >= (qc + 1) * CH) {   // wave-uniform: every slot of this task counts
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                sc[u] = group_sum<LPN>(dot8<DT>(qlo, qhi, klo[u], khi[u])) * sl2;
                bm = fmaxf(bm, sc[u]);
            }
        } else {
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const float d = group_sum<LPN>(dot8<DT>(qlo, qhi, klo[u], khi[u]));
                sc[u] = slot0 + u * SU < lim ? d * sl2 : -__builtin_inff();
                bm = fmaxf(bm, sc[u]);
            }
        }
        // v_exp_f32 directly (2^-inf = 0); ms keeps the arguments off -inf - -inf while
        // every slot seen so far is masked. Results below 2^-126 flush to zero, far below
        // the weights that matter after the max is subtracted.
        const float mn = fmaxf(m, bm);
        const float ms = mn == -__builtin_inff() ? 0.0f : mn;
        const float alpha = __builtin_amdgcn_exp2f(m - ms);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= alpha;
#pragma unroll
        for (int u = 0; u < NB; u += 2) {
            const float pa = __builtin_amdgcn_exp2f(sc[u] - ms);
            const float pc = __builtin_amdgcn_exp2f(sc[u + 1] - ms);
            l += pa + pc;   // the normaliser counts every weight; dropout scales the values
            if (DROP) {
                const float wa = (kbits >> u) & 1u ? pa * p.drop.scale : 0.0f;
                const float wc = (kbits >> (u + 1)) & 1u ? pc * p.drop.scale : 0.0f;
                pv2<DT>(acc, wa, wc, vlo[u], vhi[u], vlo[u + 1], vhi[u + 1]);
            } else {
                pv2<DT>(acc, pa, pc, vlo[u], vhi[u], vlo[u + 1], vhi[u + 1]);
            }
        }
        m = mn;
        if (qc == nb - 1) {
            const float mm = group_allreduce<LPN, true>(m);
            const float f = __builtin_amdgcn_exp2f(m - (mm == -__builtin_inff() ? 0.0f : mm));
            const float lt = group_allreduce<LPN, false>(l * f);
            float o8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o8[e] = group_allreduce<LPN, false>(acc[e] * f);
            if (grp == 0) {
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) o8[e] *= inv;
                if (lane_on) store_row8<DT, true>(reinterpret_cast<DT*>(ob + uint32_t(rc) * orow + loff), 1, o8);
                if (LSE && sub == 0) lrow[rc] = mm + log2f(lt);
            }
        }
        advance(rc, qc);
    };

    const int ntask = nrows * nb;
    uint4 kAlo[NB], kAhi[NB], vAlo[NB], vAhi[NB], kBlo[NB], kBhi[NB], vBlo[NB], vBhi[NB];
    int jA[NB], jB[NB];
    auto gather = [&](const int (&jn)[NB], uint4 (&klo)[NB], uint4 (&khi)[NB], uint4 (&vlo)[NB],
                      uint4 (&vhi)[NB]) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            int j = jn[u];
            if constexpr (!TRUST) {
                j += (j >> 31) & T;
                j = min(max(j, 0), T - 1);
            }
            ld16<DT>(kb, __umul24(uint32_t(j), krow) + loff, klo[u], khi[u]);
            ld16<DT>(vb, __umul24(uint32_t(j), vrow) + loff, vlo[u], vhi[u]);
        }
    };
    // per step: indices of task tau+2, K/V of task tau+1, compute task tau. Every load is
    // issued unconditionally (tasks past the end reload the last row's indices, in bounds,
    // unused): a load under a condition would leave the wait counts unknown and the compiler
    // would wait for every load in flight; as it is, each wait is for loads issued before the
    // gathers still in flight.
    load_idx(jA);
    gather(jA, kAlo, kAhi, vAlo, vAhi);
    load_idx(jB);
    // the load-issuing stretches run at wave priority 1, so a wave about to issue its
    // gathers is picked ahead of waves in their arithmetic (config 5 readout -1.3 %)
    for (int tau = 0; tau < ntask; tau += 2) {
        __builtin_amdgcn_s_setprio(1);
        load_idx(jA);
        gather(jB, kBlo, kBhi, vBlo, vBhi);
        __builtin_amdgcn_s_setprio(0);
        compute(kAlo, kAhi, vAlo, vAhi);
        __builtin_amdgcn_s_setprio(1);
        load_idx(jB);
        gather(jA, kAlo, kAhi, vAlo, vAhi);
        __builtin_amdgcn_s_setprio(0);
        if (tau + 1 < ntask) compute(kBlo, kBhi, vBlo, vBhi);
    }
}

// Workgroups of KFN resident at once on the current device, computed once per device from
// the kernel's occupancy and cached (one cache per kernel instantiation).
template <void (*KFN)(ReadoutParams)>
int64_t resident_cached()
{
    static std::atomic<int64_t> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return resident_workgroups(reinterpret_cast<const void*>(KFN), 64 * kWaves);
    int64_t n = cache[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        n = resident_workgroups(reinterpret_cast<const void*>(KFN), 64 * kWaves);
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Launch KFN over the grid of p. A grid larger than one residency wave runs virtual pair by
// virtual pair (head_major), a smaller one pairs blockIdx % 8 with fixed pairs.
template <void (*KFN)(ReadoutParams)>
hipError_t launch_readout(ReadoutParams p, hipStream_t s)
{
    const int64_t grid = 8 * (p.vpairs / 8) * p.wg_per_vpair;
    p.head_major = grid > resident_cached<KFN>() ? 1 : 0;
    KFN<<<dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), 0, s>>>(p);
    return hipGetLastError();
}

template <typename DT, int D>
hipError_t launch_fast_d(const ReadoutParams& p, hipStream_t s)
{
#ifndef WF_READOUT_FAST_NB
#define WF_READOUT_FAST_NB 4
#endif
    constexpr int NB = WF_READOUT_FAST_NB;
    // 16-byte index loads: K a multiple of 4 (row starts stay 16-byte aligned given an
    // aligned base and row strides that are multiples of 4)
    const bool vi = NB == 4 && p.K % 4 == 0 && p.K >= NB && reinterpret_cast<uintptr_t>(p.idx) % 16 == 0 &&
                    p.is[0] % 4 == 0 && p.is[1] % 4 == 0;
    if (p.drop_on) {   // training forward with dropout (lse2 is set)
        if (vi) return launch_readout<sparse_readout_fast<DT, D, NB, true, false, true, true>>(p, s);
        return launch_readout<sparse_readout_fast<DT, D, NB, true, false, false, true>>(p, s);
    }
    if (vi) {
        if (p.lse2) return launch_readout<sparse_readout_fast<DT, D, NB, true, false, true>>(p, s);
        if (p.flags & kFlagTrustedIndices) return launch_readout<sparse_readout_fast<DT, D, NB, false, true, true>>(p, s);
        return launch_readout<sparse_readout_fast<DT, D, NB, false, false, true>>(p, s);
    }
    if (p.lse2) return launch_readout<sparse_readout_fast<DT, D, NB, true, false, false>>(p, s);
    if (p.flags & kFlagTrustedIndices) return launch_readout<sparse_readout_fast<DT, D, NB, false, true, false>>(p, s);
    return launch_readout<sparse_readout_fast<DT, D, NB, false, false, false>>(p, s);
}

// Lane layout for head dim D: D / 8 lanes per neighbour, padded to a power of two >= 4.
template <typename DT>
hipError_t launch_fast_t(const ReadoutParams& p, hipStream_t s)
{
    if (p.D <= 32) return launch_fast_d<DT, 32>(p, s);
    if (p.D <= 64) return launch_fast_d<DT, 64>(p, s);
    if (p.D <= 128) return launch_fast_d<DT, 128>(p, s);
    return launch_fast_d<DT, 256>(p, s);
}

template <typename DT, bool VEC, int D>
hipError_t launch_d(const ReadoutParams& p, hipStream_t s)
{
#ifndef WF_READOUT_NB
#define WF_READOUT_NB 4
#endif
    constexpr int NB = WF_READOUT_NB;
    if (p.drop_on) return launch_readout<sparse_readout_kernel<DT, VEC, D, NB, true>>(p, s);
    return launch_readout<sparse_readout_kernel<DT, VEC, D, NB>>(p, s);
}

template <typename DT, bool VEC>
hipError_t launch_v(const ReadoutParams& p, hipStream_t s)
{
    if (p.D <= 32) return launch_d<DT, VEC, 32>(p, s);
    if (p.D <= 64) return launch_d<DT, VEC, 64>(p, s);
    if (p.D <= 128) return launch_d<DT, VEC, 128>(p, s);
    return launch_d<DT, VEC, 256>(p, s);
}

template <typename DT>
hipError_t launch_t(bool vec, const ReadoutParams& p, hipStream_t s)
{
    return vec ? launch_v<DT, true>(p, s) : launch_v<DT, false>(p, s);
}

}  // namespace

hipError_t launch_sparse_readout(int dtype, bool vec, bool fast, const ReadoutParams& p, hipStream_t s)
{
    if (fast) {
        if (dtype == 2) return launch_fast_t<bf16_t>(p, s);
        if (dtype == 1) return launch_fast_t<_Float16>(p, s);
        return launch_fast_t<float>(p, s);
    }
    if (dtype == 2) return launch_t<bf16_t>(vec, p, s);
    if (dtype == 1) return launch_t<_Float16>(vec, p, s);
    return launch_t<float>(vec, p, s);
}

}  // namespace wf
