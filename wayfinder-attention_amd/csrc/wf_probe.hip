// wf_probe.hip -- measurement aid: the sparse readout's gather path with no arithmetic.
//
// The readout (wf_readout.hip, sparse_readout_fast) is bound by its gathers of 16-byte
// slices of K/V rows, most of them served by L2, not by HBM bandwidth. This kernel issues
// exactly those loads -- same grid, workgroup order, rows per wave, lanes per neighbour,
// 16-byte index loads and K/V gathers, two tasks of gathers in flight per wave -- and folds
// the loaded words into one XOR per lane instead of the softmax, so its time is the speed
// of light of the readout's memory pattern at the readout's occupancy. Not part of the
// attention path; bench.py --leg gather reports the readout's time against it.
#include <atomic>

#include "wf_readout_dev.h"

namespace wf {
namespace {

template <typename DT, int D>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(4)))
void gather_probe_kernel(ReadoutParams p, uint32_t* sink)
{
    constexpr int LPN = D / 8;
    constexpr int NPS = 64 / LPN;
    constexpr int NB = 4;
    constexpr int CH = NB * NPS;
    constexpr uint32_t ES = sizeof(DT);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sub = lane % LPN;
    const int grp = lane / LPN;

    int64_t vp, chunk;
    if (p.head_major) {
        vp = blockIdx.x / p.wg_per_vpair;
        chunk = blockIdx.x % p.wg_per_vpair;
    } else {
        const int64_t it = blockIdx.x >> 3;
        vp = (it / p.wg_per_vpair) * 8 + (blockIdx.x & 7);
        chunk = it % p.wg_per_vpair;
    }
    uint32_t acc = 0;
    const int64_t gid = int64_t(blockIdx.x) * (64 * kWaves) + threadIdx.x;
    if (vp < p.vpairs) {
        const int64_t pair = vp / p.seg_per_pair;
        const int64_t seg = vp % p.seg_per_pair;
        const int64_t b = pair / p.H, h = pair % p.H;
        const int64_t t0 = p.row_begin + seg * p.rows_per_seg;
        const int64_t t1 = min(p.row_end, t0 + p.rows_per_seg);
        const int64_t tw = t0 + (chunk * kWaves + wave) * kRowsPerWave;
        if (tw < t1) {
            const int nrows = int(min(int64_t(kRowsPerWave), t1 - tw));
            const int K = int(p.K);
            const int nb = (K + CH - 1) / CH;
            const char* kb = reinterpret_cast<const char*>(static_cast<const DT*>(p.k) + b * p.ks[0] + h * p.ks[1]);
            const char* vb = reinterpret_cast<const char*>(static_cast<const DT*>(p.v) + b * p.vs[0] + h * p.vs[1]);
            const uint32_t krow = uint32_t(p.ks[2]) * ES, vrow = uint32_t(p.vs[2]) * ES;
            const uint32_t loff = uint32_t(sub) * 8u * ES;
            const int32_t* ib = p.idx + b * p.is[0] + tw * p.is[1];
            const int ntask = nrows * nb;
            auto indices = [&](int tau, int (&j)[NB]) {   // tasks past the end reload the last
                const int tt = min(tau, ntask - 1);
                const int s0 = min((tt % nb) * CH + grp * NB, K - NB);
                const uint4 w = *reinterpret_cast<const uint4*>(ib + (tt / nb) * p.is[1] + s0);
                const int Tm = int(p.T) - 1;   // clamped: the probe never reads outside K/V
                j[0] = min(max(int(w.x), 0), Tm); j[1] = min(max(int(w.y), 0), Tm);
                j[2] = min(max(int(w.z), 0), Tm); j[3] = min(max(int(w.w), 0), Tm);
            };
            auto gather = [&](const int (&j)[NB], uint4 (&kx)[NB], uint4 (&vx)[NB]) {
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    kx[u] = *reinterpret_cast<const uint4*>(kb + __umul24(uint32_t(j[u]), krow) + loff);
                    vx[u] = *reinterpret_cast<const uint4*>(vb + __umul24(uint32_t(j[u]), vrow) + loff);
                }
            };
            auto fold = [&](const uint4 (&kx)[NB], const uint4 (&vx)[NB]) {
#pragma unroll
                for (int u = 0; u < NB; ++u)
                    acc ^= kx[u].x ^ kx[u].y ^ kx[u].z ^ kx[u].w ^ vx[u].x ^ vx[u].y ^ vx[u].z ^ vx[u].w;
            };
            int jA[NB], jB[NB];
            uint4 kA[NB], vA[NB], kB[NB], vB[NB];
            indices(0, jA);
            gather(jA, kA, vA);
            indices(1, jB);
            for (int tau = 0; tau < ntask; tau += 2) {
                gather(jB, kB, vB);
                indices(tau + 2, jA);
                fold(kA, vA);
                gather(jA, kA, vA);
                indices(tau + 3, jB);
                if (tau + 1 < ntask) fold(kB, vB);
            }
        }
    }
    sink[gid] = acc;
}

template <void (*KFN)(ReadoutParams, uint32_t*)>
hipError_t launch_probe(ReadoutParams p, uint32_t* sink, hipStream_t s)
{
    static std::atomic<int64_t> cache[64];
    int dev = 0;
    int64_t resident = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) resident = cache[dev].load(std::memory_order_relaxed);
    if (resident <= 0) {
        resident = resident_workgroups(reinterpret_cast<const void*>(KFN), 64 * kWaves);
        if (dev >= 0 && dev < 64) cache[dev].store(resident, std::memory_order_relaxed);
    }
    const int64_t grid = 8 * (p.vpairs / 8) * p.wg_per_vpair;
    p.head_major = grid > resident ? 1 : 0;
    KFN<<<dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), 0, s>>>(p, sink);
    return hipGetLastError();
}

template <typename DT>
hipError_t launch_probe_t(const ReadoutParams& p, uint32_t* sink, hipStream_t s)
{
    if (p.D == 32) return launch_probe<gather_probe_kernel<DT, 32>>(p, sink, s);
    if (p.D == 64) return launch_probe<gather_probe_kernel<DT, 64>>(p, sink, s);
    return launch_probe<gather_probe_kernel<DT, 128>>(p, sink, s);
}

}  // namespace

hipError_t launch_gather_probe(int dtype, const ReadoutParams& p, uint32_t* sink, hipStream_t s)
{
    if (dtype == 2) return launch_probe_t<bf16_t>(p, sink, s);
    return launch_probe_t<_Float16>(p, sink, s);
}

}  // namespace wf
