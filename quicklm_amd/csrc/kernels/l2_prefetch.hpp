// Carrying out an L2 prefetch plan (qlm_l2_plan) from workgroups appended
// to a latency-bound kernel's grid.
//
// MI355X dispatches workgroup i of a launch to XCD i % 8, and an XCD's L2
// keeps what a kernel read for the kernels after it (measured with graph
// replays: a 12 MiB read from the L2 it was left in costs 1.8 us a launch
// against 3.6 us from HBM, and one from another XCD's L2 gains little). A
// kernel such as the DeltaNet mixer keeps HBM mostly idle for its ~5 us;
// workgroups appended to it load the next GEMV's first tiles into the L2 of
// the XCD whose workgroup will read them.
#pragma once

#include "common.hpp"

namespace {

typedef __attribute__((address_space(1))) void qlm_gvoid;
typedef __attribute__((address_space(3))) void qlm_lvoid;

constexpr int kL2Piece = 1024;  // bytes one wave instruction loads (16 a lane)

// Prefetching workgroups to append for `plan`: about 16 pieces a wave with
// 4-wave workgroups, a multiple of 8 (the same number on every XCD), at
// most 256. 0 for an empty plan.
inline int l2_plan_workgroups(const qlm_l2_plan& plan) {
    long long pieces = 0;
    for (int s = 0; s < plan.nseg && s < QLM_L2_PLAN_SEGMENTS; ++s)
        pieces += (long long)plan.tiles[s] * ((plan.bytes[s] + kL2Piece - 1) / kL2Piece);
    if (pieces <= 0) return 0;
    long long wg = (pieces + 63) / 64;
    wg = (wg + 7) / 8 * 8;
    return (int)(wg > 256 ? 256 : wg);
}

// Whether `plan` is well formed: segment count, sizes, 16-byte aligned
// pointers and strides (each lane loads 16 aligned bytes), and at most 2^26
// pieces in all (64 GB; the kernel counts pieces in 32-bit integers).
inline bool l2_plan_valid(const qlm_l2_plan& plan) {
    if (plan.nseg < 0 || plan.nseg > QLM_L2_PLAN_SEGMENTS) return false;
    long long pieces = 0;
    for (int s = 0; s < plan.nseg; ++s) {
        if (!plan.base[s] || (reinterpret_cast<uintptr_t>(plan.base[s]) & 15u) ||
            plan.bytes[s] <= 0 || plan.bytes[s] % 16 != 0 || plan.tiles[s] < 0 ||
            plan.stride[s] < 0 || plan.stride[s] % 16 != 0)
            return false;
        pieces += (long long)plan.tiles[s] * ((plan.bytes[s] + kL2Piece - 1) / kL2Piece);
    }
    return pieces <= (1ll << 26);
}

// Workgroup k of the `per` prefetching workgroups on XCD `xcd` loads its
// share of the plan's tiles t with t % 8 == xcd. The pieces of that XCD,
// counted over the segments in order (tile-major within a segment), go to
// its waves round robin. Each load lands in an LDS sink that is never read,
// so no registers are held and no load waits for another; the wave waits
// for all of them before it ends (the workgroup's LDS may be handed to
// another workgroup after that).
__device__ __forceinline__ void l2_prefetch(const qlm_l2_plan& plan, int xcd, int k, int per) {
    __shared__ __align__(16) unsigned char sink[kL2Piece];
    const int nwv = blockDim.x / QLM_WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / QLM_WAVE);
    const int lane = threadIdx.x & (QLM_WAVE - 1);
    const int step = per * nwv;
    int g = k * nwv + wave;  // this wave's next piece, over all segments
    int base = 0;            // pieces of the segments before s
#pragma unroll
    for (int s = 0; s < QLM_L2_PLAN_SEGMENTS; ++s) {
        if (s >= plan.nseg) break;
        const int cps = (plan.bytes[s] + kL2Piece - 1) / kL2Piece;
        const int ntx = xcd < plan.tiles[s] ? (plan.tiles[s] - 1 - xcd) / 8 + 1 : 0;
        const int n = ntx * cps;
        const char* b = static_cast<const char*>(plan.base[s]);
        if (g < base + n) {
            // piece (j, r): piece r of the XCD's j-th tile; advanced by step
            // pieces without a division per load
            int j = (g - base) / cps, r = (g - base) - j * cps;
            const int sj = step / cps, sr = step - sj * cps;
            for (; g < base + n; g += step) {
                // the last piece of a tile may be partial: its lanes past the
                // end read the tile's last 16 bytes again
                const int off = min(r * kL2Piece + lane * 16, plan.bytes[s] - 16);
                const char* p = b + (long long)(xcd + 8 * j) * plan.stride[s] + off;
                __builtin_amdgcn_global_load_lds((qlm_gvoid*)p, (qlm_lvoid*)sink, 16, 0, 0);
                j += sj;
                r += sr;
                if (r >= cps) {
                    r -= cps;
                    ++j;
                }
            }
        }
        base += n;
    }
    __builtin_amdgcn_s_waitcnt(0);
}

}  // namespace
