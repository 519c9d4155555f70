// Content comparison of index arrays with the snapshots kept in index plans,
// for reusing a plan only where the indices equal those it was built from:
// one pass compares the new (keys, gathers) with up to kMaxMatch plans'
// snapshots and flags each plan whose snapshot differs anywhere.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = kSnapTile / kThreads;

struct MatchLaunch {
    const uint32_t* keys[kMaxMatch];
    const uint32_t* gathers[kMaxMatch];
    const uint32_t* key_plain[kMaxMatch];
    const uint32_t* gather_plain[kMaxMatch];
    int num;
};

// Expected index of edge p in snapshot tile `tile`: the edge id where the
// tile is flagged plain, the stored value otherwise.
__device__ __forceinline__ int64_t snap_value(const uint32_t* __restrict__ vals,
                                              const uint32_t* __restrict__ plain, int64_t tile,
                                              int64_t p) {
    if (plain != nullptr && plain[tile] != 0u) return p;
    return static_cast<int64_t>(vals[p]);
}

// mismatch[c] becomes nonzero when plan c's snapshot differs from (keys,
// gathers) at some edge.  Workgroups sweep the snapshot tiles in rounds
// (tile = block + round * grid) and re-read the flags before each tile, so a
// comparison with different indices ends after the first round; the flags
// are read with device-scope loads (a stale read only delays that exit).
__global__ __launch_bounds__(kThreads) void k_plan_match(const int64_t* __restrict__ keys,
                                                         const int64_t* __restrict__ gathers,
                                                         int64_t n, MatchLaunch L,
                                                         int32_t* __restrict__ mismatch) {
    __shared__ int s_live;
    const int64_t tiles = (n + kSnapTile - 1) / kSnapTile;
    for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        __syncthreads();  // the previous round's reads of s_live are done
        if (threadIdx.x == 0) {
            int live = 0;
            for (int c = 0; c < L.num; ++c)
                if (__hip_atomic_load(mismatch + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0)
                    live |= 1 << c;
            s_live = live;
        }
        __syncthreads();
        const int live = s_live;
        if (live == 0) return;
        const int64_t base = tile * kSnapTile + threadIdx.x;
        int64_t k[kPerThread], g[kPerThread];
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int64_t p = base + i * kThreads;
            k[i] = p < n ? __builtin_nontemporal_load(keys + p) : 0;
            g[i] = (p < n && gathers != nullptr) ? __builtin_nontemporal_load(gathers + p) : 0;
        }
        for (int c = 0; c < L.num; ++c) {
            if (!((live >> c) & 1)) continue;
            int diff = 0;
#pragma unroll
            for (int i = 0; i < kPerThread; ++i) {
                const int64_t p = base + i * kThreads;
                if (p < n) {
                    diff |= k[i] != snap_value(L.keys[c], L.key_plain[c], tile, p);
                    if (gathers != nullptr)
                        diff |= g[i] != snap_value(L.gathers[c], L.gather_plain[c], tile, p);
                }
            }
            if (__syncthreads_or(diff) && threadIdx.x == 0) atomicOr(mismatch + c, 1);
        }
    }
}

}  // namespace

hipError_t launch_plan_match(const int64_t* keys, const int64_t* gathers, int64_t n,
                             const relm_mp_plan* const* plans, int num_plans, int32_t* mismatch,
                             hipStream_t s) {
    MatchLaunch L{};
    L.num = num_plans;
    for (int c = 0; c < num_plans; ++c) {
        L.keys[c] = reinterpret_cast<const uint32_t*>(plans[c]->snap_keys);
        L.key_plain[c] = plans[c]->snap_key_plain;
        L.gathers[c] = gathers != nullptr ? reinterpret_cast<const uint32_t*>(plans[c]->snap_gathers)
                                          : nullptr;
        L.gather_plain[c] = gathers != nullptr ? plans[c]->snap_gather_plain : nullptr;
    }
    hipError_t err = launch_fill_i32(mismatch, kMaxMatch, 0, s);
    if (err != hipSuccess || n == 0 || num_plans == 0) return err;
    // two workgroups per CU: enough to stream a full comparison at HBM rate
    const int64_t blocks = std::min<int64_t>((n + kSnapTile - 1) / kSnapTile, 512);
    hipLaunchKernelGGL(k_plan_match, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                       keys, gathers, n, L, mismatch);
    return hipGetLastError();
}

}  // namespace relm_mp
