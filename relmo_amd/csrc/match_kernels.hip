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

using i64x2 = int64_t __attribute__((ext_vector_type(2)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));

// mismatch[c] becomes gen when plan c's snapshot differs from (keys,
// gathers) at some edge.  One snapshot tile per workgroup round (tile = block
// + round * grid; the grid covers every tile once for up to 2^16 tiles).  A
// workgroup first reads the flags of the candidates still live (device-scope
// loads; a stale read only delays an exit) and their plain-tile flags, and
// exits when none is live, so a comparison with different indices ends after
// the first tiles.  Thread t compares the edge pairs 2 * (i * 256 + t) +
// {0, 1}: 16-byte loads of the new indices, 8-byte loads of a stored tile.
// With spread > 0 (a probe ahead of the full pass) workgroup b compares tile
// b * spread only: the full pass's workgroups all start before any of them
// can flag a difference, so a probe over tiles across the whole range lets
// them exit at once when the indices differ in many places.
__global__ __launch_bounds__(kThreads) void k_plan_match(const int64_t* __restrict__ keys,
                                                         const int64_t* __restrict__ gathers,
                                                         int64_t n, MatchLaunch L,
                                                         int32_t* __restrict__ mismatch,
                                                         int32_t gen, int64_t spread) {
    constexpr int kPairs = kPerThread / 2;
    __shared__ int s_live;
    __shared__ int s_diff;
    __shared__ int s_plain;  // bit c: plan c's key tile plain; bit 16 + c: its gather tile
    const int64_t tiles = (n + kSnapTile - 1) / kSnapTile;
    const bool vec = ((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(gathers)) & 15u) == 0;
    const int64_t first = spread > 0 ? static_cast<int64_t>(blockIdx.x) * spread : blockIdx.x;
    const int64_t step = spread > 0 ? tiles : gridDim.x;  // a probe takes one tile
    for (int64_t tile = first; tile < tiles; tile += step) {
        __syncthreads();  // the previous round's reads of the shared words are done
        if (threadIdx.x == 0) {
            int live = 0, plain = 0;
            for (int c = 0; c < L.num; ++c) {
                if (__hip_atomic_load(mismatch + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen)
                    continue;
                live |= 1 << c;
                if (L.key_plain[c] != nullptr && L.key_plain[c][tile] != 0u) plain |= 1 << c;
                if (L.gather_plain[c] != nullptr && L.gather_plain[c][tile] != 0u) plain |= 1 << (16 + c);
            }
            s_live = live;
            s_plain = plain;
            s_diff = 0;
        }
        __syncthreads();
        const int live = s_live;
        if (live == 0) return;
        const int plain = s_plain;
        const int64_t tile_base = tile * kSnapTile;
        const bool full = vec && tile_base + kSnapTile <= n;
        int diff = 0;
        if (full) {
            i64x2 k[kPairs], g[kPairs];
#pragma unroll
            for (int i = 0; i < kPairs; ++i) {
                const int64_t p = tile_base + 2 * (i * kThreads + static_cast<int64_t>(threadIdx.x));
                k[i] = __builtin_nontemporal_load(reinterpret_cast<const i64x2*>(keys + p));
                g[i] = gathers != nullptr
                           ? __builtin_nontemporal_load(reinterpret_cast<const i64x2*>(gathers + p))
                           : i64x2{0, 0};
            }
            for (int c = 0; c < L.num; ++c) {
                if (!((live >> c) & 1)) continue;
                const bool kp = (plain >> c) & 1, gp = (plain >> (16 + c)) & 1;
                int d = 0;
#pragma unroll
                for (int i = 0; i < kPairs; ++i) {
                    const int64_t p = tile_base + 2 * (i * kThreads + static_cast<int64_t>(threadIdx.x));
                    if (kp) {
                        d |= (k[i].x != p) | (k[i].y != p + 1);
                    } else {
                        const u32x2 v = *reinterpret_cast<const u32x2*>(L.keys[c] + p);
                        d |= (k[i].x != static_cast<int64_t>(v.x)) | (k[i].y != static_cast<int64_t>(v.y));
                    }
                    if (gathers == nullptr) continue;
                    if (gp) {
                        d |= (g[i].x != p) | (g[i].y != p + 1);
                    } else {
                        const u32x2 v = *reinterpret_cast<const u32x2*>(L.gathers[c] + p);
                        d |= (g[i].x != static_cast<int64_t>(v.x)) | (g[i].y != static_cast<int64_t>(v.y));
                    }
                }
                diff |= d << c;
            }
        } else {
            for (int e = static_cast<int>(threadIdx.x); e < kSnapTile; e += kThreads) {
                const int64_t p = tile_base + e;
                if (p >= n) break;
                const int64_t kv = keys[p];
                const int64_t gv = gathers != nullptr ? gathers[p] : 0;
                for (int c = 0; c < L.num; ++c) {
                    if (!((live >> c) & 1)) continue;
                    const int64_t ek = ((plain >> c) & 1) ? p : static_cast<int64_t>(L.keys[c][p]);
                    int d = kv != ek;
                    if (gathers != nullptr) {
                        const int64_t eg =
                            ((plain >> (16 + c)) & 1) ? p : static_cast<int64_t>(L.gathers[c][p]);
                        d |= gv != eg;
                    }
                    diff |= d << c;
                }
            }
        }
        if (diff != 0) atomicOr(&s_diff, diff);
        __syncthreads();
        if (threadIdx.x == 0 && s_diff != 0) {
            const int dm = s_diff;
            for (int c = 0; c < L.num; ++c)
                if ((dm >> c) & 1)
                    __hip_atomic_store(mismatch + c, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Copies the flags to host memory, then stores gen behind them: the host
// polls host[kMaxMatch] and reads the flags once it equals gen.
__global__ void k_match_publish(const int32_t* __restrict__ mismatch, int num, int32_t gen,
                                int32_t* __restrict__ host) {
    const int c = static_cast<int>(threadIdx.x);
    if (c < num) host[c] = __hip_atomic_load(mismatch + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __threadfence_system();
    __syncthreads();
    if (c == 0) __hip_atomic_store(host + kMaxMatch, gen, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace

hipError_t launch_plan_match(const int64_t* keys, const int64_t* gathers, int64_t n,
                             const relm_mp_plan* const* plans, int num_plans, int32_t* mismatch,
                             int32_t gen, int32_t* host_words, hipStream_t s) {
    MatchLaunch L{};
    L.num = num_plans;
    for (int c = 0; c < num_plans; ++c) {
        L.keys[c] = reinterpret_cast<const uint32_t*>(plans[c]->snap_keys);
        L.key_plain[c] = plans[c]->snap_key_plain;
        L.gathers[c] = gathers != nullptr ? reinterpret_cast<const uint32_t*>(plans[c]->snap_gathers)
                                          : nullptr;
        L.gather_plain[c] = gathers != nullptr ? plans[c]->snap_gather_plain : nullptr;
    }
    hipError_t err = hipSuccess;
    const int64_t tiles = (n + kSnapTile - 1) / kSnapTile;
    if (tiles > 0 && num_plans > 0) {
        constexpr int64_t kProbe = 64;
        if (tiles > 4 * kProbe) {
            hipLaunchKernelGGL(k_plan_match, dim3(static_cast<unsigned>(kProbe)), dim3(kThreads), 0,
                               s, keys, gathers, n, L, mismatch, gen, tiles / kProbe);
            err = hipGetLastError();
            if (err != hipSuccess) return err;
        }
        // one workgroup per tile (a full comparison streams at HBM rate with
        // several workgroups resident per CU), grid-stride beyond 2^16 tiles
        const int64_t blocks = std::min<int64_t>(tiles, 65536);
        hipLaunchKernelGGL(k_plan_match, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                           keys, gathers, n, L, mismatch, gen, int64_t{0});
        err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    hipLaunchKernelGGL(k_match_publish, dim3(1), dim3(64), 0, s,
                       static_cast<const int32_t*>(mismatch), num_plans, gen, host_words);
    return hipGetLastError();
}

}  // namespace relm_mp
