// Content comparison of index arrays, for reusing an index plan built from
// equal indices held in other tensors: one pass compares the new (keys,
// gathers) against up to kMaxMatch candidate pairs and flags each candidate
// that differs anywhere.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 8;
constexpr int64_t kTile = kThreads * kPerThread;

struct MatchLaunch {
    const int64_t* keys[kMaxMatch];
    const int64_t* gathers[kMaxMatch];
    int num;
};

// mismatch[c] becomes nonzero when candidate c differs from (keys, gathers) in
// some position.  The workgroups sweep the tiles in rounds (tile = block +
// round * grid) and re-read the flags before each tile, so a comparison
// against different indices ends after the first round; the flags are read
// with device-scope loads (a stale read only delays that exit).
__global__ __launch_bounds__(kThreads) void k_index_match(const int64_t* __restrict__ keys,
                                                          const int64_t* __restrict__ gathers,
                                                          int64_t n, MatchLaunch L,
                                                          int32_t* __restrict__ mismatch) {
    __shared__ int s_live;
    const int64_t tiles = (n + kTile - 1) / kTile;
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
        const int64_t base = tile * kTile + threadIdx.x;
        int64_t k[kPerThread], g[kPerThread];
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int64_t p = base + i * kThreads;
            k[i] = p < n ? keys[p] : 0;
            g[i] = (p < n && gathers != nullptr) ? gathers[p] : 0;
        }
        for (int c = 0; c < L.num; ++c) {
            if (!((live >> c) & 1)) continue;
            const int64_t* __restrict__ ck = L.keys[c];
            const int64_t* __restrict__ cg = L.gathers[c];
            int diff = 0;
#pragma unroll
            for (int i = 0; i < kPerThread; ++i) {
                const int64_t p = base + i * kThreads;
                if (p < n) {
                    diff |= ck[p] != k[i];
                    if (gathers != nullptr) diff |= cg[p] != g[i];
                }
            }
            if (__syncthreads_or(diff) && threadIdx.x == 0) atomicOr(mismatch + c, 1);
        }
    }
}

}  // namespace

hipError_t launch_index_match(const int64_t* keys, const int64_t* gathers, int64_t n,
                              const int64_t* const* cand_keys, const int64_t* const* cand_gathers,
                              int num_cand, int32_t* mismatch, hipStream_t s) {
    MatchLaunch L{};
    L.num = num_cand;
    for (int c = 0; c < num_cand; ++c) {
        L.keys[c] = cand_keys[c];
        L.gathers[c] = gathers != nullptr ? cand_gathers[c] : nullptr;
    }
    hipError_t err = launch_fill_i32(mismatch, kMaxMatch, 0, s);
    if (err != hipSuccess || n == 0 || num_cand == 0) return err;
    // two workgroups per CU: enough to stream a full comparison at HBM rate
    const int64_t blocks = std::min<int64_t>((n + kTile - 1) / kTile, 512);
    hipLaunchKernelGGL(k_index_match, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                       keys, gathers, n, L, mismatch);
    return hipGetLastError();
}

}  // namespace relm_mp
