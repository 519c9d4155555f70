// Index packing for the relm_mp pack ops (fanout/fanin_pack_multi,
// fanout/fanin_pack_from_edges): the index pairs of several parts are written,
// each element as `v * mul + add`, into two concatenated int64 arrays by one
// launch, instead of one elementwise kernel per part and a cat per array.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 4;
constexpr int64_t kBlockElems = kThreads * kPerThread;
constexpr int kPartsPerLaunch = 16;

// Parts of one launch.  Every workgroup covers kBlockElems consecutive
// elements of a single part, so the part lookup below is uniform per workgroup
// and its descriptor is read with scalar loads.  Arithmetic is unsigned: the
// results wrap modulo 2^64 as int64 tensor arithmetic does.
struct PackLaunch {
    const int64_t* a[kPartsPerLaunch];
    const int64_t* b[kPartsPerLaunch];
    uint64_t a_mul[kPartsPerLaunch];
    uint64_t a_add[kPartsPerLaunch];
    uint64_t b_mul[kPartsPerLaunch];
    uint64_t b_add[kPartsPerLaunch];
    int64_t n[kPartsPerLaunch];
    int64_t out_pos[kPartsPerLaunch];          // output position of the part's first pair
    uint32_t block_start[kPartsPerLaunch + 1];  // first workgroup of each part, then the grid
    int parts;
};

template <bool WRITE_B>
__global__ __launch_bounds__(kThreads) void k_pack_index(PackLaunch L, int64_t* __restrict__ out_a,
                                                         int64_t* __restrict__ out_b) {
    const uint32_t blk = blockIdx.x;
    int p = 0;
#pragma unroll
    for (int q = 1; q < kPartsPerLaunch; ++q)
        if (q < L.parts && blk >= L.block_start[q]) p = q;
    const int64_t n = L.n[p];
    const int64_t first = static_cast<int64_t>(blk - L.block_start[p]) * kBlockElems + threadIdx.x;
    const int64_t* __restrict__ a = L.a[p];
    const int64_t* __restrict__ b = L.b[p];
    int64_t* __restrict__ oa = out_a + L.out_pos[p];
    int64_t* __restrict__ ob = out_b + L.out_pos[p];
    uint64_t va[kPerThread], vb[kPerThread];
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        const int64_t j = first + k * kThreads;
        if (j < n) {
            va[k] = static_cast<uint64_t>(__builtin_nontemporal_load(a + j));
            if (WRITE_B) vb[k] = static_cast<uint64_t>(__builtin_nontemporal_load(b + j));
        }
    }
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        const int64_t j = first + k * kThreads;
        if (j < n) {
            oa[j] = static_cast<int64_t>(va[k] * L.a_mul[p] + L.a_add[p]);
            if (WRITE_B) ob[j] = static_cast<int64_t>(vb[k] * L.b_mul[p] + L.b_add[p]);
        }
    }
}

}  // namespace

hipError_t launch_pack_index(const relm_mp_index_part* parts, int num_parts, int64_t* out_a,
                             int64_t* out_b, hipStream_t s) {
    int64_t pos = 0;
    for (int first = 0; first < num_parts; first += kPartsPerLaunch) {
        PackLaunch L{};
        L.parts = std::min(kPartsPerLaunch, num_parts - first);
        int64_t blocks = 0;
        for (int q = 0; q < L.parts; ++q) {
            const relm_mp_index_part& P = parts[first + q];
            L.a[q] = P.a;
            L.b[q] = P.b;
            L.a_mul[q] = static_cast<uint64_t>(P.a_mul);
            L.a_add[q] = static_cast<uint64_t>(P.a_add);
            L.b_mul[q] = static_cast<uint64_t>(P.b_mul);
            L.b_add[q] = static_cast<uint64_t>(P.b_add);
            L.n[q] = P.n;
            L.out_pos[q] = pos;
            L.block_start[q] = static_cast<uint32_t>(blocks);
            blocks += (P.n + kBlockElems - 1) / kBlockElems;
            pos += P.n;
            if (blocks > 0x7fffffff) return hipErrorInvalidValue;
        }
        L.block_start[L.parts] = static_cast<uint32_t>(blocks);
        if (blocks == 0) continue;
        if (out_b != nullptr)
            hipLaunchKernelGGL(k_pack_index<true>, dim3(static_cast<unsigned>(blocks)),
                               dim3(kThreads), 0, s, L, out_a, out_b);
        else
            hipLaunchKernelGGL(k_pack_index<false>, dim3(static_cast<unsigned>(blocks)),
                               dim3(kThreads), 0, s, L, out_a, out_b);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

}  // namespace relm_mp
