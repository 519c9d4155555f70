// Index-plan kernels: validation, inverse maps, device scan, stable LSD radix
// sort by key, CSR offsets and hub lists.  All of these are integer work: the
// bound is HBM traffic over the index arrays.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>

#include "device_utils.h"
#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kThreads = 256;

inline unsigned grid_1d(int64_t work, int per_block, int64_t cap = 1ll << 20) {
    int64_t b = (work + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > cap) b = cap;
    return static_cast<unsigned>(b);
}

__global__ __launch_bounds__(kThreads) void k_fill_i32(int32_t* __restrict__ p, int64_t n,
                                                       int32_t value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        p[i] = value;
}

__global__ void k_status_init(DevStatus* st) {
    if (threadIdx.x == 0) {
        st->bad_key_edge = kNoEdge;
        st->bad_gather_edge = kNoEdge;
        st->collisions = 0;
        st->num_hubs = 0;
        st->num_chunks = 0;
        st->max_degree = 0;
        st->num_multi_hubs = 0;
        st->total_weight = 0;
        st->gather_mismatch = 0;
        st->key_mismatch = 0;
    }
}

// inv[k] = max e with keys[e] == k.  Every key and gathered index is checked;
// the smallest offending edge of each array is recorded.
__global__ __launch_bounds__(kThreads) void k_inv_build(const int64_t* __restrict__ keys,
                                                        int64_t key_bound,
                                                        const int64_t* __restrict__ gathers,
                                                        int64_t gather_bound, int64_t n,
                                                        int32_t* __restrict__ inv,
                                                        DevStatus* __restrict__ st) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    unsigned long long collisions = 0;
    bool mismatch = false;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * blockDim.x; base < n; base += stride) {
        const int64_t e = base + threadIdx.x;
        bool coll = false;
        if (e < n) {
            const int64_t k = keys[e];
            mismatch = mismatch || k != e;
            const bool bad_k = static_cast<uint64_t>(k) >= static_cast<uint64_t>(key_bound);
            if (bad_k) atomicMin(&st->bad_key_edge, static_cast<unsigned long long>(e));
            if (gathers != nullptr) {
                const int64_t g = gathers[e];
                if (static_cast<uint64_t>(g) >= static_cast<uint64_t>(gather_bound))
                    atomicMin(&st->bad_gather_edge, static_cast<unsigned long long>(e));
            }
            if (!bad_k) {
                const int32_t old = atomicMax(inv + k, static_cast<int32_t>(e));
                coll = old >= 0;
            }
        }
        collisions += __popcll(__ballot(coll));
    }
    if (lane_id() == 0 && collisions != 0) atomicAdd(&st->collisions, collisions);
    if (__ballot(mismatch) != 0 && lane_id() == 0) atomicOr(&st->key_mismatch, 1ull);
}

// ---- scan ----------------------------------------------------------------

__global__ __launch_bounds__(kScanThreads) void k_scan_tile_sums(const uint32_t* __restrict__ in,
                                                                 int64_t n,
                                                                 uint32_t* __restrict__ sums) {
    __shared__ uint32_t lds[kScanThreads / kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t p = base + static_cast<int64_t>(i) * kScanThreads + threadIdx.x;
        if (p < n) s += in[p];
    }
    uint32_t total;
    block_inclusive_scan<kScanThreads>(s, lds, total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Exclusive scan of one tile per block, in place, with a per-tile carry.
// Exclusive scan of every row of a [gridDim.x, len] array in place (one
// workgroup per row, kScanTile values per step with a running carry);
// tot[row] receives the row's sum.
__global__ __launch_bounds__(kScanThreads) void k_scan_rows(uint32_t* __restrict__ data,
                                                            int64_t len,
                                                            uint32_t* __restrict__ tot) {
    __shared__ uint32_t tile[kScanTile];
    __shared__ uint32_t lds[kScanThreads / kWave];
    uint32_t* row = data + static_cast<int64_t>(blockIdx.x) * len;
    uint32_t carry = 0;
    for (int64_t base = 0; base < len; base += kScanTile) {
        uint32_t in[kScanItems];
#pragma unroll
        for (int i = 0; i < kScanItems; ++i) {
            const int64_t p = base + static_cast<int64_t>(i) * kScanThreads + threadIdx.x;
            in[i] = p < len ? row[p] : 0u;
        }
#pragma unroll
        for (int i = 0; i < kScanItems; ++i) tile[i * kScanThreads + threadIdx.x] = in[i];
        __syncthreads();
        uint32_t v[kScanItems];
        uint32_t sum = 0;
#pragma unroll
        for (int i = 0; i < kScanItems; ++i) {
            v[i] = tile[threadIdx.x * kScanItems + i];
            sum += v[i];
        }
        uint32_t total;
        const uint32_t incl = block_inclusive_scan<kScanThreads>(sum, lds, total);
        uint32_t run = incl - sum + carry;
#pragma unroll
        for (int i = 0; i < kScanItems; ++i) {
            tile[threadIdx.x * kScanItems + i] = run;
            run += v[i];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kScanItems; ++i) {
            const int64_t p = base + static_cast<int64_t>(i) * kScanThreads + threadIdx.x;
            if (p < len) row[p] = tile[i * kScanThreads + threadIdx.x];
        }
        carry += total;
        __syncthreads();  // tile is rewritten by the next step
    }
    if (threadIdx.x == 0) tot[blockIdx.x] = carry;
}

__global__ __launch_bounds__(kScanThreads) void k_scan_tile_apply(uint32_t* __restrict__ data,
                                                                  int64_t n,
                                                                  const uint32_t* __restrict__ carry) {
    __shared__ uint32_t tile[kScanTile];
    __shared__ uint32_t lds[kScanThreads / kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t p = base + static_cast<int64_t>(i) * kScanThreads + threadIdx.x;
        tile[i * kScanThreads + threadIdx.x] = p < n ? data[p] : 0u;
    }
    __syncthreads();
    uint32_t v[kScanItems];
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        v[i] = tile[threadIdx.x * kScanItems + i];
        s += v[i];
    }
    uint32_t total;
    const uint32_t incl = block_inclusive_scan<kScanThreads>(s, lds, total);
    uint32_t run = incl - s + (carry != nullptr ? carry[blockIdx.x] : 0u);
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        tile[threadIdx.x * kScanItems + i] = run;
        run += v[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t p = base + static_cast<int64_t>(i) * kScanThreads + threadIdx.x;
        if (p < n) data[p] = tile[i * kScanThreads + threadIdx.x];
    }
}

// ---- radix sort ----------------------------------------------------------

// Tile digit histogram in LDS: kSubHists copies per wave (lane & 3), so that
// lanes holding the same digit - frequent for hub keys - rarely hit the same
// address; plain LDS atomics, no cross-lane matching.
constexpr int kSubHists = 4;

__device__ __forceinline__ void hist_clear(uint32_t* h) {
    for (int i = static_cast<int>(threadIdx.x); i < (kSortThreads / kWave) * kSubHists * kSortBins;
         i += kSortThreads)
        h[i] = 0;
}

__device__ __forceinline__ void hist_add(uint32_t* h, uint32_t d) {
    const int copy = (static_cast<int>(threadIdx.x) / kWave) * kSubHists + (lane_id() & (kSubHists - 1));
    atomicAdd(&h[copy * kSortBins + d], 1u);
}

// Sum of the copies for digit threadIdx.x (call after a barrier).
__device__ __forceinline__ uint32_t hist_total(const uint32_t* h) {
    uint32_t t = 0;
#pragma unroll
    for (int c = 0; c < (kSortThreads / kWave) * kSubHists; ++c) t += h[c * kSortBins + threadIdx.x];
    return t;
}

// First pass over the caller's int64 arrays: validates every key (and
// gathered index), narrows both to int32 for the sort passes and counts the
// tile's digits of the first pass (hist[d * nblocks + tile]).  Gathered
// indices equal to their edge ids (or no gathers) are common; a tile made of
// those only is flagged in tile_plain instead of written, and the first
// scatter generates its values.
__global__ __launch_bounds__(kSortThreads) void k_radix_narrow(
    const int64_t* __restrict__ keys, const int64_t* __restrict__ gathers, int64_t n, int shift,
    int bits, int64_t key_bound, int64_t gather_bound, uint32_t* __restrict__ keys32,
    uint32_t* __restrict__ vals32, uint32_t* __restrict__ tile_plain, uint32_t* __restrict__ hist,
    int64_t nblocks, DevStatus* __restrict__ st) {
    __shared__ uint32_t h[(kSortThreads / kWave) * kSubHists * kSortBins];
    hist_clear(h);
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
    const uint32_t dmask = (1u << bits) - 1u;
    unsigned long long bad_k = kNoEdge, bad_g = kNoEdge;
    uint32_t key[kSortItems], val[kSortItems];
    int mismatch = 0;
#pragma unroll
    for (int i = 0; i < kSortItems; ++i) {
        const int64_t p = base + static_cast<int64_t>(i) * kSortThreads + threadIdx.x;
        key[i] = 0;
        val[i] = 0;
        if (p < n) {
            const int64_t k = keys[p];
            if (static_cast<uint64_t>(k) >= static_cast<uint64_t>(key_bound))
                bad_k = min(bad_k, static_cast<unsigned long long>(p));
            else
                key[i] = static_cast<uint32_t>(k);
            if (gathers != nullptr) {
                const int64_t g = gathers[p];
                if (static_cast<uint64_t>(g) >= static_cast<uint64_t>(gather_bound))
                    bad_g = min(bad_g, static_cast<unsigned long long>(p));
                else
                    val[i] = static_cast<uint32_t>(g);
                mismatch |= g != p ? 1 : 0;
            }
        }
    }
    // block-wide: does any gathered index differ from its edge id?  (also the
    // barrier after clearing h)
    const int any = __syncthreads_or(mismatch);
#pragma unroll
    for (int i = 0; i < kSortItems; ++i) {
        const int64_t p = base + static_cast<int64_t>(i) * kSortThreads + threadIdx.x;
        if (p < n) {
            keys32[p] = key[i];
            if (any) vals32[p] = val[i];
        }
    }
#pragma unroll
    for (int i = 0; i < kSortItems; ++i) {
        const int64_t p = base + static_cast<int64_t>(i) * kSortThreads + threadIdx.x;
        if (p < n) hist_add(h, (key[i] >> shift) & dmask);
    }
    if (bad_k != kNoEdge) atomicMin(&st->bad_key_edge, bad_k);
    if (bad_g != kNoEdge) atomicMin(&st->bad_gather_edge, bad_g);
    if (threadIdx.x == 0) {
        tile_plain[blockIdx.x] = any ? 0u : 1u;
        if (any) atomicOr(&st->gather_mismatch, 1ull);
    }
    __syncthreads();
    hist[static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x] = hist_total(h);
}

// Per-tile digit histogram of the narrowed keys, written digit-major:
// hist[d * nblocks + tile].
__global__ __launch_bounds__(kSortThreads) void k_radix_upsweep(const uint32_t* __restrict__ keys,
                                                                int64_t n, int shift, int bits,
                                                                uint32_t* __restrict__ hist,
                                                                int64_t nblocks) {
    __shared__ uint32_t h[(kSortThreads / kWave) * kSubHists * kSortBins];
    hist_clear(h);
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
    const uint32_t dmask = (1u << bits) - 1u;
    uint32_t key[kSortItems];
#pragma unroll
    for (int i = 0; i < kSortItems; ++i) {
        const int64_t p = base + static_cast<int64_t>(i) * kSortThreads + threadIdx.x;
        key[i] = p < n ? keys[p] : 0u;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSortItems; ++i) {
        const int64_t p = base + static_cast<int64_t>(i) * kSortThreads + threadIdx.x;
        if (p < n) hist_add(h, (key[i] >> shift) & dmask);
    }
    __syncthreads();
    hist[static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x] = hist_total(h);
}

// Stable scatter of one tile.  Wave w owns tile positions [w*1024, (w+1)*1024)
// in 16 rounds of 64, so the order (wave, round, lane) is the edge order; each
// key's rank is counted in that order, the tile is staged in LDS in digit order
// and written out in runs per digit.  In the first pass a tile flagged in
// tile_plain takes the edge ids as its values.
__global__ __launch_bounds__(kSortThreads) void k_radix_downsweep(
    const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
    const uint32_t* __restrict__ tile_plain, int64_t n, int shift, int bits,
    const uint32_t* __restrict__ hist_scanned, const uint32_t* __restrict__ digit_tot,
    int64_t nblocks, uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out) {
    constexpr int kWaves = kSortThreads / kWave;
    constexpr int kPerWave = kSortTile / kWaves;
    __shared__ uint32_t wcnt[kWaves][kSortBins];
    __shared__ uint32_t dstart[kSortBins];
    __shared__ uint32_t gbase[kSortBins];
    __shared__ uint32_t scan_lds[kSortThreads / kWave];
    __shared__ uint32_t sk[kSortTile];
    __shared__ uint32_t sv[kSortTile];

    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int64_t tile_base = static_cast<int64_t>(blockIdx.x) * kSortTile;
    const uint32_t dmask = (1u << bits) - 1u;
    // this tile's start within each digit does not depend on the keys: fetch
    // it together with them
    const uint32_t tile_prefix = hist_scanned[static_cast<int64_t>(threadIdx.x) * nblocks + blockIdx.x];
    const uint32_t dt = digit_tot[threadIdx.x];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wcnt[w][threadIdx.x] = 0;
    __syncthreads();

    uint32_t key[kSortItems], val[kSortItems], rank[kSortItems];
    const bool plain = tile_plain != nullptr && tile_plain[blockIdx.x] != 0u;
    const int64_t wave_base = tile_base + wave * kPerWave + lane;
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const int64_t p = wave_base + r * kWave;
        uint32_t k = 0, v = 0;
        if (p < n) {
            k = keys[p];
            v = plain ? static_cast<uint32_t>(p) : vals[p];
        }
        key[r] = k;
        val[r] = v;
    }
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const bool active = wave_base + r * kWave < n;
        const uint32_t d = (key[r] >> shift) & dmask;
        const unsigned long long peers = match_digit(d, bits, __ballot(active));
        const uint32_t below = __popcll(peers & lanemask_lt());
        uint32_t before = 0;
        if (active) before = wcnt[wave][d];
        rank[r] = before + below;
        if (active && below == 0) wcnt[wave][d] = before + __popcll(peers);
    }

    __syncthreads();

    // Per digit (one thread per digit): exclusive prefix over waves, tile total.
    const int dd = static_cast<int>(threadIdx.x);
    uint32_t run = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const uint32_t c = wcnt[w][dd];
        wcnt[w][dd] = run;
        run += c;
    }
    uint32_t total;
    const uint32_t incl = block_inclusive_scan<kSortThreads>(run, scan_lds, total);
    dstart[dd] = incl - run;
    // global start of digit dd: all smaller digits of every tile, then this
    // digit in the tiles before this one (rows of hist_scanned)
    uint32_t all;
    const uint32_t dincl = block_inclusive_scan<kSortThreads>(dt, scan_lds, all);
    gbase[dd] = (dincl - dt) + tile_prefix;
    __syncthreads();

    const int64_t rem = n - tile_base;
    const int count = rem < kSortTile ? static_cast<int>(rem) : kSortTile;
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const int local = wave * kPerWave + r * kWave + lane;
        if (local < count) {
            const uint32_t d = (key[r] >> shift) & dmask;
            const uint32_t pos = dstart[d] + wcnt[wave][d] + rank[r];
            if (pos < static_cast<uint32_t>(count)) {
                sk[pos] = key[r];
                sv[pos] = val[r];
            }
        }
    }
    __syncthreads();
    for (int i = static_cast<int>(threadIdx.x); i < count; i += kSortThreads) {
        const uint32_t k = sk[i];
        const uint32_t d = (k >> shift) & dmask;
        const int64_t op = static_cast<int64_t>(gbase[d]) + (i - static_cast<int64_t>(dstart[d]));
        if (op >= 0 && op < n) {
            keys_out[op] = k;
            vals_out[op] = sv[i];
        }
    }
}

// offsets[k] = first sorted position with key >= k; offsets[num_keys] = n.
__global__ __launch_bounds__(kThreads) void k_offsets_from_sorted(const uint32_t* __restrict__ ks,
                                                                  int64_t n, int64_t num_keys,
                                                                  int32_t* __restrict__ offsets) {
    // thread t covers positions [4t, 4t + 4) (one 16-byte load) and writes
    // offsets[k] = i for every key k in (ks[i - 1], ks[i]]; position n closes
    // the keys after the last edge.
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; 4 * t <= n;
         t += stride) {
        const int64_t i0 = 4 * t;
        int64_t cur[4];
        if (i0 + 4 <= n) {
            const uint4 v = *reinterpret_cast<const uint4*>(ks + i0);
            cur[0] = v.x; cur[1] = v.y; cur[2] = v.z; cur[3] = v.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) cur[j] = i0 + j < n ? static_cast<int64_t>(ks[i0 + j]) : num_keys;
        }
        int64_t prev = i0 == 0 ? -1 : static_cast<int64_t>(ks[i0 - 1]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (i0 + j > n) break;
            const int64_t c = cur[j] > num_keys ? num_keys : cur[j];
            for (int64_t k = prev + 1; k <= c; ++k) offsets[k] = static_cast<int32_t>(i0 + j);
            prev = c > prev ? c : prev;
        }
    }
}

// Hub list in two passes over the segment sizes, without global atomics:
// k_hub_count writes per-block counts (hubs, chunks, big hubs) and the block's
// longest segment; the counts are scanned; k_hub_write gives every hub its
// slot (hubs in key order) and chunk range.
struct HubFlags {
    uint32_t hub;
    uint32_t chunks;
    uint32_t multi;
    int64_t deg;
};

__device__ __forceinline__ HubFlags hub_flags(const int32_t* __restrict__ offsets, int64_t k,
                                              int64_t num_keys) {
    HubFlags f{0u, 0u, 0u, 0};
    if (k < num_keys) f.deg = static_cast<int64_t>(offsets[k + 1]) - offsets[k];
    if (f.deg > kHubThreshold) {
        f.hub = 1u;
        f.chunks = static_cast<uint32_t>((f.deg + kChunkSize - 1) / kChunkSize);
        f.multi = f.chunks > 1u ? 1u : 0u;
    }
    return f;
}

__global__ __launch_bounds__(kThreads) void k_hub_count(const int32_t* __restrict__ offsets,
                                                        int64_t num_keys, int64_t nblk,
                                                        uint32_t* __restrict__ counts) {
    __shared__ uint32_t lds[kThreads / kWave];
    __shared__ uint32_t wmax[kThreads / kWave];
    const int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const HubFlags f = hub_flags(offsets, k, num_keys);
    uint32_t th, tc, tb;
    block_inclusive_scan<kThreads>(f.hub, lds, th);
    block_inclusive_scan<kThreads>(f.chunks, lds, tc);
    block_inclusive_scan<kThreads>(f.multi, lds, tb);
    uint32_t m = f.deg > 0 ? static_cast<uint32_t>(f.deg) : 0u;
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const uint32_t other = __shfl_xor(m, o, kWave);
        m = other > m ? other : m;
    }
    if (lane_id() == 0) wmax[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t mm = 0;
        for (int w = 0; w < kThreads / kWave; ++w) mm = wmax[w] > mm ? wmax[w] : mm;
        const int64_t stride = nblk + 1;
        counts[blockIdx.x] = th;
        counts[stride + blockIdx.x] = tc;
        counts[2 * stride + blockIdx.x] = tb;
        counts[3 * stride + blockIdx.x] = mm;
        if (blockIdx.x == 0) {
            counts[nblk] = 0;
            counts[stride + nblk] = 0;
            counts[2 * stride + nblk] = 0;
        }
    }
}

__global__ __launch_bounds__(kThreads) void k_hub_write(const int32_t* __restrict__ offsets,
                                                        int64_t num_keys, int64_t nblk,
                                                        const uint32_t* __restrict__ counts,
                                                        int32_t* __restrict__ hub_key,
                                                        int32_t* __restrict__ hub_chunk_base,
                                                        int32_t* __restrict__ multi_hubs,
                                                        int64_t hub_capacity) {
    __shared__ uint32_t lds[kThreads / kWave];
    const int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const HubFlags f = hub_flags(offsets, k, num_keys);
    uint32_t th, tc, tb;
    const uint32_t ih = block_inclusive_scan<kThreads>(f.hub, lds, th);
    const uint32_t ic = block_inclusive_scan<kThreads>(f.chunks, lds, tc);
    const uint32_t ib = block_inclusive_scan<kThreads>(f.multi, lds, tb);
    if (!f.hub) return;
    const int64_t stride = nblk + 1;
    const int64_t slot = static_cast<int64_t>(counts[blockIdx.x]) + ih - 1;
    if (slot < 0 || slot >= hub_capacity) return;
    hub_key[slot] = static_cast<int32_t>(k);
    hub_chunk_base[slot] = static_cast<int32_t>(counts[stride + blockIdx.x] + ic - f.chunks);
    if (f.multi) {
        const int64_t b = static_cast<int64_t>(counts[2 * stride + blockIdx.x]) + ib - 1;
        if (b >= 0 && b < hub_capacity) multi_hubs[b] = static_cast<int32_t>(slot);
    }
}

// Totals of the scanned counts and the longest segment into the status.
__global__ __launch_bounds__(kThreads) void k_hub_totals(const uint32_t* __restrict__ counts,
                                                         int64_t nblk, DevStatus* __restrict__ st) {
    const int64_t stride = nblk + 1;
    uint32_t m = 0;
    for (int64_t b = threadIdx.x; b < nblk; b += kThreads) {
        const uint32_t v = counts[3 * stride + b];
        m = v > m ? v : m;
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const uint32_t other = __shfl_xor(m, o, kWave);
        m = other > m ? other : m;
    }
    __shared__ uint32_t wmax[kThreads / kWave];
    if (lane_id() == 0) wmax[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t mm = 0;
        for (int w = 0; w < kThreads / kWave; ++w) mm = wmax[w] > mm ? wmax[w] : mm;
        st->max_degree = mm;
        st->num_hubs = counts[nblk];
        st->num_chunks = counts[stride + nblk];
        st->num_multi_hubs = counts[2 * stride + nblk];
    }
}

// Walk items are balanced by a per-key weight: 1 (the key's output row) plus
// its messages for non-hub keys (hub messages are reduced elsewhere).  With
// W the exclusive scan of the weights (W[num_keys] = total),
// item_first[j] = first key k with W[k] >= j * kItemSize, and
// item_first[num_items] = num_keys.
__global__ __launch_bounds__(kThreads) void k_item_weights(const int32_t* __restrict__ offsets,
                                                           int64_t num_keys,
                                                           uint32_t* __restrict__ w) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; k <= num_keys;
         k += stride) {
        uint32_t v = 0;
        if (k < num_keys) {
            const int64_t deg = static_cast<int64_t>(offsets[k + 1]) - offsets[k];
            v = 1u + (deg > 0 && deg <= kHubThreshold ? static_cast<uint32_t>(deg) : 0u);
        }
        w[k] = v;
    }
}

__global__ __launch_bounds__(kThreads) void k_item_first(const uint32_t* __restrict__ W,
                                                         int64_t num_keys,
                                                         int32_t* __restrict__ item_first,
                                                         int32_t* __restrict__ item_short,
                                                         int64_t num_items,
                                                         DevStatus* __restrict__ st) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; k <= num_keys;
         k += stride) {
        const int64_t o = W[k];
        const int64_t op = k == 0 ? -1 : static_cast<int64_t>(W[k - 1]);
        // items j with op < j * kItemSize <= o (weights are at most kHubThreshold + 1,
        // so a key covers at most two items)
        const int64_t j0 = op < 0 ? 0 : op / kItemSize + 1;
        // the key past the end also closes the last used item (j = total / kItemSize + 1)
        int64_t j1 = k == num_keys ? o / kItemSize + 1 : o / kItemSize;
        if (j1 > num_items) j1 = num_items;
        // W[k] counts one per key before k plus their short messages
        const int32_t so = static_cast<int32_t>(o - k);
        for (int64_t j = j0; j <= j1; ++j) {
            item_first[j] = static_cast<int32_t>(k);
            item_short[j] = so;
        }
        if (k == num_keys) st->total_weight = static_cast<unsigned long long>(o);
    }
}

// short_off[k] = W[k] - k; the gathered rows of each non-hub segment are
// copied to short_gather[short_off[k] ...], so the short segments lie back to
// back in key order.
__global__ __launch_bounds__(kThreads) void k_short_index(const int32_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ gs,
                                                          const uint32_t* __restrict__ W,
                                                          int64_t num_keys,
                                                          int32_t* __restrict__ short_off,
                                                          int32_t* __restrict__ short_gather) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; k <= num_keys;
         k += stride) {
        const int64_t so = static_cast<int64_t>(W[k]) - k;
        short_off[k] = static_cast<int32_t>(so);
        if (k == num_keys) continue;
        const int64_t b = offsets[k];
        const int64_t deg = static_cast<int64_t>(offsets[k + 1]) - b;
        if (deg <= 0 || deg > kHubThreshold) continue;
        int64_t j = 0;
        for (; j + 4 <= deg; j += 4) {
            const int32_t a0 = gs[b + j], a1 = gs[b + j + 1], a2 = gs[b + j + 2], a3 = gs[b + j + 3];
            short_gather[so + j] = a0;
            short_gather[so + j + 1] = a1;
            short_gather[so + j + 2] = a2;
            short_gather[so + j + 3] = a3;
        }
        for (; j < deg; ++j) short_gather[so + j] = gs[b + j];
    }
}

// chunk_hub[hub_chunk_base[h] + j] = h for the chunks of hub h (one block per hub).
__global__ __launch_bounds__(kThreads) void k_chunk_map(const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ hub_key,
                                                        const int32_t* __restrict__ hub_chunk_base,
                                                        int64_t num_hubs, int64_t num_chunks,
                                                        int32_t* __restrict__ chunk_hub) {
    for (int64_t h = blockIdx.x; h < num_hubs; h += gridDim.x) {
        const int64_t k = hub_key[h];
        const int64_t deg = static_cast<int64_t>(offsets[k + 1]) - offsets[k];
        const int64_t nch = (deg + kChunkSize - 1) / kChunkSize;
        const int64_t base = hub_chunk_base[h];
        for (int64_t j = threadIdx.x; j < nch; j += blockDim.x) {
            if (base + j >= 0 && base + j < num_chunks) chunk_hub[base + j] = static_cast<int32_t>(h);
        }
    }
}

}  // namespace

hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_1d(n, kThreads * 4)), dim3(kThreads), 0, s, p, n,
                       value);
    return hipGetLastError();
}

hipError_t launch_status_init(DevStatus* st, hipStream_t s) {
    hipLaunchKernelGGL(k_status_init, dim3(1), dim3(64), 0, s, st);
    return hipGetLastError();
}

hipError_t launch_inv_build(const int64_t* keys, int64_t key_bound, const int64_t* gathers,
                            int64_t gather_bound, int64_t n, int32_t* inv, DevStatus* st,
                            hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_inv_build, dim3(grid_1d(n, kThreads * 4)), dim3(kThreads), 0, s, keys,
                       key_bound, gathers, gather_bound, n, inv, st);
    return hipGetLastError();
}

size_t scan_tmp_words(int64_t n) {
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    if (tiles <= 1) return 0;
    return align_up(static_cast<size_t>(tiles), 64) + scan_tmp_words(tiles);
}

hipError_t launch_exclusive_scan_u32(uint32_t* data, int64_t n, uint32_t* tmp, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    if (tiles == 1) {
        hipLaunchKernelGGL(k_scan_tile_apply, dim3(1), dim3(kScanThreads), 0, s, data, n,
                           static_cast<const uint32_t*>(nullptr));
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_scan_tile_sums, dim3(static_cast<unsigned>(tiles)), dim3(kScanThreads), 0,
                       s, data, n, tmp);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    err = launch_exclusive_scan_u32(tmp, tiles, tmp + align_up(static_cast<size_t>(tiles), 64), s);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_scan_tile_apply, dim3(static_cast<unsigned>(tiles)), dim3(kScanThreads), 0,
                       s, data, n, static_cast<const uint32_t*>(tmp));
    return hipGetLastError();
}

int64_t sort_tiles(int64_t n) { return std::max<int64_t>(1, (n + kSortTile - 1) / kSortTile); }

size_t sort_hist_words(int64_t n) {
    const int64_t nblocks = std::max<int64_t>(1, (n + kSortTile - 1) / kSortTile);
    // per-tile digit counts, then the digit totals
    return static_cast<size_t>(kSortBins) * static_cast<size_t>(nblocks + 1);
}

hipError_t sort_by_key(const int64_t* keys, int64_t key_bound, const int64_t* gathers,
                       int64_t gather_bound, int64_t n, const SortBuffers& buf,
                       uint32_t* keys_out, uint32_t* vals_out, DevStatus* st, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int bits = 0;
    while (bits < 32 && (1ll << bits) < key_bound) ++bits;
    const int passes = std::max(1, (bits + 7) / 8);
    const int64_t nblocks = (n + kSortTile - 1) / kSortTile;
    const int64_t hist_n = static_cast<int64_t>(kSortBins) * nblocks;
    uint32_t* digit_tot = buf.hist + hist_n;
    // the narrowed input goes to the b buffers; pass p writes a, b, a, ... and
    // the last pass the plan arrays
    const uint32_t* in_k = buf.keys_b;
    const uint32_t* in_v = buf.vals_b;
    int shift = 0;
    for (int p = 0; p < passes; ++p) {
        const int width = bits / passes + (p < bits % passes ? 1 : 0);
        const bool last = p == passes - 1;
        uint32_t* out_k = last ? keys_out : (p % 2 == 0 ? buf.keys_a : buf.keys_b);
        uint32_t* out_v = last ? vals_out : (p % 2 == 0 ? buf.vals_a : buf.vals_b);
        if (p == 0) {
            hipLaunchKernelGGL(k_radix_narrow, dim3(static_cast<unsigned>(nblocks)), dim3(kSortThreads),
                               0, s, keys, gathers, n, shift, width, key_bound, gather_bound,
                               buf.keys_b, buf.vals_b, buf.tile_plain, buf.hist, nblocks, st);
        } else {
            hipLaunchKernelGGL(k_radix_upsweep, dim3(static_cast<unsigned>(nblocks)), dim3(kSortThreads),
                               0, s, in_k, n, shift, width, buf.hist, nblocks);
        }
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        hipLaunchKernelGGL(k_scan_rows, dim3(kSortBins), dim3(kScanThreads), 0, s, buf.hist, nblocks,
                           digit_tot);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
        hipLaunchKernelGGL(k_radix_downsweep, dim3(static_cast<unsigned>(nblocks)), dim3(kSortThreads),
                           0, s, in_k, in_v,
                           p == 0 ? static_cast<const uint32_t*>(buf.tile_plain) : nullptr, n, shift,
                           width, static_cast<const uint32_t*>(buf.hist),
                           static_cast<const uint32_t*>(digit_tot), nblocks, out_k, out_v);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
        in_k = out_k;
        in_v = out_v;
        shift += width;
    }
    return hipSuccess;
}

hipError_t launch_offsets_from_sorted(const uint32_t* keys_sorted, int64_t n, int64_t num_keys,
                                      int32_t* offsets, hipStream_t s) {
    hipLaunchKernelGGL(k_offsets_from_sorted, dim3(grid_1d(n / 4 + 1, kThreads)), dim3(kThreads), 0,
                       s, keys_sorted, n, num_keys, offsets);
    return hipGetLastError();
}

size_t hub_list_words(int64_t num_keys) {
    const int64_t nblk = std::max<int64_t>(1, (num_keys + kThreads - 1) / kThreads);
    return static_cast<size_t>(4 * (nblk + 1));
}

hipError_t launch_hub_list(const int32_t* offsets, int64_t num_keys, int32_t* hub_key,
                           int32_t* hub_chunk_base, int32_t* multi_hubs, int64_t hub_capacity,
                           uint32_t* counts, uint32_t* scan_tmp, DevStatus* st, hipStream_t s) {
    if (num_keys <= 0) return hipSuccess;
    const int64_t nblk = (num_keys + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(k_hub_count, dim3(static_cast<unsigned>(nblk)), dim3(kThreads), 0, s, offsets,
                       num_keys, nblk, counts);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    // the three count arrays are consecutive rows of nblk + 1 values
    hipLaunchKernelGGL(k_scan_rows, dim3(3), dim3(kScanThreads), 0, s, counts, nblk + 1, scan_tmp);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_hub_write, dim3(static_cast<unsigned>(nblk)), dim3(kThreads), 0, s, offsets,
                       num_keys, nblk, static_cast<const uint32_t*>(counts), hub_key, hub_chunk_base,
                       multi_hubs, hub_capacity);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_hub_totals, dim3(1), dim3(kThreads), 0, s, static_cast<const uint32_t*>(counts),
                       nblk, st);
    return hipGetLastError();
}

int64_t item_capacity_for(int64_t num_keys) {
    return num_keys * (kHubThreshold + 1) / kItemSize + 1;
}

hipError_t launch_item_first(const int32_t* offsets, const int32_t* gather_sorted,
                             int64_t num_keys, uint32_t* weights, uint32_t* scan_tmp,
                             int32_t* item_first, int32_t* item_short, int64_t item_capacity,
                             int32_t* short_off, int32_t* short_gather, DevStatus* st,
                             hipStream_t s) {
    hipLaunchKernelGGL(k_item_weights, dim3(grid_1d(num_keys + 1, kThreads * 4)), dim3(kThreads), 0,
                       s, offsets, num_keys, weights);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    err = launch_exclusive_scan_u32(weights, num_keys + 1, scan_tmp, s);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_item_first, dim3(grid_1d(num_keys + 1, kThreads)), dim3(kThreads), 0, s,
                       static_cast<const uint32_t*>(weights), num_keys, item_first, item_short,
                       item_capacity, st);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_short_index, dim3(grid_1d(num_keys + 1, kThreads)), dim3(kThreads), 0, s,
                       offsets, gather_sorted, static_cast<const uint32_t*>(weights), num_keys,
                       short_off, short_gather);
    return hipGetLastError();
}

hipError_t launch_chunk_map(const int32_t* offsets, const int32_t* hub_key,
                            const int32_t* hub_chunk_base, int64_t num_hubs, int64_t num_chunks,
                            int32_t* chunk_hub, hipStream_t s) {
    if (num_hubs <= 0) return hipSuccess;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(num_hubs, 1 << 16));
    hipLaunchKernelGGL(k_chunk_map, dim3(blocks), dim3(kThreads), 0, s, offsets, hub_key,
                       hub_chunk_base, num_hubs, num_chunks, chunk_hub);
    return hipGetLastError();
}

}  // namespace relm_mp
