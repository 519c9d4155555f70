// Index-plan kernels: validation, inverse maps, device scan, stable LSD radix
// sort by key, CSR offsets and hub lists.  All of these are integer work: the
// bound is HBM traffic over the index arrays.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <type_traits>

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

// Resets the status and zeroes `nclear` words (counters that later kernels
// add to with atomics), grid-stride as 16-byte stores where aligned.
__device__ __forceinline__ void clear_words(uint32_t* __restrict__ clear, int64_t nclear) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if ((reinterpret_cast<uintptr_t>(clear) & 15u) == 0) {
        const int64_t n4 = nclear / 4;
        for (int64_t i = tid; i < n4; i += stride) reinterpret_cast<uint4*>(clear)[i] = uint4{0u, 0u, 0u, 0u};
        for (int64_t i = 4 * n4 + tid; i < nclear; i += stride) clear[i] = 0u;
    } else {
        for (int64_t i = tid; i < nclear; i += stride) clear[i] = 0u;
    }
}

__global__ void k_status_init(DevStatus* st, uint32_t* __restrict__ clear, int64_t nclear,
                              uint32_t* __restrict__ clear2, int64_t nclear2) {
    clear_words(clear, nclear);
    clear_words(clear2, nclear2);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
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

// Copies the status to host memory mapped for the device (vector stores),
// then stores `gen` behind it with a system-scope release: the host polls
// *host_gen and reads the status once it equals gen.  Run by one workgroup
// of a kernel that starts after every update of the status (a kernel
// boundary behind them).
__device__ __forceinline__ void publish_status(const DevStatus* __restrict__ st,
                                               DevStatus* __restrict__ host,
                                               relm_mp_plan_counts* __restrict__ pc,
                                               int32_t* __restrict__ host_gen, int32_t gen) {
    constexpr int kWords = static_cast<int>(sizeof(DevStatus) / sizeof(unsigned long long));
    const int i = static_cast<int>(threadIdx.x);
    if (i < kWords)
        reinterpret_cast<unsigned long long*>(host)[i] = reinterpret_cast<const unsigned long long*>(st)[i];
    if (pc != nullptr && i == 0) {
        pc->collisions = static_cast<int64_t>(st->collisions);
        pc->identity = st->key_mismatch == 0 ? 1 : 0;
    }
    __threadfence_system();
    __syncthreads();
    if (i == 0 && host_gen != nullptr)
        __hip_atomic_store(host_gen, gen, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void k_status_publish(const DevStatus* __restrict__ st, DevStatus* __restrict__ host,
                                 relm_mp_plan_counts* __restrict__ pc, int32_t* __restrict__ host_gen,
                                 int32_t gen) {
    publish_status(st, host, pc, host_gen, gen);
}

// inv[k] = max e with keys[e] == k.  Every key and gathered index is checked;
// the smallest offending edge of each array is recorded.  Workgroups take
// tiles of kSnapTile edges (grid-stride); with a snapshot, a tile's narrowed
// indices are stored unless they are the tile's own edge ids, which the
// tile's plain flag records instead.
__global__ __launch_bounds__(kThreads) void k_inv_build(const int64_t* __restrict__ keys,
                                                        int64_t key_bound,
                                                        const int64_t* __restrict__ gathers,
                                                        int64_t gather_bound, int64_t n,
                                                        int32_t* __restrict__ inv, SnapOut snap,
                                                        DevStatus* __restrict__ st) {
    constexpr int kItems = kSnapTile / kThreads;
    const int64_t tiles = (n + kSnapTile - 1) / kSnapTile;
    const bool snapshot = snap.keys != nullptr || snap.gathers != nullptr;
    unsigned long long collisions = 0, bad_k = kNoEdge, bad_g = kNoEdge;
    int key_mismatch = 0;
    for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
        const int64_t base = t * kSnapTile + threadIdx.x;
        uint32_t k32[kItems], g32[kItems];
        int kmis = 0, gmis = 0;
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int64_t p = base + static_cast<int64_t>(i) * kThreads;
            bool coll = false;
            k32[i] = g32[i] = 0;
            if (p < n) {
                const int64_t k = keys[p];
                kmis |= k != p ? 1 : 0;
                if (static_cast<uint64_t>(k) < static_cast<uint64_t>(key_bound)) {
                    k32[i] = static_cast<uint32_t>(k);
                    coll = atomicMax(inv + k, static_cast<int32_t>(p)) >= 0;
                } else {
                    bad_k = min(bad_k, static_cast<unsigned long long>(p));
                }
                if (gathers != nullptr) {
                    const int64_t g = gathers[p];
                    gmis |= g != p ? 1 : 0;
                    if (static_cast<uint64_t>(g) < static_cast<uint64_t>(gather_bound))
                        g32[i] = static_cast<uint32_t>(g);
                    else
                        bad_g = min(bad_g, static_cast<unsigned long long>(p));
                }
            }
            collisions += __popcll(__ballot(coll));
        }
        key_mismatch |= kmis;
        if (snapshot) {
            const int any_k = __syncthreads_or(kmis);
            const int any_g = __syncthreads_or(gmis);
#pragma unroll
            for (int i = 0; i < kItems; ++i) {
                const int64_t p = base + static_cast<int64_t>(i) * kThreads;
                if (p >= n) continue;
                if (snap.keys != nullptr && any_k) snap.keys[p] = k32[i];
                if (snap.gathers != nullptr && any_g) snap.gathers[p] = g32[i];
            }
            if (threadIdx.x == 0) {
                if (snap.key_plain != nullptr) snap.key_plain[t] = any_k ? 0u : 1u;
                if (snap.gather_plain != nullptr) snap.gather_plain[t] = any_g ? 0u : 1u;
            }
        }
    }
    if (bad_k != kNoEdge) atomicMin(&st->bad_key_edge, bad_k);
    if (bad_g != kNoEdge) atomicMin(&st->bad_gather_edge, bad_g);
    if (lane_id() == 0 && collisions != 0) atomicAdd(&st->collisions, collisions);
    // a flag that only ever becomes 1: a plain store from one thread per
    // workgroup (atomics on one word from thousands of workgroups serialise)
    if (__syncthreads_or(key_mismatch) && threadIdx.x == 0) st->key_mismatch = 1ull;
}

// Inverse map of a CSR plan's gathered indices, from the plan's int32
// snapshot of them (tiles flagged plain hold the edge ids): inv[g(e)] = e with
// plain stores.  The snapshot was validated by the plan's build; an index at
// or past key_bound is skipped here and counted by k_inv_verify.  With
// repeated indices one writer wins per row; k_inv_verify finds the others.
__device__ __forceinline__ int64_t snap_index(const int32_t* __restrict__ snap,
                                              const uint32_t* __restrict__ plain, int64_t e) {
    return plain != nullptr && plain[e / kSnapTile] != 0u ? e : static_cast<int64_t>(snap[e]);
}

__global__ __launch_bounds__(kThreads) void k_inv_scatter(const int32_t* __restrict__ snap,
                                                          const uint32_t* __restrict__ plain,
                                                          int64_t n, int64_t key_bound,
                                                          int32_t* __restrict__ inv) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
        const int64_t r = snap_index(snap, plain, e);
        if (static_cast<uint64_t>(r) < static_cast<uint64_t>(key_bound)) inv[r] = static_cast<int32_t>(e);
    }
}

// Counts the edges e with inv[g(e)] != e (g(e) read by another edge too, or
// out of range) into st->collisions, and flags g(e) != e in st->key_mismatch.
__global__ __launch_bounds__(kThreads) void k_inv_verify(const int32_t* __restrict__ snap,
                                                         const uint32_t* __restrict__ plain,
                                                         int64_t n, int64_t key_bound,
                                                         const int32_t* __restrict__ inv,
                                                         DevStatus* __restrict__ st) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    unsigned long long lost = 0;
    int mismatch = 0;
    for (int64_t e0 = static_cast<int64_t>(blockIdx.x) * blockDim.x; e0 < n; e0 += stride) {
        const int64_t e = e0 + threadIdx.x;
        bool bad = false;
        if (e < n) {
            const int64_t r = snap_index(snap, plain, e);
            const bool in = static_cast<uint64_t>(r) < static_cast<uint64_t>(key_bound);
            bad = !in || inv[in ? r : 0] != static_cast<int32_t>(e);
            mismatch |= r != e ? 1 : 0;
        }
        lost += __popcll(__ballot(bad));
    }
    // one atomic per workgroup that lost edges; the mismatch flag (only ever 1)
    // as a plain store - atomics on one word from thousands of workgroups
    // serialise
    __shared__ unsigned long long s_lost;
    if (threadIdx.x == 0) s_lost = 0;
    __syncthreads();
    if (lane_id() == 0 && lost != 0) atomicAdd(&s_lost, lost);
    const int any_mismatch = __syncthreads_or(mismatch);
    if (threadIdx.x == 0) {
        if (s_lost != 0) atomicAdd(&st->collisions, s_lost);
        if (any_mismatch) st->key_mismatch = 1ull;
    }
}

// ---- scan ----------------------------------------------------------------

// Exclusive scan of every row of a [gridDim.x, len] array in place (one
// workgroup per row, kScanTile values per step with a running carry);
// tot[row] receives the row's sum.
// Thread t's kScanItems consecutive values lie kScanItems + 1 words apart in
// LDS (padded rows: no two threads of a wave in one bank).
constexpr int kScanPad = kScanItems + 1;

__global__ __launch_bounds__(kScanThreads) void k_scan_rows(uint32_t* __restrict__ data,
                                                            int64_t len,
                                                            uint32_t* __restrict__ tot) {
    __shared__ uint32_t tile[kScanThreads * kScanPad];
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
        for (int i = 0; i < kScanItems; ++i) {
            const int e = i * kScanThreads + static_cast<int>(threadIdx.x);  // element of the tile
            tile[(e / kScanItems) * kScanPad + e % kScanItems] = in[i];
        }
        __syncthreads();
        uint32_t v[kScanItems];
        uint32_t sum = 0;
#pragma unroll
        for (int i = 0; i < kScanItems; ++i) {
            v[i] = tile[threadIdx.x * kScanPad + i];
            sum += v[i];
        }
        uint32_t total;
        const uint32_t incl = block_inclusive_scan<kScanThreads>(sum, lds, total);
        uint32_t run = incl - sum + carry;
#pragma unroll
        for (int i = 0; i < kScanItems; ++i) {
            tile[threadIdx.x * kScanPad + i] = run;
            run += v[i];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kScanItems; ++i) {
            const int64_t p = base + static_cast<int64_t>(i) * kScanThreads + threadIdx.x;
            const int e = i * kScanThreads + static_cast<int>(threadIdx.x);
            if (p < len) row[p] = tile[(e / kScanItems) * kScanPad + e % kScanItems];
        }
        carry += total;
        __syncthreads();  // tile is rewritten by the next step
    }
    if (threadIdx.x == 0) tot[blockIdx.x] = carry;
}

// Exclusive scan over tiles of tile-major digit counts: hist[t * kSortBins + d]
// becomes the number of keys with digit d in the tiles before t; tot[d] the
// count over all tiles.  Workgroup (g, c) covers digits [32g, 32g + 32) of the
// tile chunk [c * kColChunk, (c + 1) * kColChunk): for each tile those counts
// are one 128-byte line, so every load is a full line (digit-major counts
// written by concurrent tiles on different XCDs would be partial lines).
// Thread t handles digit 32g + t % 32 over kColItems consecutive tiles.  The
// chunk sums come from the counting kernels (atomics into chunk_sum); each
// chunk adds the sums of the chunks before it.
constexpr int kColDigits = 32;
constexpr int kColItems = 16;
constexpr int kColLanes = kScanThreads / kColDigits;  // tile lanes per digit
constexpr int kColChunk = kColLanes * kColItems;      // tiles per workgroup

__global__ __launch_bounds__(kScanThreads) void k_scan_cols(uint32_t* __restrict__ hist,
                                                            int64_t ntiles,
                                                            const uint32_t* __restrict__ chunk_sum,
                                                            uint32_t* __restrict__ tot,
                                                            StatusPublish pub) {
    __shared__ uint32_t part[kColLanes][kColDigits];
    __shared__ uint32_t prior[kColLanes][kColDigits];
    const int dl = static_cast<int>(threadIdx.x) % kColDigits;
    const int tl = static_cast<int>(threadIdx.x) / kColDigits;
    const int64_t d = static_cast<int64_t>(blockIdx.x) * kColDigits + dl;
    const int64_t c = blockIdx.y;
    const int64_t t0 = c * kColChunk + static_cast<int64_t>(tl) * kColItems;
    uint32_t v[kColItems];
#pragma unroll
    for (int i = 0; i < kColItems; ++i) v[i] = t0 + i < ntiles ? hist[(t0 + i) * kSortBins + d] : 0u;
    // the chunks before this one, split over the tile lanes
    uint32_t pri = 0;
    for (int64_t cc = tl; cc < c; cc += kColLanes) pri += chunk_sum[cc * kSortBins + d];
    uint32_t sum = 0;
#pragma unroll
    for (int i = 0; i < kColItems; ++i) sum += v[i];
    part[tl][dl] = sum;
    prior[tl][dl] = pri;
    __syncthreads();
    uint32_t before = 0;
#pragma unroll
    for (int l = 0; l < kColLanes; ++l) {
        if (l < tl) before += part[l][dl];
        before += prior[l][dl];
    }
#pragma unroll
    for (int i = 0; i < kColItems; ++i) {
        if (t0 + i < ntiles) hist[(t0 + i) * kSortBins + d] = before;
        before += v[i];
    }
    if (tl == kColLanes - 1 && c == static_cast<int64_t>(gridDim.y) - 1) tot[d] = before;
    // The first pass's scan starts behind the validating pass: one workgroup
    // publishes the validation status to the host (no kernel of its own).
    if (pub.host != nullptr && blockIdx.x == 0 && blockIdx.y == 0)
        publish_status(pub.st, pub.host, nullptr, pub.host_gen, pub.gen);
}

// ---- radix sort ----------------------------------------------------------

// The tile's count of digit threadIdx.x: its row of the tile-major counts
// and, when the tiles form more than one column chunk, the running sum of its
// chunk (chunk_sum, zeroed before the sort).
__device__ __forceinline__ void store_tile_counts(uint32_t* __restrict__ hist,
                                                  uint32_t* __restrict__ chunk_sum, uint32_t t) {
    hist[static_cast<int64_t>(blockIdx.x) * kSortBins + threadIdx.x] = t;
    if (chunk_sum != nullptr && t != 0u)
        atomicAdd(chunk_sum + static_cast<int64_t>(blockIdx.x / kColChunk) * kSortBins + threadIdx.x, t);
}

// Tile digit histogram in LDS: kSubHists copies per wave (lane & 3), so that
// lanes holding the same digit - frequent for hub keys - rarely hit the same
// address; plain LDS atomics, no cross-lane matching.  The copies lie
// kSortBins + 1 words apart, so one digit of different copies falls in
// different banks.
constexpr int kSubHists = 4;
constexpr int kHistStride = kSortBins + 1;
constexpr int kHistWords = (kSortThreads / kWave) * kSubHists * kHistStride;

__device__ __forceinline__ void hist_clear(uint32_t* h) {
    for (int i = static_cast<int>(threadIdx.x); i < kHistWords; i += kSortThreads) h[i] = 0;
}

__device__ __forceinline__ void hist_add(uint32_t* h, uint32_t d) {
    const int copy = (static_cast<int>(threadIdx.x) / kWave) * kSubHists + (lane_id() & (kSubHists - 1));
    atomicAdd(&h[copy * kHistStride + d], 1u);
}

// Sum of the copies for digit threadIdx.x (call after a barrier).
__device__ __forceinline__ uint32_t hist_total(const uint32_t* h) {
    uint32_t t = 0;
#pragma unroll
    for (int c = 0; c < (kSortThreads / kWave) * kSubHists; ++c) t += h[c * kHistStride + threadIdx.x];
    return t;
}

// First pass over the caller's int64 arrays: validates every key (and
// gathered index), narrows both to int32 for the sort passes and counts the
// tile's digits of the first pass (hist[tile * kSortBins + d]).  Gathered
// indices equal to their edge ids (or no gathers) are common; a tile made of
// those only is flagged in tile_plain instead of written, and the first
// scatter generates its values.
using i64x2 = int64_t __attribute__((ext_vector_type(2)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

// One index checked against its bound: the narrowed value (0 if bad), the
// smallest bad edge so far.
__device__ __forceinline__ uint32_t narrow_index(int64_t v, int64_t bound, int64_t p,
                                                 unsigned long long& bad) {
    const bool ok = static_cast<uint64_t>(v) < static_cast<uint64_t>(bound);
    bad = ok ? bad : min(bad, static_cast<unsigned long long>(p));
    return ok ? static_cast<uint32_t>(v) : 0u;
}

// The same check without the edge: `all_ok` clears on a bad index (whose edge
// is then found again from memory, a path only invalid input takes).
__device__ __forceinline__ uint32_t narrow_checked(int64_t v, int64_t bound, bool& all_ok) {
    const bool ok = static_cast<uint64_t>(v) < static_cast<uint64_t>(bound);
    all_ok = all_ok && ok;
    return ok ? static_cast<uint32_t>(v) : 0u;
}

__global__ __launch_bounds__(kSortThreads) void k_radix_narrow(
    const int64_t* __restrict__ keys, const int64_t* __restrict__ gathers, int64_t n, int shift,
    int bits, int64_t key_bound, int64_t gather_bound, uint32_t* __restrict__ keys32,
    uint32_t* __restrict__ vals32, uint32_t* __restrict__ tile_plain, uint32_t* __restrict__ hist,
    uint32_t* __restrict__ chunk_sum, int64_t nblocks, DevStatus* __restrict__ st) {
    __shared__ uint32_t h[kHistWords];
    hist_clear(h);
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
    const uint32_t dmask = (1u << bits) - 1u;
    unsigned long long bad_k = kNoEdge, bad_g = kNoEdge;
    uint32_t key[kSortItems], val[kSortItems];
    int mismatch = 0;
    // Full tiles of 16-byte aligned arrays: thread t owns the element pairs
    // 2 * (i * 256 + t) + {0, 1}, read as 16-byte streaming loads and written
    // as 8-byte stores.  The last, partial tile (or unaligned arrays) go
    // element by element.
    const bool full = base + kSortTile <= n &&
                      ((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(gathers)) & 15u) == 0;
    constexpr int kPairs = kSortItems / 2;
    if (full) {
        bool keys_ok = true, gathers_ok = true;
#pragma unroll
        for (int i = 0; i < kPairs; ++i) {
            const int64_t p = base + 2 * (static_cast<int64_t>(i) * kSortThreads + threadIdx.x);
            const i64x2 k2 = __builtin_nontemporal_load(reinterpret_cast<const i64x2*>(keys + p));
            key[2 * i] = narrow_checked(k2.x, key_bound, keys_ok);
            key[2 * i + 1] = narrow_checked(k2.y, key_bound, keys_ok);
            val[2 * i] = val[2 * i + 1] = 0;
        }
        if (gathers != nullptr) {
#pragma unroll
            for (int i = 0; i < kPairs; ++i) {
                const int64_t p = base + 2 * (static_cast<int64_t>(i) * kSortThreads + threadIdx.x);
                const i64x2 g2 =
                    __builtin_nontemporal_load(reinterpret_cast<const i64x2*>(gathers + p));
                val[2 * i] = narrow_checked(g2.x, gather_bound, gathers_ok);
                val[2 * i + 1] = narrow_checked(g2.y, gather_bound, gathers_ok);
                mismatch |= (g2.x != p) | (g2.y != p + 1);
            }
        }
        // a bad index: the thread's smallest bad edge, from memory
        if (!keys_ok || !gathers_ok) {
            for (int i = 0; i < kPairs; ++i) {
                const int64_t p = base + 2 * (static_cast<int64_t>(i) * kSortThreads + threadIdx.x);
                for (int j = 0; j < 2; ++j) {
                    if (!keys_ok) (void)narrow_index(keys[p + j], key_bound, p + j, bad_k);
                    if (!gathers_ok) (void)narrow_index(gathers[p + j], gather_bound, p + j, bad_g);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < kSortItems; ++i) {
            const int64_t p = base + static_cast<int64_t>(i) * kSortThreads + threadIdx.x;
            key[i] = 0;
            val[i] = 0;
            if (p < n) {
                key[i] = narrow_index(keys[p], key_bound, p, bad_k);
                if (gathers != nullptr) {
                    const int64_t g = gathers[p];
                    val[i] = narrow_index(g, gather_bound, p, bad_g);
                    mismatch |= g != p ? 1 : 0;
                }
            }
        }
    }
    // block-wide: does any gathered index differ from its edge id?  (also the
    // barrier after clearing h)
    const int any = __syncthreads_or(mismatch);
    if (full) {
#pragma unroll
        for (int i = 0; i < kPairs; ++i) {
            const int64_t p = base + 2 * (static_cast<int64_t>(i) * kSortThreads + threadIdx.x);
            *reinterpret_cast<u32x2*>(keys32 + p) = u32x2{key[2 * i], key[2 * i + 1]};
            if (any) *reinterpret_cast<u32x2*>(vals32 + p) = u32x2{val[2 * i], val[2 * i + 1]};
        }
#pragma unroll
        for (int i = 0; i < kSortItems; ++i) hist_add(h, (key[i] >> shift) & dmask);
    } else {
#pragma unroll
        for (int i = 0; i < kSortItems; ++i) {
            const int64_t p = base + static_cast<int64_t>(i) * kSortThreads + threadIdx.x;
            if (p < n) {
                keys32[p] = key[i];
                if (any) vals32[p] = val[i];
                hist_add(h, (key[i] >> shift) & dmask);
            }
        }
    }
    if (bad_k != kNoEdge) atomicMin(&st->bad_key_edge, bad_k);
    if (bad_g != kNoEdge) atomicMin(&st->bad_gather_edge, bad_g);
    if (threadIdx.x == 0) {
        tile_plain[blockIdx.x] = any ? 0u : 1u;
        if (any) st->gather_mismatch = 1ull;  // only ever 1: a plain store, no atomic
    }
    __syncthreads();
    store_tile_counts(hist, chunk_sum, hist_total(h));
}

// Per-tile digit histogram of the narrowed keys, written tile-major:
// hist[tile * kSortBins + d] (one contiguous row per tile).  Counting ignores
// the order: each lane adds its keys with LDS atomics to one of kCountCopies
// copies per wave (lane & 7; copies one word apart in banks), and a wave whose
// active lanes all hold one digit - the runs of one key that hubs form once
// the earlier passes have grouped the keys - adds their number once.
constexpr int kCountCopies = 8;

template <int BITS>
__global__ __launch_bounds__(kSortThreads) void k_radix_upsweep(const uint32_t* __restrict__ keys,
                                                                int64_t n, int shift,
                                                                uint32_t* __restrict__ hist,
                                                                uint32_t* __restrict__ chunk_sum,
                                                                int64_t nblocks) {
    constexpr int kWaves = kSortThreads / kWave;
    constexpr int kDigits = 1 << BITS;
    constexpr int kStride = kDigits + 1;
    constexpr int kWords = kWaves * kCountCopies * kStride;
    __shared__ uint32_t h[kWords];
    for (int i = static_cast<int>(threadIdx.x); i < kWords; i += kSortThreads) h[i] = 0;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kSortTile;
    constexpr uint32_t dmask = (1u << BITS) - 1u;
    // A full tile is read as 16-byte loads (thread t holds elements
    // 4 * (j * 256 + t) + {0..3}); a partial tile element by element, with the
    // elements past n inactive.
    uint32_t key[kSortItems];
    uint32_t* wh = h + (static_cast<int>(threadIdx.x) / kWave) * kCountCopies * kStride;
    uint32_t* mine = wh + (lane_id() & (kCountCopies - 1)) * kStride;
    if (base + kSortTile <= n && (reinterpret_cast<uintptr_t>(keys) & 15u) == 0) {
#pragma unroll
        for (int j = 0; j < kSortItems / 4; ++j) {
            const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                keys + base + 4 * (static_cast<int64_t>(j) * kSortThreads + threadIdx.x)));
            key[4 * j] = v.x;
            key[4 * j + 1] = v.y;
            key[4 * j + 2] = v.z;
            key[4 * j + 3] = v.w;
        }
        __syncthreads();
        // a full tile: every lane holds kSortItems keys
#pragma unroll
        for (int i = 0; i < kSortItems; ++i) {
            const uint32_t d = (key[i] >> shift) & dmask;
            const uint32_t d0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(d)));
            if (__ballot(d != d0) == 0ull) {
                if (lane_id() == 0) atomicAdd(&wh[d0], static_cast<uint32_t>(kWave));
            } else {
                atomicAdd(&mine[d], 1u);
            }
        }
    } else {
        int valid = 0;
#pragma unroll
        for (int i = 0; i < kSortItems; ++i) {
            const int64_t p = base + static_cast<int64_t>(i) * kSortThreads + threadIdx.x;
            key[i] = p < n ? keys[p] : 0u;
            valid += p < n ? 1 : 0;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kSortItems; ++i) {
            // thread t's valid elements are its first `valid`
            const bool active = i < valid;
            const uint32_t d = (key[i] >> shift) & dmask;
            const unsigned long long act = __ballot(active);
            if (act == 0ull) continue;  // uniform over the wave
            const uint32_t d0 = static_cast<uint32_t>(
                __builtin_amdgcn_readlane(static_cast<int>(d), __builtin_ctzll(act)));
            if (__ballot(active && d != d0) == 0ull) {
                if (lane_id() == 0) atomicAdd(&wh[d0], static_cast<uint32_t>(__popcll(act)));
            } else if (active) {
                atomicAdd(&mine[d], 1u);
            }
        }
    }
    __syncthreads();
    uint32_t t = 0;
    if (static_cast<int>(threadIdx.x) < kDigits) {
#pragma unroll
        for (int c = 0; c < kWaves * kCountCopies; ++c) t += h[c * kStride + threadIdx.x];
    }
    store_tile_counts(hist, chunk_sum, t);
}

// Stable scatter of one tile by kDownThreads threads (eight waves: more waves
// per CU than the 39 KB of LDS per workgroup would give four-wave workgroups).
// Wave w owns tile positions [w * kPerWave, (w + 1) * kPerWave) in rounds of
// 64, so the order (wave, round, lane) is the edge order; each key's rank is
// counted in that order, the tile is staged in LDS in digit order and written
// out in runs per digit.  In the first pass a tile flagged in tile_plain takes
// the edge ids as its values.  Threads below kSortBins also own one digit each.
//
// The last pass (LAST) writes the values and, in place of the sorted keys, the
// CSR offsets: offsets[k] = the first sorted position with key >= k.  Its input
// is sorted by the lower digits, so each digit's run within a tile is sorted by
// the whole key, and the runs follow each other in the output in (digit, tile)
// order.  An element whose key k exceeds the key p of the element before it in
// its run writes offsets[p + 1 .. k] = its position, and the last element of
// the output the offsets behind the largest key (= n).  For the first element
// of each run the predecessor lies in another tile: the pass records the run's
// first key and its last key + 1 (0: empty run; with the maximum per column
// chunk in chunk_last) for k_run_heads.  Every offset has one writer.
constexpr int kDownThreads = 512;
constexpr int kDownItems = kSortTile / kDownThreads;
static_assert(kDownThreads >= kSortBins, "one thread per digit");

template <int BITS, bool LAST>
__global__ __launch_bounds__(kDownThreads) void k_radix_downsweep(
    const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
    const uint32_t* __restrict__ tile_plain, int64_t n, int shift,
    const uint32_t* __restrict__ hist_scanned, const uint32_t* __restrict__ digit_tot,
    int64_t nblocks, uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out,
    int32_t* __restrict__ offsets, int64_t num_keys, uint32_t* __restrict__ run_first,
    uint32_t* __restrict__ run_last, uint32_t* __restrict__ chunk_last) {
    constexpr int kWaves = kDownThreads / kWave;
    constexpr int kPerWave = kSortTile / kWaves;
    constexpr int kDigits = 1 << BITS;
    // per-wave counts of this pass's digits only: at 7 bits and less the
    // tile's LDS (39 KB) leaves room for four workgroups per CU
    __shared__ uint32_t wcnt[kWaves][kDigits];
    __shared__ uint32_t dstart[kSortBins];
    __shared__ int32_t gdelta[kSortBins];  // global start of the digit minus its tile start
    __shared__ uint32_t scan_lds[kDownThreads / kWave];
    __shared__ uint32_t sk[kSortTile];
    __shared__ uint32_t sv[kSortTile];

    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int64_t tile = xcd_tile(blockIdx.x, nblocks);
    const int64_t tile_base = tile * kSortTile;
    constexpr uint32_t dmask = (1u << BITS) - 1u;
    const int dd = static_cast<int>(threadIdx.x);  // the digit of threads below kSortBins
    const bool owns_digit = dd < kSortBins;
    // this tile's start within each digit does not depend on the keys: fetch
    // it together with them
    uint32_t tile_prefix = 0, dt = 0;
    if (owns_digit) {
        tile_prefix = hist_scanned[tile * kSortBins + dd];
        dt = digit_tot[dd];
    }
    for (int i = dd; i < kWaves * kDigits; i += kDownThreads) (&wcnt[0][0])[i] = 0;
    __syncthreads();

    uint32_t key[kDownItems], val[kDownItems], rank[kDownItems];
    const bool plain = tile_plain != nullptr && tile_plain[tile] != 0u;
    const int64_t wave_base = tile_base + wave * kPerWave + lane;
    // Every tile but a partial last one is full: its loads and ranks need no
    // bounds (FULL), the last tile's go element by element.
    auto load_and_rank = [&](auto full_t) {
        constexpr bool FULL = decltype(full_t)::value;
        if constexpr (FULL) {
            const uint32_t* kp = keys + wave_base;
#pragma unroll
            for (int r = 0; r < kDownItems; ++r) key[r] = __builtin_nontemporal_load(kp + r * kWave);
            if (plain) {
#pragma unroll
                for (int r = 0; r < kDownItems; ++r) val[r] = static_cast<uint32_t>(wave_base) + r * kWave;
            } else {
                const uint32_t* vp = vals + wave_base;
#pragma unroll
                for (int r = 0; r < kDownItems; ++r) val[r] = __builtin_nontemporal_load(vp + r * kWave);
            }
        } else {
#pragma unroll
            for (int r = 0; r < kDownItems; ++r) {
                const int64_t p = wave_base + r * kWave;
                uint32_t k = 0, v = 0;
                if (p < n) {
                    k = __builtin_nontemporal_load(keys + p);
                    v = plain ? static_cast<uint32_t>(p) : __builtin_nontemporal_load(vals + p);
                }
                key[r] = k;
                val[r] = v;
            }
        }
#pragma unroll
        for (int r = 0; r < kDownItems; ++r) {
            const bool active = FULL || wave_base + r * kWave < n;
            const uint32_t d = (key[r] >> shift) & dmask;
            const unsigned long long peers = match_digit<BITS>(d, FULL ? ~0ull : __ballot(active));
            const uint32_t below = __popcll(peers & lanemask_lt());
            uint32_t before = 0;
            if (active) before = wcnt[wave][d];
            rank[r] = before + below;
            if (active && below == 0) wcnt[wave][d] = before + __popcll(peers);
        }
    };
    if (tile_base + kSortTile <= n)
        load_and_rank(std::integral_constant<bool, true>{});
    else
        load_and_rank(std::integral_constant<bool, false>{});

    __syncthreads();

    // Per digit (one thread per digit): exclusive prefix over waves, tile total.
    uint32_t run = 0;
    if (dd < kDigits) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t c = wcnt[w][dd];
            wcnt[w][dd] = run;
            run += c;
        }
    }
    uint32_t total;
    const uint32_t incl = block_inclusive_scan<kDownThreads>(run, scan_lds, total);
    // global start of digit dd: all smaller digits of every tile, then this
    // digit in the tiles before this one (this tile's row of hist_scanned)
    uint32_t all;
    const uint32_t dincl = block_inclusive_scan<kDownThreads>(dt, scan_lds, all);
    if (owns_digit) {
        dstart[dd] = incl - run;
        gdelta[dd] = static_cast<int32_t>((dincl - dt) + tile_prefix) - static_cast<int32_t>(incl - run);
    }
    __syncthreads();

    const int64_t rem = n - tile_base;
    const int count = rem < kSortTile ? static_cast<int>(rem) : kSortTile;
    if (count == kSortTile) {
        // every element is staged; the mask keeps a position in the tile
#pragma unroll
        for (int r = 0; r < kDownItems; ++r) {
            const uint32_t d = (key[r] >> shift) & dmask;
            const uint32_t pos = (dstart[d] + wcnt[wave][d] + rank[r]) & (kSortTile - 1);
            sk[pos] = key[r];
            sv[pos] = val[r];
        }
    } else {
#pragma unroll
        for (int r = 0; r < kDownItems; ++r) {
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
    }
    __syncthreads();
    if constexpr (LAST) {
        if (owns_digit) {
            const uint32_t first = dstart[dd];
            const uint32_t last1 = run > 0 ? sk[first + run - 1] + 1u : 0u;
            run_first[tile * kSortBins + dd] = run > 0 ? sk[first] : 0u;
            run_last[tile * kSortBins + dd] = last1;
            if (last1 != 0u) atomicMax(chunk_last + (tile / kColChunk) * kSortBins + dd, last1);
        }
    }
    // Element i of the staged tile goes to output position gdelta[d] + i.
    auto put = [&](int i, uint32_t k, uint32_t v, uint32_t pk, int32_t gd) {
        const uint32_t d = (k >> shift) & dmask;
        const int64_t op = static_cast<int64_t>(gd) + i;
        if (static_cast<uint64_t>(op) < static_cast<uint64_t>(n)) {
            vals_out[op] = v;
            if constexpr (!LAST) {
                keys_out[op] = k;
            } else {
                if (i > 0 && ((pk >> shift) & dmask) == d)
                    for (int64_t kk = static_cast<int64_t>(pk) + 1; kk <= static_cast<int64_t>(k); ++kk)
                        offsets[kk] = static_cast<int32_t>(op);
                if (op == n - 1)
                    for (int64_t kk = static_cast<int64_t>(k) + 1; kk <= num_keys; ++kk)
                        offsets[kk] = static_cast<int32_t>(n);
            }
        }
    };
    if (count == kSortTile) {
        // a full tile: every LDS read of the thread's elements is issued
        // before the first is used
        uint32_t ks[kDownItems], vs[kDownItems], ps[kDownItems];
        int32_t gd[kDownItems];
#pragma unroll
        for (int r = 0; r < kDownItems; ++r) {
            const int i = static_cast<int>(threadIdx.x) + r * kDownThreads;
            ks[r] = sk[i];
            vs[r] = sv[i];
            ps[r] = LAST && i > 0 ? sk[i - 1] : 0u;
        }
#pragma unroll
        for (int r = 0; r < kDownItems; ++r) gd[r] = gdelta[(ks[r] >> shift) & dmask];
#pragma unroll
        for (int r = 0; r < kDownItems; ++r)
            put(static_cast<int>(threadIdx.x) + r * kDownThreads, ks[r], vs[r], ps[r], gd[r]);
    } else {
        for (int i = static_cast<int>(threadIdx.x); i < count; i += kDownThreads) {
            const uint32_t k = sk[i];
            put(i, k, sv[i], LAST && i > 0 ? sk[i - 1] : 0u, gdelta[(k >> shift) & dmask]);
        }
    }
}

// The offsets of the runs' first elements in the last pass (see
// k_radix_downsweep): the key before the first element of run (tile t, digit
// d) in the output is the largest key of the runs before it in (digit, tile)
// order, so offsets[that key + 1 .. first key] = the run's output position.
// Workgroup (g, c) walks digits [32g, 32g + 32) over the tile chunk c like
// k_scan_cols, with the prefix maximum of the runs' last keys (+1) over the
// tiles, the chunk maxima of the chunks before c, and the maximum over the
// smaller digits; hist / digit_tot are the last pass's scanned counts.
__global__ __launch_bounds__(kScanThreads) void k_run_heads(
    const uint32_t* __restrict__ hist_scanned, const uint32_t* __restrict__ digit_tot,
    const uint32_t* __restrict__ run_first, const uint32_t* __restrict__ run_last,
    const uint32_t* __restrict__ chunk_last, int64_t ntiles, int64_t nchunks,
    int32_t* __restrict__ offsets) {
    static_assert(kScanThreads == kSortBins, "one thread per digit");
    __shared__ uint32_t dlow[kSortBins];   // largest key + 1 of the smaller digits
    __shared__ uint32_t dbase[kSortBins];  // first output position of each digit
    __shared__ uint32_t part[kColLanes][kColDigits];
    __shared__ uint32_t prior[kColLanes][kColDigits];
    __shared__ uint32_t scan_lds[kScanThreads / kWave];
    const int td = static_cast<int>(threadIdx.x);
    const int dl = td % kColDigits;
    const int tl = td / kColDigits;
    const int64_t d = static_cast<int64_t>(blockIdx.x) * kColDigits + dl;
    const int64_t c = blockIdx.y;
    const int64_t t0 = c * kColChunk + static_cast<int64_t>(tl) * kColItems;
    // this thread's column of runs: loaded before the scans below
    uint32_t v[kColItems], first[kColItems], pre[kColItems];
#pragma unroll
    for (int i = 0; i < kColItems; ++i) {
        const bool in = t0 + i < ntiles;
        const int64_t t = in ? t0 + i : 0;
        v[i] = in ? run_last[t * kSortBins + d] : 0u;
        first[i] = run_first[t * kSortBins + d];
        pre[i] = hist_scanned[t * kSortBins + d];
    }
    // every load of a group issued before the first is used
    uint32_t cm = 0;
    for (int64_t c0 = 0; c0 < nchunks; c0 += 16) {
        uint32_t m[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) m[j] = c0 + j < nchunks ? chunk_last[(c0 + j) * kSortBins + td] : 0u;
#pragma unroll
        for (int j = 0; j < 16; ++j) cm = max(cm, m[j]);
    }
    const uint32_t tot_d = digit_tot[td];
    const uint32_t below = block_exclusive_max<kScanThreads>(cm, scan_lds);
    uint32_t all;
    const uint32_t dincl = block_inclusive_scan<kScanThreads>(tot_d, scan_lds, all);
    dlow[td] = below;
    dbase[td] = dincl - tot_d;

    uint32_t lm = 0, pm = 0;
#pragma unroll
    for (int i = 0; i < kColItems; ++i) lm = max(lm, v[i]);
    for (int64_t cc = tl; cc < c; cc += kColLanes) pm = max(pm, chunk_last[cc * kSortBins + d]);
    part[tl][dl] = lm;
    prior[tl][dl] = pm;
    __syncthreads();
    uint32_t lo = dlow[d];
#pragma unroll
    for (int l = 0; l < kColLanes; ++l) {
        if (l < tl) lo = max(lo, part[l][dl]);
        lo = max(lo, prior[l][dl]);
    }
    const uint32_t base = dbase[d];
#pragma unroll
    for (int i = 0; i < kColItems; ++i) {
        if (v[i] != 0u) {
            const int32_t pos = static_cast<int32_t>(base + pre[i]);
            for (int64_t kk = lo; kk <= static_cast<int64_t>(first[i]); ++kk) offsets[kk] = pos;
            lo = max(lo, v[i]);
        }
    }
}

// Per-key index of a CSR plan in two passes over the keys k = 0..num_keys,
// without global atomics beyond one maximum per workgroup:
//  * k_key_stats: per workgroup of kThreads keys the number of hubs (segments
//    longer than kHubThreshold), their chunks, the hubs of more than one chunk
//    and the hub messages;
//  * these four rows are scanned (k_scan_rows);
//  * k_key_write: every hub gets its slot in key order, its chunk range and the
//    chunk -> hub map; with S[k] = short messages before key k (= offsets[k]
//    minus the hub messages before k) and the walk weight W[k] = k + S[k], the
//    walk items, short_off = S and the short-segment gather copy.
struct KeyFlags {
    uint32_t hub;
    uint32_t chunks;
    uint32_t multi;
    uint32_t hub_edges;
    int64_t deg;
};

__device__ __forceinline__ KeyFlags key_flags(const int32_t* __restrict__ offsets, int64_t k,
                                              int64_t num_keys) {
    KeyFlags f{0u, 0u, 0u, 0u, 0};
    if (k < num_keys) f.deg = static_cast<int64_t>(offsets[k + 1]) - offsets[k];
    if (f.deg > kHubThreshold) {
        f.hub = 1u;
        f.chunks = static_cast<uint32_t>((f.deg + kChunkSize - 1) / kChunkSize);
        f.multi = f.chunks > 1u ? 1u : 0u;
        f.hub_edges = static_cast<uint32_t>(f.deg);
    }
    return f;
}

constexpr int kKeyRows = 4;  // scanned rows: hubs, chunks, multi-chunk hubs, hub messages;
                             // a fifth row holds each workgroup's longest segment

__global__ __launch_bounds__(kThreads) void k_key_stats(const int32_t* __restrict__ offsets,
                                                        int64_t num_keys, int64_t nblk,
                                                        uint32_t* __restrict__ counts,
                                                        DevStatus* __restrict__ st) {
    __shared__ uint32_t lds[kThreads / kWave];
    const int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const KeyFlags f = key_flags(offsets, k, num_keys);
    // hubs and multi-chunk hubs (at most kThreads each) in one scan
    uint32_t thm, tc, te;
    block_inclusive_scan<kThreads>(f.hub | f.multi << 16, lds, thm);
    block_inclusive_scan<kThreads>(f.chunks, lds, tc);
    block_inclusive_scan<kThreads>(f.hub_edges, lds, te);
    const uint32_t th = thm & 0xFFFFu, tm = thm >> 16;
    __shared__ uint32_t wmax[kThreads / kWave];
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
        counts[2 * stride + blockIdx.x] = tm;
        counts[3 * stride + blockIdx.x] = te;
        counts[4 * stride + blockIdx.x] = mm;
        if (blockIdx.x == 0) {
            for (int r = 0; r < kKeyRows; ++r) counts[r * stride + nblk] = 0;
        }
    }
    (void)st;
}

__global__ __launch_bounds__(kThreads) void k_key_write(
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ gs, int64_t num_keys,
    int64_t nblk, const uint32_t* __restrict__ counts, const uint32_t* __restrict__ totals,
    int32_t* __restrict__ hub_key, int32_t* __restrict__ hub_chunk_base,
    int32_t* __restrict__ multi_hubs, int32_t* __restrict__ chunk_hub, int64_t hub_capacity,
    int64_t chunk_capacity, int32_t* __restrict__ item_first, int32_t* __restrict__ item_short,
    int64_t item_capacity, int32_t* __restrict__ short_off, int32_t* __restrict__ short_gather,
    relm_mp_plan_counts* __restrict__ pc, DevStatus* __restrict__ st) {
    __shared__ uint32_t lds[kThreads / kWave];
    __shared__ int32_t blk_slot[kThreads];
    __shared__ int64_t blk_cbase[kThreads];
    __shared__ uint32_t blk_chunks[kThreads];
    const int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t stride = nblk + 1;
    // the workgroup's prefixes of the scanned rows and the totals do not
    // depend on this kernel's work: loaded with the offsets
    const int64_t pre_hub = counts[blockIdx.x];
    const int64_t pre_chunk = counts[stride + blockIdx.x];
    const int64_t pre_multi = counts[2 * stride + blockIdx.x];
    const int64_t pre_edges = counts[3 * stride + blockIdx.x];
    const uint32_t total_hubs = totals[0];
    const KeyFlags f = key_flags(offsets, k, num_keys);
    // hubs and multi-chunk hubs (at most kThreads each) in one scan
    uint32_t thm, tc, te;
    const uint32_t ihm = block_inclusive_scan<kThreads>(f.hub | f.multi << 16, lds, thm);
    const uint32_t ic = block_inclusive_scan<kThreads>(f.chunks, lds, tc);
    const uint32_t ie = block_inclusive_scan<kThreads>(f.hub_edges, lds, te);
    const uint32_t ih = ihm & 0xFFFFu, im = ihm >> 16, th = thm & 0xFFFFu;
    if (blockIdx.x == 0) {
        // totals (within the capacities the plan arrays were sized for) and
        // the longest segment into the plan's counts and the status
        uint32_t m = 0;
        for (int64_t b = threadIdx.x; b < nblk; b += kThreads) {
            const uint32_t v = counts[4 * stride + b];
            m = v > m ? v : m;
        }
#pragma unroll
        for (int o = kWave / 2; o > 0; o >>= 1) {
            const uint32_t other = __shfl_xor(m, o, kWave);
            m = other > m ? other : m;
        }
        if (lane_id() == 0) lds[threadIdx.x / kWave] = m;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < kThreads / kWave; ++w) m = lds[w] > m ? lds[w] : m;
            const int64_t hubs = min(static_cast<int64_t>(totals[0]), hub_capacity);
            const int64_t chunks = min(static_cast<int64_t>(totals[1]), chunk_capacity);
            const int64_t multi = min(static_cast<int64_t>(totals[2]), hubs);
            pc->max_degree = m;
            pc->num_hubs = hubs;
            pc->num_chunks = chunks;
            pc->num_multi_hubs = multi;
            st->max_degree = m;
            st->num_hubs = totals[0];
            st->num_chunks = totals[1];
            st->num_multi_hubs = totals[2];
        }
    }
    // hub slot, chunk range; the workgroup fills the chunk -> hub map of its
    // hubs together (a hub can have hundreds of chunks)
    if (f.hub) {
        const int64_t slot = pre_hub + ih - 1;
        const int64_t cbase = pre_chunk + ic - f.chunks;
        blk_slot[ih - 1] = static_cast<int32_t>(slot);
        blk_cbase[ih - 1] = cbase;
        blk_chunks[ih - 1] = f.chunks;
        if (slot >= 0 && slot < hub_capacity) {
            hub_key[slot] = static_cast<int32_t>(k);
            hub_chunk_base[slot] = static_cast<int32_t>(cbase);
            if (f.multi) {
                const int64_t mslot = pre_multi + im - 1;
                if (mslot >= 0 && mslot < hub_capacity) multi_hubs[mslot] = static_cast<int32_t>(slot);
            }
        }
    }
    __syncthreads();
    for (uint32_t h = 0; h < th; ++h) {
        const int64_t slot = blk_slot[h];
        if (slot < 0 || slot >= hub_capacity) continue;
        for (int64_t c = threadIdx.x; c < blk_chunks[h]; c += kThreads) {
            const int64_t at = blk_cbase[h] + c;
            if (at >= 0 && at < chunk_capacity) chunk_hub[at] = static_cast<int32_t>(slot);
        }
    }
    // S[k]: short messages before k; W[k] = k + S[k]
    const bool live = k <= num_keys;
    const int64_t hub_before = pre_edges + ie - f.hub_edges;
    const int64_t S = live ? static_cast<int64_t>(offsets[k]) - hub_before : 0;
    if (live) {
        const int64_t W = k + S;
        int64_t Wprev = -1;
        if (k > 0) {
            const int64_t dprev = static_cast<int64_t>(offsets[k]) - offsets[k - 1];
            Wprev = W - 1 - (dprev > 0 && dprev <= kHubThreshold ? dprev : 0);
        }
        short_off[k] = static_cast<int32_t>(S);
        // items j with Wprev < j * kItemSize <= W; the key past the end also
        // closes the last used item (j = W / kItemSize + 1)
        const int64_t j0 = Wprev < 0 ? 0 : Wprev / kItemSize + 1;
        int64_t j1 = k == num_keys ? W / kItemSize + 1 : W / kItemSize;
        if (j1 > item_capacity) j1 = item_capacity;
        for (int64_t j = j0; j <= j1; ++j) {
            item_first[j] = static_cast<int32_t>(k);
            item_short[j] = static_cast<int32_t>(S);
        }
        if (k == num_keys) {
            st->total_weight = static_cast<unsigned long long>(W);
            pc->num_items = min(W / kItemSize + 1, item_capacity);
            pc->num_short = W - num_keys;
        }
    }
    // The short segments' gathered rows, back to back in key order (without
    // hubs that is gather_sorted itself: nothing to copy, the walker reads
    // it).  The workgroup's keys own one contiguous range of short_gather;
    // its threads copy that range position by position (coalesced), each
    // finding its key among the workgroup's segment starts in LDS.
    if (total_hubs == 0) return;  // uniform over the grid
    __shared__ int32_t seg_start[kThreads + 1];
    __shared__ int32_t seg_src[kThreads];
    const bool short_key = live && k < num_keys && f.deg > 0 && f.deg <= kHubThreshold;
    __shared__ int64_t blk_s0;  // S of the workgroup's first key (always live)
    if (threadIdx.x == 0) blk_s0 = S;
    __syncthreads();
    const int64_t base = blk_s0;
    seg_start[threadIdx.x] = static_cast<int32_t>(live ? S - base : 0);
    seg_src[threadIdx.x] = short_key ? offsets[k] : 0;
    // the end of the workgroup's range: the last live key's start plus its
    // short messages
    const int64_t last = min(static_cast<int64_t>(blockIdx.x) * kThreads + kThreads - 1, num_keys);
    if (k == last) seg_start[kThreads] = static_cast<int32_t>(S - base + (short_key ? f.deg : 0));
    __syncthreads();
    const int nlive = static_cast<int>(last - static_cast<int64_t>(blockIdx.x) * kThreads + 1);
    const int total = seg_start[kThreads];
    // Each position's key: up to kLabelCap positions labelled in LDS - every
    // key with short messages marks its first position, a block-wide running
    // maximum fills the rest; larger ranges search the segment starts.
    constexpr int kLabelItems = 16;
    constexpr int kLabelCap = kThreads * kLabelItems;
    __shared__ uint16_t lbl[kLabelCap];
    __shared__ uint32_t lbl_scan[kThreads / kWave];
    if (total <= kLabelCap) {  // uniform: total is read from LDS
        const int t0 = static_cast<int>(threadIdx.x) * kLabelItems;
#pragma unroll
        for (int i = 0; i < kLabelItems; ++i) lbl[t0 + i] = 0;
        __syncthreads();
        // keys with short messages start at distinct positions
        if (short_key) lbl[S - base] = static_cast<uint16_t>(threadIdx.x);
        __syncthreads();
        uint32_t v[kLabelItems];
        uint32_t run = 0;
#pragma unroll
        for (int i = 0; i < kLabelItems; ++i) {
            v[i] = lbl[t0 + i];
            run = max(run, v[i]);
        }
        uint32_t cur = block_exclusive_max<kThreads>(run, lbl_scan);
#pragma unroll
        for (int i = 0; i < kLabelItems; ++i) {
            cur = max(cur, v[i]);
            lbl[t0 + i] = static_cast<uint16_t>(cur);
        }
        __syncthreads();
        int32_t val[kLabelItems];
#pragma unroll
        for (int i = 0; i < kLabelItems; ++i) {
            const int j = static_cast<int>(threadIdx.x) + i * kThreads;
            if (j < total) {
                const int key = lbl[j];
                val[i] = gs[static_cast<int64_t>(seg_src[key]) + (j - seg_start[key])];
            }
        }
#pragma unroll
        for (int i = 0; i < kLabelItems; ++i) {
            const int j = static_cast<int>(threadIdx.x) + i * kThreads;
            if (j < total) short_gather[base + j] = val[i];
        }
        return;
    }
    for (int j = static_cast<int>(threadIdx.x); j < total; j += kThreads) {
        // the last key whose start is <= j (a key of no short messages shares
        // its start with the next key, so the last such key has messages)
        int lo = 0, hi = nlive;  // seg_start[lo] <= j < seg_start[hi] (hi == nlive: the end)
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (seg_start[mid] <= j) lo = mid; else hi = mid;
        }
        short_gather[base + j] = gs[static_cast<int64_t>(seg_src[lo]) + (j - seg_start[lo])];
    }
}

}  // namespace

hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_1d(n, kThreads * 4)), dim3(kThreads), 0, s, p, n,
                       value);
    return hipGetLastError();
}

hipError_t launch_status_init(DevStatus* st, hipStream_t s, uint32_t* clear, int64_t nclear,
                              uint32_t* clear2, int64_t nclear2) {
    // one workgroup per 16 KB of counters
    const unsigned blocks =
        static_cast<unsigned>(std::min<int64_t>(std::max<int64_t>(1, (nclear + nclear2) / 4096), 256));
    hipLaunchKernelGGL(k_status_init, dim3(blocks), dim3(256), 0, s, st, clear, nclear, clear2, nclear2);
    return hipGetLastError();
}

hipError_t launch_status_publish(const DevStatus* st, DevStatus* host_mapped,
                                 relm_mp_plan_counts* pc, int32_t* host_gen, int32_t gen,
                                 hipStream_t s) {
    hipLaunchKernelGGL(k_status_publish, dim3(1), dim3(64), 0, s, st, host_mapped, pc, host_gen, gen);
    return hipGetLastError();
}

hipError_t launch_inv_build(const int64_t* keys, int64_t key_bound, const int64_t* gathers,
                            int64_t gather_bound, int64_t n, int32_t* inv, const SnapOut& snap,
                            DevStatus* st, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_inv_build, dim3(grid_1d(n, kSnapTile)), dim3(kThreads), 0, s, keys,
                       key_bound, gathers, gather_bound, n, inv, snap, st);
    return hipGetLastError();
}

// Layout of SortBuffers::hist, in rows of kSortBins words: the per-tile digit
// counts (nblocks), the digit totals (1), the per-chunk digit sums of every
// pass and the last pass's per-chunk maxima of its runs' last keys
// ((kSortMaxPasses + 1) * chunks, zeroed together before the sort), then the
// last pass's first and last keys of each tile's runs (nblocks each).
struct HistLayout {
    int64_t nblocks, chunks;
    int64_t tot() const { return nblocks; }
    int64_t chunk_sums(int p) const { return nblocks + 1 + p * chunks; }
    int64_t chunk_last() const { return nblocks + 1 + kSortMaxPasses * chunks; }
    int64_t run_first() const { return chunk_last() + chunks; }
    int64_t run_last() const { return run_first() + nblocks; }
    int64_t rows() const { return run_last() + nblocks; }
};

HistLayout hist_layout(int64_t n) {
    const int64_t nblocks = std::max<int64_t>(1, (n + kSortTile - 1) / kSortTile);
    return {nblocks, (nblocks + kColChunk - 1) / kColChunk};
}

SortZero sort_zero_region(const SortBuffers& buf, int64_t n) {
    const HistLayout hl = hist_layout(n);
    if (n <= 0) return {nullptr, 0};
    return {buf.hist + static_cast<int64_t>(kSortBins) * hl.chunk_sums(0),
            static_cast<int64_t>(kSortBins) * (kSortMaxPasses + 1) * hl.chunks};
}

int64_t sort_tiles(int64_t n) { return std::max<int64_t>(1, (n + kSortTile - 1) / kSortTile); }

size_t sort_hist_words(int64_t n) {
    return static_cast<size_t>(kSortBins) * static_cast<size_t>(hist_layout(n).rows());
}

namespace {

// Calls f(std::integral_constant<int, bits>) for a digit width of 0..8 bits.
template <class F>
void with_digit_bits(int bits, F&& f) {
    switch (bits) {
        case 0: f(std::integral_constant<int, 0>{}); break;
        case 1: f(std::integral_constant<int, 1>{}); break;
        case 2: f(std::integral_constant<int, 2>{}); break;
        case 3: f(std::integral_constant<int, 3>{}); break;
        case 4: f(std::integral_constant<int, 4>{}); break;
        case 5: f(std::integral_constant<int, 5>{}); break;
        case 6: f(std::integral_constant<int, 6>{}); break;
        case 7: f(std::integral_constant<int, 7>{}); break;
        default: f(std::integral_constant<int, 8>{}); break;
    }
}

// Calls f(std::integral_constant<bool, flag>{}).
template <class F>
void with_flag(bool flag, F&& f) {
    if (flag)
        f(std::integral_constant<bool, true>{});
    else
        f(std::integral_constant<bool, false>{});
}

}  // namespace

hipError_t sort_by_key(const int64_t* keys, int64_t key_bound, const int64_t* gathers,
                       int64_t gather_bound, int64_t n, const SortBuffers& buf,
                       uint32_t* keys_tmp, uint32_t* vals_out, int32_t* offsets, DevStatus* st,
                       hipStream_t s, const StatusPublish& pub) {
    if (n <= 0) return hipSuccess;
    int bits = 0;
    while (bits < 32 && (1ll << bits) < key_bound) ++bits;
    const int passes = std::max(1, (bits + 7) / 8);
    const HistLayout hl = hist_layout(n);
    const int64_t nblocks = hl.nblocks;
    uint32_t* const rows = buf.hist;
    uint32_t* digit_tot = rows + kSortBins * hl.tot();
    // per-chunk sums (zeroed by launch_status_init; a single chunk has no
    // chunks before it and needs none)
    const bool chunked = hl.chunks > 1;
    uint32_t* chunk_last = rows + kSortBins * hl.chunk_last();
    uint32_t* run_first = rows + kSortBins * hl.run_first();
    uint32_t* run_last = rows + kSortBins * hl.run_last();
    // The narrowed input goes to the n buffers (the plan's snapshot).  Counted
    // back from the last pass, which writes the plan's values and offsets, the
    // passes write keys_tmp / vals_out and the a buffers in turn (an earlier
    // pass's values in vals_out are overwritten two passes later), so the sort
    // needs one pair of scratch buffers.
    const uint32_t* in_k = buf.keys_n;
    const uint32_t* in_v = buf.vals_n;
    int shift = 0;
    for (int p = 0; p < passes; ++p) {
        const int width = bits / passes + (p < bits % passes ? 1 : 0);
        const bool last = p == passes - 1;
        const bool to_plan = (passes - 1 - p) % 2 == 0;
        uint32_t* out_k = last ? nullptr : to_plan ? keys_tmp : buf.keys_a;
        uint32_t* out_v = to_plan ? vals_out : buf.vals_a;
        const dim3 grid(static_cast<unsigned>(nblocks)), block(kSortThreads);
        uint32_t* chunk_sum = chunked ? rows + kSortBins * hl.chunk_sums(p) : nullptr;
        if (p == 0) {
            hipLaunchKernelGGL(k_radix_narrow, grid, block, 0, s, keys, gathers, n, shift, width,
                               key_bound, gather_bound, buf.keys_n, buf.vals_n, buf.tile_plain, rows,
                               chunk_sum, nblocks, st);
        } else {
            with_digit_bits(width, [&](auto bt) {
                hipLaunchKernelGGL((k_radix_upsweep<decltype(bt)::value>), grid, block, 0, s, in_k,
                                   n, shift, rows, chunk_sum, nblocks);
            });
        }
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        const dim3 cgrid(kSortBins / kColDigits, static_cast<unsigned>(hl.chunks));
        const StatusPublish none{};
        hipLaunchKernelGGL(k_scan_cols, cgrid, dim3(kScanThreads), 0, s, rows, nblocks,
                           static_cast<const uint32_t*>(chunk_sum), digit_tot, p == 0 ? pub : none);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
        const uint32_t* plain = p == 0 ? static_cast<const uint32_t*>(buf.tile_plain) : nullptr;
        with_digit_bits(width, [&](auto bt) {
            with_flag(last, [&](auto lt) {
                hipLaunchKernelGGL((k_radix_downsweep<decltype(bt)::value, decltype(lt)::value>),
                                   grid, dim3(kDownThreads), 0, s, in_k, in_v, plain, n, shift,
                                   static_cast<const uint32_t*>(rows),
                                   static_cast<const uint32_t*>(digit_tot), nblocks, out_k, out_v,
                                   offsets, key_bound, run_first, run_last, chunk_last);
            });
        });
        err = hipGetLastError();
        if (err != hipSuccess) return err;
        if (last) {
            // digit groups of kColDigits that hold digits of this pass
            const dim3 hgrid(static_cast<unsigned>(((1 << width) + kColDigits - 1) / kColDigits),
                             static_cast<unsigned>(hl.chunks));
            hipLaunchKernelGGL(k_run_heads, hgrid, dim3(kScanThreads), 0, s,
                               static_cast<const uint32_t*>(rows),
                               static_cast<const uint32_t*>(digit_tot),
                               static_cast<const uint32_t*>(run_first),
                               static_cast<const uint32_t*>(run_last),
                               static_cast<const uint32_t*>(chunk_last), nblocks, hl.chunks, offsets);
            err = hipGetLastError();
            if (err != hipSuccess) return err;
        }
        in_k = out_k;
        in_v = out_v;
        shift += width;
    }
    return hipSuccess;
}

hipError_t launch_inv_from_snapshot(const int32_t* snap, const uint32_t* plain, int64_t n,
                                    int64_t key_bound, int32_t* inv, DevStatus* st, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const dim3 grid(grid_1d(n, kThreads * 8, 1 << 16));
    hipLaunchKernelGGL(k_inv_scatter, grid, dim3(kThreads), 0, s, snap, plain, n, key_bound, inv);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_inv_verify, grid, dim3(kThreads), 0, s, snap, plain, n, key_bound,
                       static_cast<const int32_t*>(inv), st);
    return hipGetLastError();
}

size_t key_index_words(int64_t num_keys) {
    const int64_t nblk = (num_keys + 1 + kThreads - 1) / kThreads;
    return static_cast<size_t>((kKeyRows + 1) * (nblk + 1) + 64);
}

int64_t item_capacity_for(int64_t num_keys) {
    return num_keys * (kHubThreshold + 1) / kItemSize + 1;
}

hipError_t launch_key_index(const int32_t* offsets, const int32_t* gather_sorted, int64_t num_keys,
                            uint32_t* scratch, int32_t* hub_key, int32_t* hub_chunk_base,
                            int32_t* multi_hubs, int32_t* chunk_hub, int64_t hub_capacity,
                            int64_t chunk_capacity, int32_t* item_first, int32_t* item_short,
                            int64_t item_capacity, int32_t* short_off, int32_t* short_gather,
                            relm_mp_plan_counts* pc, DevStatus* st, hipStream_t s) {
    const int64_t nblk = (num_keys + 1 + kThreads - 1) / kThreads;
    uint32_t* counts = scratch;
    uint32_t* totals = scratch + (kKeyRows + 1) * (nblk + 1);
    hipLaunchKernelGGL(k_key_stats, dim3(static_cast<unsigned>(nblk)), dim3(kThreads), 0, s, offsets,
                       num_keys, nblk, counts, st);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_scan_rows, dim3(kKeyRows), dim3(kScanThreads), 0, s, counts, nblk + 1,
                       totals);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_key_write, dim3(static_cast<unsigned>(nblk)), dim3(kThreads), 0, s, offsets,
                       gather_sorted, num_keys, nblk, static_cast<const uint32_t*>(counts),
                       static_cast<const uint32_t*>(totals), hub_key, hub_chunk_base, multi_hubs,
                       chunk_hub, hub_capacity, chunk_capacity, item_first, item_short,
                       item_capacity, short_off, short_gather, pc, st);
    return hipGetLastError();
}

}  // namespace relm_mp
