// Internal declarations shared by the HIP translation units of librelm_mp_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "relm_mp.h"

namespace relm_mp {

// Validation / plan statistics written by the plan kernels and read back to
// the host once per plan build (64 bytes).
struct DevStatus {
    unsigned long long bad_key_edge;     // smallest edge with a key out of range
    unsigned long long bad_gather_edge;  // smallest edge with a gathered index out of range
    unsigned long long collisions;       // inverse plans: edges whose key was already claimed
    unsigned long long num_hubs;         // CSR plans: segments longer than the hub threshold
    unsigned long long num_chunks;       // CSR plans: chunks over all hubs
    unsigned long long max_degree;       // CSR plans: longest segment
    unsigned long long num_multi_hubs;   // CSR plans: hubs of more than one chunk
    unsigned long long total_weight;     // CSR plans: sum of the walk weights of all keys
    unsigned long long gather_mismatch;  // CSR plans: nonzero if gathers[e] != e for some edge
    unsigned long long key_mismatch;     // inverse plans: nonzero if keys[e] != e for some edge
};
static_assert(sizeof(DevStatus) % sizeof(unsigned long long) == 0 &&
                  sizeof(DevStatus) / sizeof(unsigned long long) <= 64,
              "status words fit one wave");

constexpr unsigned long long kNoEdge = ~0ull;

// Geometry of CSR plans (see relm_mp.h): segments with more than
// kHubThreshold messages are hubs, reduced in chunks of kChunkSize messages;
// the others are walked in items of kItemSize positions.
constexpr int kHubThreshold = RELM_MP_HUB_THRESHOLD;
constexpr int kChunkSize = RELM_MP_CHUNK_SIZE;
constexpr int kItemSize = RELM_MP_ITEM_SIZE;

// Radix sort geometry (LSD, 8-bit digits at most).
constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;  // 4096 keys per block
constexpr int kSortMaxPasses = 4;                     // 32-bit keys, <= 8-bit digits
constexpr int kSortBins = 256;
constexpr int kSnapTile = RELM_MP_SNAP_TILE;
static_assert(kSnapTile == kSortTile, "the sort's first pass writes the snapshot tiles");

// Scan geometry.
constexpr int kScanThreads = 256;
constexpr int kScanItems = 32;
constexpr int kScanTile = kScanThreads * kScanItems;

int set_error(int code, const std::string& msg);
int hip_error(hipError_t err, const char* what);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---- plan kernels (plan_kernels.hip) -------------------------------------
hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t s);
// Resets the status; also zeroes `nclear` words at `clear` (sort_zero_region)
// and `nclear2` words at `clear2` (key_index_zero_region).
hipError_t launch_status_init(DevStatus* st, hipStream_t s, uint32_t* clear = nullptr,
                              int64_t nclear = 0, uint32_t* clear2 = nullptr, int64_t nclear2 = 0);
// Copies *st to pinned host memory through its device mapping, then stores
// `gen` to *host_gen (also mapped host memory) with a system-scope release,
// for the host to poll; with `pc`, also stores the inverse-plan statistics
// (collisions, identity) there.
hipError_t launch_status_publish(const DevStatus* st, DevStatus* host_mapped,
                                 relm_mp_plan_counts* pc, int32_t* host_gen, int32_t gen,
                                 hipStream_t s);
// Index snapshot written by a plan build (relm_mp_plan::snap_*): int32 per
// edge, tiles of kSnapTile edges whose values are their edge ids flagged in
// the plain arrays and not stored.  Null members are not written.
struct SnapOut {
    uint32_t* keys;
    uint32_t* gathers;
    uint32_t* key_plain;
    uint32_t* gather_plain;
};
hipError_t launch_inv_build(const int64_t* keys, int64_t key_bound, const int64_t* gathers,
                            int64_t gather_bound, int64_t n, int32_t* inv, const SnapOut& snap,
                            DevStatus* st, hipStream_t s);
// inv (filled with -1 before) [g(e)] = e for the n edges of a plan's int32
// snapshot (g(e) = e on tiles flagged in `plain`, which may be null), with plain
// stores; then st->collisions counts the edges whose row another edge took or
// whose index is >= key_bound, and st->key_mismatch flags g(e) != e.
hipError_t launch_inv_from_snapshot(const int32_t* snap, const uint32_t* plain, int64_t n,
                                    int64_t key_bound, int32_t* inv, DevStatus* st, hipStream_t s);


// Stable LSD radix sort of (key, value) by key into CSR form.  The first pass
// reads the caller's int64 keys / gathers, validates them against the bounds
// (bad entries are recorded in `st` and replaced by 0) and narrows them to 32
// bit into keys_n / vals_n in edge order (a plan keeps these as its snapshot);
// the scatter passes alternate between the a buffers and (keys_tmp,
// vals_out).  The last pass writes the values in key order to vals_out and,
// instead of the sorted keys, offsets[k] = the first sorted position with key
// >= k (key_bound + 1 entries, offsets[key_bound] = n).
struct SortBuffers {
    uint32_t* keys_n;
    uint32_t* vals_n;
    uint32_t* tile_plain;  // sort_tiles(n): tiles whose values are the edge ids (vals_n not written)
    uint32_t* keys_a;
    uint32_t* vals_a;
    uint32_t* hist;        // sort_hist_words(n): per-tile digit counts and key maxima, totals
};
int64_t sort_tiles(int64_t n);
size_t sort_hist_words(int64_t n);
// The words of buf.hist that must be zero when sort_by_key starts (the
// counting kernels add their per-chunk digit sums there with atomics).
struct SortZero {
    uint32_t* p;
    int64_t n;
};
SortZero sort_zero_region(const SortBuffers& buf, int64_t n);
// Where a build publishes its validation status to the host (memory mapped
// for the device; see launch_status_publish).  host == nullptr: nowhere.
struct StatusPublish {
    const DevStatus* st = nullptr;
    DevStatus* host = nullptr;
    int32_t* host_gen = nullptr;
    int32_t gen = 0;
};
// The status `st` holds the validation result once the first pass has run;
// the first pass's column scan publishes it as `pub` says.
// keys_tmp holds n words, free until the sort ends.
hipError_t sort_by_key(const int64_t* keys, int64_t key_bound, const int64_t* gathers,
                       int64_t gather_bound, int64_t n, const SortBuffers& buf,
                       uint32_t* keys_tmp, uint32_t* vals_out, int32_t* offsets, DevStatus* st,
                       hipStream_t s, const StatusPublish& pub);
// Per-key index of a CSR plan (deterministic, hubs in key order): hub list,
// chunk ranges and chunk -> hub map, walk items (balanced by weight: 1 plus the
// messages of a non-hub key), the short-segment index (short_off[k] = messages
// of non-hub keys before key k, num_keys + 1 entries; short_gather =
// gather_sorted without the hub segments; item_short[j] =
// short_off[item_first[j]]).  `scratch` holds key_index_words(num_keys) words;
// item_first and item_short have item_capacity + 1 entries
// (item_capacity_for(num_keys)).
size_t key_index_words(int64_t num_keys);
int64_t item_capacity_for(int64_t num_keys);
hipError_t launch_key_index(const int32_t* offsets, const int32_t* gather_sorted, int64_t num_keys,
                            uint32_t* scratch, int32_t* hub_key, int32_t* hub_chunk_base,
                            int32_t* multi_hubs, int32_t* chunk_hub, int64_t hub_capacity,
                            int64_t chunk_capacity, int32_t* item_first, int32_t* item_short,
                            int64_t item_capacity, int32_t* short_off, int32_t* short_gather,
                            relm_mp_plan_counts* counts, DevStatus* st, hipStream_t s);

// Capacities of the hub arrays of a CSR plan over num_edges edges.
inline int64_t max_hubs(int64_t num_edges) { return num_edges / (kHubThreshold + 1) + 1; }
inline int64_t max_chunks(int64_t num_edges) {
    return num_edges / kChunkSize + max_hubs(num_edges) + 1;
}

// ---- index packing (pack_kernels.hip) -------------------------------------
hipError_t launch_pack_index(const relm_mp_index_part* parts, int num_parts, int64_t* out_a,
                             int64_t* out_b, hipStream_t s);

// ---- FiLM step with Mish (film_kernels.hip) ---------------------------------
constexpr int kFilmMaxRanges = RELM_MP_FILM_MAX_RANGES;
// Blocks of RELM_MP_FILM_ROWS_PER_BLOCK rows of a range of `rows` rows.
inline int64_t film_range_blocks(int64_t rows) {
    return rows <= 0 ? 0 : (rows + RELM_MP_FILM_ROWS_PER_BLOCK - 1) / RELM_MP_FILM_ROWS_PER_BLOCK;
}
// range_start: num_ranges + 1 ascending host values from 0 to the row count
// (checked by the caller).
hipError_t launch_film_mish(const float* s, int64_t width, const int64_t* range_start,
                            int32_t num_ranges, const float* gamma, const float* beta,
                            const float* add, float* y, hipStream_t st);
hipError_t launch_film_mish_backward(const float* s, const float* dy, int64_t width,
                                     const int64_t* range_start, int32_t num_ranges,
                                     const float* gamma, const float* beta, const float* add,
                                     float* ds, double* partial, hipStream_t st);

// ---- content comparison (match_kernels.hip) -------------------------------
constexpr int kMaxMatch = RELM_MP_MAX_MATCH;
// After the launches mismatch[c] == gen iff the snapshot of plans[c] differs
// from (keys, gathers) (gathers null: keys only; every plan has num_edges ==
// n).  mismatch is not cleared first: a word left from an earlier call that
// happens to equal gen only reads as a difference (a rebuild, never a stale
// plan).  Then the num_plans words and, last, `gen` itself (a system-scope
// release) are stored to host_words[0..num_plans] and host_words[kMaxMatch]:
// host memory mapped for the device, which the host polls.
hipError_t launch_plan_match(const int64_t* keys, const int64_t* gathers, int64_t n,
                             const relm_mp_plan* const* plans, int num_plans, int32_t* mismatch,
                             int32_t gen, int32_t* host_words, hipStream_t s);

// ---- compute kernels (reduce_kernels.hip) --------------------------------
int compute_gather_last(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                        const void* table, int64_t emb, void* out, hipStream_t s);
// Rows in groups (relm_mp.h): the output of the gather, the table of the sum.
int compute_gather_last_grouped(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                                const void* table, int64_t emb, int64_t group,
                                int64_t group_stride, void* out, hipStream_t s);
int compute_segment_sum_grouped(int dtype, const relm_mp_plan& plan, const void* table,
                                int64_t emb, int64_t group, int64_t group_stride, void* out,
                                void* scratch, size_t scratch_bytes, hipStream_t s);
int compute_segment_reduce(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                           const void* table, int64_t emb, int64_t mode, void* out,
                           void* scratch, size_t scratch_bytes, hipStream_t s);
int compute_logsumexp_backward(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                               const void* grad_out, const void* out, const void* rel_flat,
                               int64_t emb, void* grad_rel, void* scratch, size_t scratch_bytes,
                               hipStream_t s);
int compute_fill(int dtype, void* out, int64_t count, double value, hipStream_t s);
int compute_segment_sum_scaled(int dtype, const relm_mp_plan& plan, const void* table,
                               int64_t emb, int div_kind, const int64_t* div_values,
                               const void* base, void* out, void* scratch, size_t scratch_bytes,
                               hipStream_t s);
int compute_segment_sum_msgdiv(int dtype, const relm_mp_plan& plan, const void* table, int64_t emb,
                               const int32_t* msg_div_offsets, const void* base, void* out,
                               void* scratch, size_t scratch_bytes, hipStream_t s);
int compute_rows_scale(int dtype, const void* in, const int64_t* gather, int div_kind,
                       const int32_t* div_offsets, const int64_t* div_values, const void* base,
                       int64_t rows, int64_t emb, void* out, hipStream_t s);
// Backward of fanin_reduce (mode 0 / 1) over a CSR plan keyed by destination
// whose gathered rows are the identity (plan.gather_identity); rows
// [num_edges, rel_rows) of grad_rel become zero.
int compute_backward_by_key(int dtype, const relm_mp_plan& plan, const int64_t* dst_idx,
                            int64_t mode, const void* grad_out, const void* out,
                            const void* rel_flat, int64_t emb, void* grad_rel, int64_t rel_rows,
                            hipStream_t s);
// Backward of fanin_reduce (mode 0 / 1) by rows of grad_rel through inv_plan
// (an inverse map of flat_src built without atomics, launch_inv_from_snapshot:
// the kernels do nothing on the device when its count of collisions is
// nonzero), each row's destination from dst_plan's int32 snapshot of dst_idx
// (dst_plan: the forward's CSR plan).
int compute_backward_by_src(int dtype, const relm_mp_plan& dst_plan, const relm_mp_plan& inv_plan,
                            int64_t mode, const void* grad_out, const void* out,
                            const void* rel_flat, int64_t emb, void* grad_rel, hipStream_t s);
size_t hub_partial_bytes(const relm_mp_plan& plan, int64_t emb, int dtype, int64_t mode);

}  // namespace relm_mp
