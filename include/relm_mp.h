/*
 * relm_mp.h - C ABI of the MI355X (gfx950) relational message-passing library
 * (librelm_mp_hip.so).
 *
 * Plain pointers, sizes and a HIP stream handle; no torch types.  All device
 * pointers are HIP device memory on the device that is current on the calling
 * thread.  Every entry point enqueues its kernels on `stream` (a hipStream_t
 * passed as void*).  Entry points that build an index plan validate every
 * index, and therefore synchronise `stream` once to read the validation status
 * back; the compute-only entry points (relm_mp_plan_*) never synchronise.
 *
 * Return value: RELM_MP_OK (0) or one of the RELM_MP_ERR_* codes.  On error,
 * relm_mp_last_error() returns a thread-local message that matches the
 * reference library's wording where the reference defines one.
 *
 * Reference interface replaced (maichmueller/relmo, src/_ops/mp/mp_ops.cpp):
 *   relm_mp_fanout_scatter                 <- relm::mp::fanout_scatter            mp_ops.cpp:3038-3101
 *   relm_mp_fanout_scatter_backward        <- relm::mp::fanout_scatter_backward   mp_ops.cpp:3103-3166
 *   relm_mp_fanin_reduce                   <- relm::mp::fanin_reduce (mode 0/1)   mp_ops.cpp:3327-3348,
 *                                             fanin_reduce_sum 3168-3222, fanin_reduce_logsumexp 3005-3036
 *   relm_mp_fanin_reduce_sum_backward      <- relm::mp::fanin_reduce_sum_backward mp_ops.cpp:3224-3284
 *   relm_mp_fanin_reduce_logsumexp_backward<- relm::mp::fanin_reduce_logsumexp_backward mp_ops.cpp:3286-3325
 *   relm_mp_build_info                     <- relm::mp::build_info                mp_ops.cpp:3745-3750
 * The reference binds these through TORCH_LIBRARY(relm_mp) (mp_ops.cpp:3754-3838);
 * this library's torch binding (relm_mp_ops.so) registers the same schemas
 * and calls the functions below.
 *
 * Index plans (relm_mp_inv_plan_*, relm_mp_csr_plan_*, relm_mp_plan_*) have no
 * counterpart in the reference: they expose the index preprocessing that the
 * op-level entry points perform internally, so that a caller can build a plan
 * once and reuse it while the index tensors stay unchanged.
 */
#ifndef RELM_MP_H
#define RELM_MP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* relm_mp_stream_t; /* hipStream_t */

enum relm_mp_status {
    RELM_MP_OK = 0,
    RELM_MP_ERR_INVALID_ARGUMENT = 1, /* negative size, size limit, mode */
    RELM_MP_ERR_INDEX_OUT_OF_BOUNDS = 2,
    RELM_MP_ERR_UNSUPPORTED_MODE = 3,
    RELM_MP_ERR_WORKSPACE = 4, /* workspace missing or too small */
    RELM_MP_ERR_HIP = 5        /* HIP runtime / launch error */
};

enum relm_mp_dtype { RELM_MP_F32 = 0, RELM_MP_F64 = 1 };

enum relm_mp_mode { RELM_MP_MODE_SUM = 0, RELM_MP_MODE_LOGSUMEXP = 1 };

/* Sizes accepted by the HIP path: every row count and edge count must be
 * below 2^31 - 1 (indices are narrowed to int32 inside plans). */
#define RELM_MP_MAX_ROWS 2147483646LL

/* CSR plans: segments with more messages than RELM_MP_HUB_THRESHOLD are hubs,
 * reduced in chunks of RELM_MP_CHUNK_SIZE messages (one workgroup per chunk);
 * hubs spanning more than one chunk combine their chunk results in chunk
 * order with one workgroup per hub.  The other segments are walked in items:
 * key k weighs 1 plus its message count (1 for a hub), W[k] is the sum of
 * the weights of the keys before k, and item j holds the keys with
 * W[k] in [j * RELM_MP_ITEM_SIZE, (j + 1) * RELM_MP_ITEM_SIZE). */
#define RELM_MP_HUB_THRESHOLD 64
#define RELM_MP_CHUNK_SIZE 2048
#define RELM_MP_ITEM_SIZE 32

const char* relm_mp_last_error(void);
/* "build_torch=...;build_cuda_tag=cpu;..." is produced by the torch binding;
 * this returns the HIP-side part: "hip=<ver>;arch=gfx950;kernels=..." */
const char* relm_mp_build_info(void);

/* ------------------------------------------------------------------------ */
/* Op-level entry points (one per reference op).  `workspace` is device      */
/* memory of at least *_workspace_size(...) bytes, 256-byte aligned.  The    */
/* output buffer is fully written (rows without messages become 0, or -inf   */
/* for the logsumexp forward); the caller need not clear it.                 */
/* ------------------------------------------------------------------------ */

/* out[out_rows, emb]: out[flat_dst[e]] = x_cat[src_global_idx[e]], the last
 * edge (largest e) wins on duplicate flat_dst, untouched rows are zero. */
size_t relm_mp_fanout_scatter_workspace_size(int64_t num_edges, int64_t out_rows);
int relm_mp_fanout_scatter(int dtype, const void* x_cat, int64_t x_rows, int64_t emb,
                           const int64_t* src_global_idx, const int64_t* flat_dst,
                           int64_t num_edges, int64_t out_rows, void* out,
                           void* workspace, size_t workspace_bytes, relm_mp_stream_t stream);

/* grad_x[x_rows, emb]: grad_x[src_global_idx[e]] += grad_out[flat_dst[e]]. */
size_t relm_mp_fanout_scatter_backward_workspace_size(int64_t num_edges, int64_t x_rows,
                                                      int64_t emb, int dtype);
int relm_mp_fanout_scatter_backward(int dtype, const void* grad_out, int64_t grad_out_rows,
                                    int64_t emb, const int64_t* src_global_idx,
                                    const int64_t* flat_dst, int64_t num_edges, int64_t x_rows,
                                    void* grad_x, void* workspace, size_t workspace_bytes,
                                    relm_mp_stream_t stream);

/* out[dim_size, emb]: mode 0: out[dst_idx[e]] += rel_flat[flat_src[e]];
 * mode 1: out[d] = log(sum exp(rel - max)) + max over the messages of d,
 * -inf for d without messages. */
size_t relm_mp_fanin_reduce_workspace_size(int64_t num_edges, int64_t dim_size, int64_t emb,
                                           int dtype);
int relm_mp_fanin_reduce(int dtype, const void* rel_flat, int64_t rel_rows, int64_t emb,
                         const int64_t* flat_src, const int64_t* dst_idx, int64_t num_edges,
                         int64_t dim_size, int64_t mode, void* out, void* workspace,
                         size_t workspace_bytes, relm_mp_stream_t stream);

/* relm_mp_fanin_reduce without a workspace and without allocating: no
 * counterpart in the reference.  For callers that cannot allocate device or
 * pinned host memory (tight serving loops, harnesses that forbid hipMalloc).
 * It cannot run under HIP graph capture: it synchronises `stream` once (the
 * index check), like relm_mp_fanin_reduce.  The plan, sort buffers and hub
 * partials live in a device array of RELM_MP_NOALLOC_SCRATCH_BYTES that the
 * library holds on every device it runs on until the process ends; a call
 * whose relm_mp_fanin_reduce_workspace_size exceeds it fails with
 * RELM_MP_ERR_WORKSPACE before launching anything (64 MiB: about 1.5 million
 * messages at emb 32).  All calls on one device share that array, so they are
 * serialised: host threads one at a time, and on the device each call's
 * kernels wait for the previous call's (an event per device, recorded behind
 * every call, which the next call's stream waits on), whatever streams the
 * calls use.  The array keeps the last call's contents, and every call writes
 * what it reads. */
#define RELM_MP_NOALLOC_SCRATCH_BYTES (64LL << 20)
int relm_mp_fanin_reduce_noalloc(int dtype, const void* rel_flat, int64_t rel_rows, int64_t emb,
                                 const int64_t* flat_src, const int64_t* dst_idx,
                                 int64_t num_edges, int64_t dim_size, int64_t mode, void* out,
                                 relm_mp_stream_t stream);

/* grad_rel[rel_rows, emb]: grad_rel[flat_src[e]] += grad_out[dst_idx[e]]. */
size_t relm_mp_fanin_reduce_sum_backward_workspace_size(int64_t num_edges, int64_t rel_rows,
                                                        int64_t emb, int dtype);
int relm_mp_fanin_reduce_sum_backward(int dtype, const void* grad_out, int64_t grad_out_rows,
                                      int64_t emb, const int64_t* flat_src,
                                      const int64_t* dst_idx, int64_t num_edges,
                                      int64_t rel_rows, void* grad_rel, void* workspace,
                                      size_t workspace_bytes, relm_mp_stream_t stream);

/* grad_rel[rel_rows, emb]:
 * grad_rel[flat_src[e]] += grad_out[d] * exp(rel_flat[flat_src[e]] - out[d]), d = dst_idx[e]. */
size_t relm_mp_fanin_reduce_logsumexp_backward_workspace_size(int64_t num_edges, int64_t rel_rows,
                                                              int64_t emb, int dtype);
int relm_mp_fanin_reduce_logsumexp_backward(int dtype, const void* grad_out, int64_t dim_size,
                                            int64_t emb, const void* rel_flat,
                                            int64_t rel_flat_rows, const int64_t* flat_src,
                                            const int64_t* dst_idx, int64_t num_edges,
                                            const void* out, int64_t rel_rows, void* grad_rel,
                                            void* workspace, size_t workspace_bytes,
                                            relm_mp_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Index plans (no reference counterpart).                                   */
/* ------------------------------------------------------------------------ */

enum relm_mp_plan_kind { RELM_MP_PLAN_INVERSE = 1, RELM_MP_PLAN_CSR = 2 };

/* Statistics of a plan as the build's kernels write them into plan memory.
 * They are valid in stream order after the build, so compute entry points
 * read them there and a plan is usable before the host has them. */
typedef struct relm_mp_plan_counts {
    int64_t max_degree;      /* CSR plans */
    int64_t num_hubs;
    int64_t num_chunks;
    int64_t num_multi_hubs;
    int64_t num_items;
    int64_t num_short;
    int64_t collisions;      /* inverse plans */
    int64_t identity;        /* inverse plans: 1 if keys[e] == e for every edge */
} relm_mp_plan_counts;

/* Descriptor of a plan.  All pointers point into the caller's plan memory.
 * The CSR statistics max_degree .. num_short are -1 after
 * relm_mp_csr_plan_build_async until relm_mp_plan_read_counts fills them. */
typedef struct relm_mp_plan {
    int32_t kind;
    int32_t hub_threshold;   /* CSR: segments longer than this use the hub path */
    int32_t chunk_size;      /* CSR: edges per hub chunk                        */
    int32_t gather_identity; /* CSR: 1 if gathers[e] == e for every edge (or no gathers) */
    int64_t num_keys;        /* rows on the scatter (keyed) side               */
    int64_t num_edges;
    int64_t num_gather;      /* rows on the gathered side                      */
    int64_t collisions;      /* inverse: edges whose key another edge also has */
    int64_t max_degree;      /* CSR: longest segment                           */
    int64_t num_hubs;        /* CSR: segments longer than hub_threshold        */
    int64_t num_chunks;      /* CSR: hub chunks                                */
    int64_t num_multi_hubs;  /* CSR: hubs with more than one chunk             */
    int64_t num_items;       /* CSR: walk items (see RELM_MP_ITEM_SIZE)        */
    int64_t num_short;       /* CSR: edges of the segments of at most hub_threshold */
    int32_t* inv;            /* inverse: [num_keys] largest edge id per key or -1;
                                NULL = identity (key k <-> edge k for k < num_edges) */
    int32_t* offsets;        /* CSR: [num_keys + 1] segment offsets            */
    int32_t* gather_sorted;  /* CSR: [num_edges] gathered row per edge, stable key order
                                (the keys in that order are not kept: key k holds
                                positions offsets[k] .. offsets[k + 1] - 1) */
    int32_t* hub_key;        /* CSR: [num_hubs] key of each hub                */
    int32_t* hub_chunk_base; /* CSR: [num_hubs] first chunk of each hub        */
    int32_t* chunk_hub;      /* CSR: [num_chunks] hub of each chunk            */
    int32_t* multi_hubs;     /* CSR: [num_multi_hubs] hub slots of those hubs  */
    int32_t* item_first;     /* CSR: [num_items + 1] first key of each item    */
    int32_t* item_short;     /* CSR: [num_items + 1] short_off[item_first[j]]  */
    int32_t* short_off;      /* CSR: [num_keys + 1] edges of non-hub segments before each key */
    int32_t* short_gather;   /* CSR: [num_short] gather_sorted without the hub segments;
                                equal to gather_sorted when there is no hub (set so once the
                                statistics are read: a waiting build, relm_mp_plan_read_counts) */
    const relm_mp_plan_counts* counts; /* the statistics, in device memory */
    /* The indices the plan was built from, as validated, in edge order: int32
     * per edge, for recognising them again (relm_mp_plan_match).  A tile of
     * RELM_MP_SNAP_TILE edges flagged in the *_plain array holds the edge ids
     * themselves (index[e] == e) and is not stored.  NULL where the plan keeps
     * no snapshot (snap_keys) or has no gathers (snap_gathers); a NULL *_plain
     * array means every tile is stored. */
    const int32_t* snap_keys;
    const int32_t* snap_gathers;
    const uint32_t* snap_key_plain;
    const uint32_t* snap_gather_plain;
} relm_mp_plan;

/* Edges per tile of a plan's index snapshot. */
#define RELM_MP_SNAP_TILE 4096
/* Flag of the inverse-plan builds: keep a snapshot of the indices. */
#define RELM_MP_PLAN_SNAPSHOT 1

/* Inverse plan: inv[k] = largest e with keys[e] == k, or -1 (plan->inv is
 * set to NULL when keys[e] == e for every edge: the identity).  Validates keys
 * against key_bound and gathers (if non-NULL) against gather_bound; the first
 * edge (in edge order) with a bad index is reported, `gather_checked_first`
 * choosing which array the reference checks first within one edge.  With
 * flags & RELM_MP_PLAN_SNAPSHOT the plan also keeps a snapshot of the indices
 * (plan memory from relm_mp_inv_plan_bytes with the same flags).
 * Synchronises `stream` once. */
size_t relm_mp_inv_plan_bytes(int64_t num_keys, int64_t num_edges, int flags);
int relm_mp_inv_plan_build(const int64_t* keys, int64_t key_bound, const char* key_name,
                           const int64_t* gathers, int64_t gather_bound, const char* gather_name,
                           int gather_checked_first, int64_t num_edges, int flags, void* plan_mem,
                           size_t plan_bytes, relm_mp_plan* plan, relm_mp_stream_t stream);
/* The same build without waiting: the validation result is pending until
 * relm_mp_plan_validate(plan).  Meanwhile relm_mp_plan_gather_last may be
 * enqueued on the plan (its kernels read the identity flag from
 * plan->counts; bad indices never make them access memory out of bounds),
 * but its result is only valid once relm_mp_plan_validate returns OK.
 * collisions is -1 until then, and `keys` / `gathers` must stay valid until
 * then (a bad index's value is read back for the message).  One validation
 * may be pending per host thread and device; a plan build on that thread
 * fails until it is done.
 * No counterpart in the reference: it lets fanout_scatter enqueue its gather
 * before the host waits for the index check. */
int relm_mp_inv_plan_build_async(const int64_t* keys, int64_t key_bound, const char* key_name,
                                 const int64_t* gathers, int64_t gather_bound,
                                 const char* gather_name, int gather_checked_first,
                                 int64_t num_edges, int flags, void* plan_mem, size_t plan_bytes,
                                 relm_mp_plan* plan, relm_mp_stream_t stream);
/* Waits for the pending validation of `plan` (relm_mp_inv_plan_build_async)
 * and reports it like relm_mp_inv_plan_build; fills collisions and sets
 * inv to NULL for the identity.  Returns OK at once if nothing is pending. */
int relm_mp_plan_validate(relm_mp_plan* plan);

/* CSR plan: stable counting order of the edges by key (edge order kept inside
 * each segment), offsets, the gathered row of every edge in that order, and the
 * list of hub segments.  Validates like relm_mp_inv_plan_build.  Waits for
 * `stream` to finish the build and fills the statistics.  CSR plans always
 * keep the snapshot of their indices (the sort's first pass writes it). */
size_t relm_mp_csr_plan_bytes(int64_t num_keys, int64_t num_edges);
size_t relm_mp_csr_plan_scratch_bytes(int64_t num_keys, int64_t num_edges);
int relm_mp_csr_plan_build(const int64_t* keys, int64_t key_bound, const char* key_name,
                           const int64_t* gathers, int64_t gather_bound, const char* gather_name,
                           int gather_checked_first, int64_t num_edges, void* plan_mem,
                           size_t plan_bytes, void* scratch, size_t scratch_bytes,
                           relm_mp_plan* plan, relm_mp_stream_t stream);
/* The same build, returning as soon as the indices are validated (after the
 * first sort pass; the rest of the build stays queued on `stream`): the
 * host-side statistics are -1 and gather_identity is set.  No counterpart in
 * the reference: callers that go on to enqueue compute work on the plan use
 * it so that the device does not idle while the host waits. */
int relm_mp_csr_plan_build_async(const int64_t* keys, int64_t key_bound, const char* key_name,
                                 const int64_t* gathers, int64_t gather_bound,
                                 const char* gather_name, int gather_checked_first,
                                 int64_t num_edges, void* plan_mem, size_t plan_bytes,
                                 void* scratch, size_t scratch_bytes, relm_mp_plan* plan,
                                 relm_mp_stream_t stream);
/* Copies plan->counts into the host-side statistics of a CSR plan
 * (synchronises `stream`). */
int relm_mp_plan_read_counts(relm_mp_plan* plan, relm_mp_stream_t stream);

/* Scratch needed by the compute entry points below for hub partial results
 * of a CSR plan (0 for inverse plans). */
size_t relm_mp_plan_compute_scratch_bytes(const relm_mp_plan* plan, int64_t emb, int dtype,
                                          int64_t mode);

/* out[num_keys, emb] = per key: inverse plan -> table[gathers[inv[k]]] or 0;
 * CSR plan -> last edge of the segment (fanout "last wins") or 0. */
int relm_mp_plan_gather_last(int dtype, const relm_mp_plan* plan, const int64_t* gathers,
                             const void* table, int64_t emb, void* out,
                             relm_mp_stream_t stream);
/* out[num_keys, emb] = per key, sum over the segment of table[gathered row]
 * (inverse plans require collisions == 0), or logsumexp (mode 1, CSR plans). */
int relm_mp_plan_segment_reduce(int dtype, const relm_mp_plan* plan, const int64_t* gathers,
                                const void* table, int64_t emb, int64_t mode, void* out,
                                void* scratch, size_t scratch_bytes, relm_mp_stream_t stream);
/* grad_rel[num_keys, emb] = per key r, sum over its edges of
 * grad_out[d] * exp(rel_flat[r] - out[d]) with d the gathered row. */
int relm_mp_plan_logsumexp_backward(int dtype, const relm_mp_plan* plan, const int64_t* gathers,
                                    const void* grad_out, const void* out, const void* rel_flat,
                                    int64_t emb, void* grad_rel, void* scratch,
                                    size_t scratch_bytes, relm_mp_stream_t stream);
/* Backward of fanin_reduce over the FORWARD's CSR plan (keys = dst_idx,
 * gathers = flat_src) when flat_src is the identity (dst_plan->gather_identity,
 * which also makes every message row distinct).  dst_idx is the int64 array the
 * plan was built from (validated by that build).  For every edge e:
 * mode 0: grad_rel[e] = grad_out[dst_idx[e]];
 * mode 1: grad_rel[e] = grad_out[d] * exp(rel_flat[e] - out[d]), d = dst_idx[e];
 * rows [num_edges, rel_rows) become 0.  Requires num_edges <= rel_rows.  The
 * result equals relm_mp_fanin_reduce_sum_backward / _logsumexp_backward for
 * the same tensors, without building the inverse plan; rel_flat and out are
 * read in mode 1 only. */
int relm_mp_plan_fanin_backward_by_dst(int dtype, const relm_mp_plan* dst_plan,
                                       const int64_t* dst_idx, int64_t mode,
                                       const void* grad_out, const void* out,
                                       const void* rel_flat, int64_t emb, void* grad_rel,
                                       int64_t rel_rows, relm_mp_stream_t stream);
/* Backward of fanin_reduce over the FORWARD's CSR plan when flat_src is not the
 * identity: the inverse map of flat_src (rows of grad_rel -> edges) is built
 * from the plan's int32 snapshot of flat_src (validated by the plan's build)
 * with plain stores - no atomics, no second validation - and a second pass
 * counts the edges whose row another edge also reads (collisions).  The
 * backward kernel is queued right after and does nothing on the device when
 * that count is nonzero; the call then waits for the count and stores it in
 * *collisions.  0: grad_rel [rel_rows, emb] holds what
 * relm_mp_fanin_reduce_sum_backward (mode 0) / _logsumexp_backward (mode 1)
 * give for the same tensors (rows no edge reads are 0).  Nonzero: flat_src
 * repeats and grad_rel is unspecified (use a CSR plan keyed by flat_src).
 * Requires rel_rows >= dst_plan->num_gather; rel_flat has rel_rows rows (read
 * in mode 1 only).  inv_mem holds relm_mp_inv_plan_bytes(rel_rows,
 * dst_plan->num_edges, 0) bytes.  map_ready != 0: inv_mem already holds the
 * map an earlier call built for this dst_plan and rel_rows with no collision
 * (that call's work on `stream` precedes this one); only the backward kernel is
 * launched, without waiting, and *collisions is 0.  With rel_rows ==
 * num_edges the map is built without an initial fill (an injective flat_src
 * writes every row) and the sum (mode 0) runs in edge order over the plan's
 * snapshots, each edge writing its own row.  No reference counterpart:
 * it replaces the inverse-plan build of the backward ops (mp_ops.cpp:3224-3325
 * take flat_src and dst_idx afresh) for callers that hold the forward's plan. */
int relm_mp_plan_fanin_backward_by_src(int dtype, const relm_mp_plan* dst_plan, int64_t mode,
                                       const void* grad_out, const void* out, const void* rel_flat,
                                       int64_t emb, void* grad_rel, int64_t rel_rows, void* inv_mem,
                                       size_t inv_bytes, int map_ready, int64_t* collisions,
                                       relm_mp_stream_t stream);

/* ---- row epilogues (the LGAN indexed reductions) ------------------------- */

#define RELM_MP_DIV_NONE 0    /* d_j = 1                                          */
#define RELM_MP_DIV_SEGMENT 1 /* d_j = max(1, div_offsets[j+1] - div_offsets[j])  */
#define RELM_MP_DIV_VALUES 2  /* d_j = max(1, (T)div_values[j])                   */

/* For r < rows: j = gather ? gather[r] : r (gather: valid rows of `in` and of
 * the divisor array), out[r] = base[r] + in[j] / d_j; `in` NULL reads zeros,
 * `base` NULL adds nothing (out = in[j] / d_j).  out may equal base, or in
 * when gather is NULL.  The epilogues of the reference's LGAN aggregations
 * (relm::mp::lgan_pool_reduce / _relation_graph_step and their backward,
 * mp_ops.cpp:3350-3743): division by the arity or the message count, the
 * residual addition, the per-slot gradient; with div_offsets the offsets of a
 * CSR plan keyed by the aggregation's destinations.  Row-major [*, emb]. */
int relm_mp_rows_scale(int dtype, const void* in, const int64_t* gather, int div_kind,
                       const int32_t* div_offsets, const int64_t* div_values, const void* base,
                       int64_t rows, int64_t emb, void* out, relm_mp_stream_t stream);

/* out[num_keys, emb] = per key k of a CSR plan: base[k] + S_k / d_k, S_k the
 * sum over the segment of table[gathered row] (as relm_mp_plan_segment_reduce
 * mode 0), d_k = 1 (RELM_MP_DIV_NONE), max(1, segment size) (RELM_MP_DIV_SEGMENT:
 * the mean) or max(1, (T)div_values[k]) (RELM_MP_DIV_VALUES); base may be NULL
 * and must not alias out.  One pass: the LGAN aggregations with their epilogue
 * (mp_ops.cpp:3439-3467, 3650-3655: sum or mean, the residual addition, the
 * division by the arity). */
int relm_mp_plan_segment_sum_scaled(int dtype, const relm_mp_plan* plan, const void* table,
                                    int64_t emb, int div_kind, const int64_t* div_values,
                                    const void* base, void* out, void* scratch,
                                    size_t scratch_bytes, relm_mp_stream_t stream);

/* As relm_mp_plan_segment_sum_scaled with RELM_MP_DIV_NONE, but each gathered
 * row g is divided by its own message count before it is added: out[k] =
 * base[k] + sum over the segment of table[g] / max(1, msg_div_offsets[g + 1] -
 * msg_div_offsets[g]), msg_div_offsets the offsets of a CSR plan keyed by the
 * table's rows (valid for every gathered row).  The transposed mean of the LGAN
 * aggregations in one pass (mp_ops.cpp:3548-3557: gathered rows divided by
 * their counts, then index_add_), without the divided copy of the table that
 * relm_mp_rows_scale would write; the same results bit for bit. */
int relm_mp_plan_segment_sum_msgdiv(int dtype, const relm_mp_plan* plan, const void* table,
                                    int64_t emb, const int32_t* msg_div_offsets, const void* base,
                                    void* out, void* scratch, size_t scratch_bytes,
                                    relm_mp_stream_t stream);

/* ---- rows in groups (fanout straight into a wider input matrix) ----------- */

/* Grouped row layout: row r of a [rows, emb] operand lies at element offset
 * (r / group) * group_stride + (r % group) * emb from its base pointer, i.e.
 * `group` consecutive rows per line of a wider row-major matrix whose lines
 * are group_stride elements apart (group >= 1, group_stride >= group * emb).
 * The relational models assemble their central MLP input as [nodes, width]
 * lines of context columns followed by max_arity argument slots of emb
 * columns (relmo/models/hetero_mp/fused.py:299-375: fanout_scatter into
 * args_flat [nodes * max_arity, emb], reshape, copy into all_inputs).  With
 * group = max_arity, group_stride = width and the base pointer at the first
 * argument column, the fanout writes there directly and its backward reads
 * the gradient from there, without the [nodes * max_arity, emb] copy.  No
 * counterpart in the reference, which has no out-variant of the op. */

/* relm_mp_plan_gather_last with grouped output rows: row k (k < num_keys,
 * num_keys a multiple of group) is written at the grouped offset; the
 * elements between the rows (other columns of the lines) are not touched. */
int relm_mp_plan_gather_last_grouped(int dtype, const relm_mp_plan* plan, const int64_t* gathers,
                                     const void* table, int64_t emb, int64_t group,
                                     int64_t group_stride, void* out, relm_mp_stream_t stream);
/* relm_mp_plan_segment_reduce mode 0 over a CSR plan whose gathered rows are
 * read from `table` in the grouped layout (gathered index r < table_rows, a
 * multiple of group); out[num_keys, emb] is row-major. */
int relm_mp_plan_segment_sum_grouped(int dtype, const relm_mp_plan* plan, const void* table,
                                     int64_t table_rows, int64_t emb, int64_t group,
                                     int64_t group_stride, void* out, void* scratch,
                                     size_t scratch_bytes, relm_mp_stream_t stream);

/* ---- content match (plan reuse across equal indices) ----------------------- */

/* No counterpart in the reference (its ops build their index structures in
 * every call).  A caller that keeps plans (the torch binding's plan cache)
 * uses this to reuse a plan only for index arrays whose contents equal the
 * snapshot the plan was built from - so a plan is never served for indices
 * that were changed after the build, however they were changed. */
#define RELM_MP_MAX_MATCH 8

size_t relm_mp_plan_match_workspace_size(void);

/* match[c] = 1 if n == plans[c]->num_edges, keys[0..n) equal the plan's key
 * snapshot and (when gathers is not NULL) gathers[0..n) equal its gather
 * snapshot, else 0; 0 <= num_plans <= RELM_MP_MAX_MATCH, every plan with a
 * snapshot (and a gather snapshot when gathers is not NULL).  keys / gathers
 * are device memory, `match` host memory.  Enqueues one pass on `stream`
 * (the plans' builds must precede it in stream order) and returns once the
 * result is known. */
int relm_mp_plan_match(const int64_t* keys, const int64_t* gathers, int64_t n,
                       const relm_mp_plan* const* plans, int32_t num_plans, int32_t* match,
                       void* workspace, size_t workspace_bytes, relm_mp_stream_t stream);

/* ---- index packing (the pack ops) -------------------------------------- */

/* One part of a packing call: n index pairs (a[i], b[i]) written as
 * a[i] * a_mul + a_add and b[i] * b_mul + b_add. */
typedef struct relm_mp_index_part {
    const int64_t* a;
    const int64_t* b;
    int64_t n;
    int64_t a_mul;
    int64_t a_add;
    int64_t b_mul;
    int64_t b_add;
} relm_mp_index_part;

/* out_a / out_b [sum of n] = the parts' transformed pairs, back to back in part
 * order; device pointers, one kernel launch per 16 parts.  out_b may be NULL:
 * then only out_a is written and the parts' b arrays are not read.  The index arithmetic
 * of relm::mp::fanout_pack_multi (mp_ops.cpp:412-484: src + row offset, flat_dst
 * unchanged), fanin_pack_multi (:486-570: flat_src + row offset, dst unchanged),
 * fanout_pack_from_edges (:2511-2634: src + part offset, slot_offset +
 * dst * arity + pos) and fanin_pack_from_edges (:2636-2772: src * arity + pos +
 * part offset, or src + part offset, dst unchanged) - the torch binding maps
 * each op's parts onto this. */
int relm_mp_pack_index(const relm_mp_index_part* parts, int32_t num_parts, int64_t* out_a,
                       int64_t* out_b, relm_mp_stream_t stream);

/* ---- FiLM step with Mish for central layers (no counterpart in the reference,
 * which runs it as torch ops inside its central module: relmo/models/film.py
 * conditioning, relational_gnn.py:757-787) ------------------------------------
 * Rows [range_start[k], range_start[k + 1]) of s [rows, width] (float32,
 * row-major) form range k and share row k of gamma, beta and add [num_ranges,
 * width] (add may be NULL: zero):
 *   y[r] = mish(beta[k] + gamma[k] * (s[r] + add[k])),  mish(u) = u tanh(softplus(u)).
 * range_start: num_ranges + 1 ascending host values from 0 to rows,
 * 1 <= num_ranges <= RELM_MP_FILM_MAX_RANGES. */
#define RELM_MP_FILM_MAX_RANGES 16
#define RELM_MP_FILM_ROWS_PER_BLOCK 512
int relm_mp_film_mish(const float* s, int64_t rows, int64_t width, const int64_t* range_start,
                      int32_t num_ranges, const float* gamma, const float* beta, const float* add,
                      float* y, relm_mp_stream_t stream);

/* Blocks of the backward's partial sums for these ranges (each range in blocks of
 * RELM_MP_FILM_ROWS_PER_BLOCK rows); -1 for invalid ranges. */
int64_t relm_mp_film_mish_blocks(const int64_t* range_start, int32_t num_ranges);

/* Backward of relm_mp_film_mish given dy [rows, width]: ds = du * gamma[k] with
 * du = dy * mish'(u), u = beta[k] + gamma[k] * (s + add[k]); partial [blocks, 2,
 * width] (float64) receives per block (the blocks of range k are consecutive, in
 * row order) the column sums of du * (s + add[k]) and of du over its rows, each
 * fp32 term added in fp64: summed over range k's blocks they are the gradients of
 * gamma[k] and of beta[k] (that of add[k] is gamma[k] times the latter).
 * partial_blocks >= relm_mp_film_mish_blocks(...). */
int relm_mp_film_mish_backward(const float* s, const float* dy, int64_t rows, int64_t width,
                               const int64_t* range_start, int32_t num_ranges, const float* gamma,
                               const float* beta, const float* add, float* ds, double* partial,
                               int64_t partial_blocks, relm_mp_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RELM_MP_H */
