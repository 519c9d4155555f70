// C ABI of librelm_mp_hip.so: index plans and the op-level entry points that
// stand in for the reference's fanout_scatter / fanin_reduce ops
// (maichmueller/relmo src/_ops/mp/mp_ops.cpp:3038-3348).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <string>

#include "internal.h"
#include "relm_mp.h"

namespace relm_mp {

namespace {

thread_local std::string g_last_error;

// Bump allocator over caller memory; every piece is 256-byte aligned.
struct Carver {
    char* base;
    size_t off = 0;
    explicit Carver(void* b) : base(static_cast<char*>(b)) {}
    template <typename T>
    T* take(size_t count) {
        off = align_up(off, 256);
        T* p = base != nullptr ? reinterpret_cast<T*>(base + off) : nullptr;
        off += std::max<size_t>(count, 1) * sizeof(T);
        return p;
    }
    size_t used() const { return align_up(off, 256); }
};

int check_rows(int64_t v, const char* name) {
    if (v < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, std::string(name) + " must be >= 0.");
    if (v > RELM_MP_MAX_ROWS)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         std::string("relm_mp HIP path: ") + name + " exceeds 2^31 - 2.");
    return RELM_MP_OK;
}

int check_dtype(int dtype) {
    if (dtype != RELM_MP_F32 && dtype != RELM_MP_F64)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp HIP path: dtype must be f32 or f64");
    return RELM_MP_OK;
}

#define RELM_TRY(expr)                      \
    do {                                    \
        const int _rc = (expr);             \
        if (_rc != RELM_MP_OK) return _rc;  \
    } while (0)

#define RELM_HIP(expr, what)                                  \
    do {                                                      \
        const hipError_t _e = (expr);                         \
        if (_e != hipSuccess) return hip_error(_e, what);     \
    } while (0)

// Turns a bad index recorded in a status read back to the host into the
// reference's message "<name> index out of bounds: i not in [0, n)." for the
// first offending edge in edge order.
int check_validation(const DevStatus& host, const int64_t* keys, int64_t key_bound,
                     const char* key_name, const int64_t* gathers, int64_t gather_bound,
                     const char* gather_name, int gather_checked_first) {
    const unsigned long long ek = host.bad_key_edge;
    const unsigned long long eg = gathers != nullptr ? host.bad_gather_edge : kNoEdge;
    if (ek == kNoEdge && eg == kNoEdge) return RELM_MP_OK;
    bool use_gather;
    if (ek == eg) {
        use_gather = gather_checked_first != 0;
    } else {
        use_gather = eg < ek;
    }
    const int64_t* arr = use_gather ? gathers : keys;
    const unsigned long long e = use_gather ? eg : ek;
    int64_t value = 0;
    RELM_HIP(hipMemcpy(&value, arr + e, sizeof(int64_t), hipMemcpyDeviceToHost),
             "relm_mp index copy");
    const char* name = use_gather ? gather_name : key_name;
    const int64_t bound = use_gather ? gather_bound : key_bound;
    char buf[256];
    std::snprintf(buf, sizeof(buf), "%s index out of bounds: %lld not in [0, %lld).",
                  name != nullptr ? name : "index", static_cast<long long>(value),
                  static_cast<long long>(bound));
    return set_error(RELM_MP_ERR_INDEX_OUT_OF_BOUNDS, buf);
}

// Per host thread and device: pinned host memory (a few hundred bytes,
// allocated on the thread's first build on that device and kept until the
// process ends) into which the device publishes a plan's status, its
// counts and plan-match flags, each publication followed by a generation
// word that the host polls.  A build waits for its own publication before
// returning, so one slot per thread suffices.
//
// An index validation whose result has not been read yet (inverse plans
// built without waiting): what the error message needs.
struct PendingCheck {
    bool active = false;
    const void* plan_counts = nullptr;  // identifies the plan
    const int64_t* keys = nullptr;
    int64_t key_bound = 0;
    std::string key_name;
    const int64_t* gathers = nullptr;
    int64_t gather_bound = 0;
    std::string gather_name;
    int gather_checked_first = 0;
    int32_t gen = 0;           // the status publication to wait for
    hipStream_t stream = nullptr;
};

struct HostSlot {
    int device = -1;
    DevStatus* status = nullptr;         // host address
    DevStatus* status_mapped = nullptr;  // the same memory as the device addresses it
    relm_mp_plan_counts* counts = nullptr;
    int32_t* match = nullptr;         // host address: kMaxMatch flags, then the generation word
    int32_t* match_mapped = nullptr;  // the same words as the device addresses them
    int32_t match_gen = 0;            // generation of the last plan match from this slot
    int32_t* status_gen = nullptr;         // host address of the status publication word
    int32_t* status_gen_mapped = nullptr;  // the same word as the device addresses it
    int32_t status_issued = 0;             // generation of the last status publication
    PendingCheck pending;

    // Enqueues the publication of `st` (and, with pc, the inverse-plan
    // statistics) to this slot's host status; returns its generation.
    hipError_t publish_status(const DevStatus* st, relm_mp_plan_counts* pc, hipStream_t s,
                              int32_t* gen) {
        *gen = next_gen();
        return launch_status_publish(st, status_mapped, pc, status_gen_mapped, *gen, s);
    }
    // The target of a publication that a kernel of the caller's makes.
    StatusPublish publish_target(const DevStatus* st, int32_t* gen) {
        *gen = next_gen();
        return StatusPublish{st, status_mapped, status_gen_mapped, *gen};
    }
    int32_t next_gen() {
        status_issued = static_cast<int32_t>(static_cast<uint32_t>(status_issued) + 1u);
        return status_issued;
    }
};

// Waits until the device has stored `want` into *word (host memory mapped for
// the device, written with a system-scope release behind the data it
// guards).  Spins; after 2 ms without the store, and every millisecond from
// then on, asks whether the stream has failed or drained without storing it
// (either is an error).  Not earlier: a stream query can leave a marker in
// the stream, a pause of several microseconds between the kernels around it,
// and most waits end within a few hundred microseconds.
int wait_host_word(const int32_t* word, int32_t want, hipStream_t s, const char* what) {
    using Clock = std::chrono::steady_clock;
    const Clock::time_point start = Clock::now();
    Clock::time_point next_query = start + std::chrono::milliseconds(2);
    for (uint64_t spin = 1;; ++spin) {
        if (__atomic_load_n(word, __ATOMIC_ACQUIRE) == want) return RELM_MP_OK;
        if ((spin & 255) == 0) {
            const Clock::time_point now = Clock::now();
            if (now >= next_query) {
                next_query = now + std::chrono::milliseconds(1);
                const hipError_t q = hipStreamQuery(s);
                if (q == hipSuccess) {
                    if (__atomic_load_n(word, __ATOMIC_ACQUIRE) == want) return RELM_MP_OK;
                    return set_error(RELM_MP_ERR_HIP,
                                     std::string(what) + ": the device did not publish its result");
                }
                if (q != hipErrorNotReady) {
                    (void)hipGetLastError();
                    return set_error(RELM_MP_ERR_HIP, std::string(what) + ": " + hipGetErrorString(q));
                }
            }
            if (now - start > std::chrono::milliseconds(20)) std::this_thread::yield();
        }
        __builtin_ia32_pause();
    }
}

int no_pending(const HostSlot* hs) {
    if (hs->pending.active)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         "relm_mp: a plan built without waiting has not been validated yet "
                         "(relm_mp_plan_validate)");
    return RELM_MP_OK;
}

int host_slot(HostSlot** out) {
    thread_local HostSlot slots[16];
    int dev = 0;
    RELM_HIP(hipGetDevice(&dev), "relm_mp device query");
    for (HostSlot& h : slots) {
        if (h.device == dev) {
            *out = &h;
            return RELM_MP_OK;
        }
    }
    for (HostSlot& h : slots) {
        if (h.device < 0) {
            void* mem = nullptr;
            RELM_HIP(hipHostMalloc(&mem,
                                   sizeof(DevStatus) + sizeof(relm_mp_plan_counts) +
                                       (kMaxMatch + 2) * sizeof(int32_t),
                                   hipHostMallocDefault),
                     "relm_mp pinned status");
            h.status = static_cast<DevStatus*>(mem);
            h.counts = reinterpret_cast<relm_mp_plan_counts*>(static_cast<char*>(mem) + sizeof(DevStatus));
            h.match = reinterpret_cast<int32_t*>(h.counts + 1);
            void* mapped = nullptr;
            RELM_HIP(hipHostGetDevicePointer(&mapped, mem, 0), "relm_mp pinned status mapping");
            h.status_mapped = static_cast<DevStatus*>(mapped);
            h.match_mapped = reinterpret_cast<int32_t*>(static_cast<char*>(mapped) +
                                                        (reinterpret_cast<char*>(h.match) - static_cast<char*>(mem)));
            h.match[kMaxMatch] = 0;
            h.status_gen = h.match + kMaxMatch + 1;
            h.status_gen_mapped = h.match_mapped + kMaxMatch + 1;
            *h.status_gen = 0;
            h.device = dev;
            *out = &h;
            return RELM_MP_OK;
        }
    }
    return set_error(RELM_MP_ERR_HIP, "relm_mp: too many devices for one host thread");
}

int read_counts(relm_mp_plan* plan, hipStream_t s) {
    if (plan->kind != RELM_MP_PLAN_CSR || plan->counts == nullptr) return RELM_MP_OK;
    HostSlot* hs = nullptr;
    RELM_TRY(host_slot(&hs));
    RELM_HIP(hipMemcpyAsync(hs->counts, plan->counts, sizeof(relm_mp_plan_counts),
                            hipMemcpyDeviceToHost, s),
             "relm_mp counts copy");
    RELM_HIP(hipStreamSynchronize(s), "relm_mp counts sync");
    const relm_mp_plan_counts c = *hs->counts;
    plan->max_degree = c.max_degree;
    plan->num_hubs = c.num_hubs;
    plan->num_chunks = c.num_chunks;
    plan->num_multi_hubs = c.num_multi_hubs;
    plan->num_items = c.num_items;
    plan->num_short = c.num_short;
    // without hubs the short segments are the whole sorted gather array, which
    // the key index then does not copy
    if (c.num_hubs == 0) plan->short_gather = plan->gather_sorted;
    return RELM_MP_OK;
}

struct InvLayout {
    DevStatus* status;
    relm_mp_plan_counts* counts;
    int32_t* inv;
    SnapOut snap;  // all null without RELM_MP_PLAN_SNAPSHOT
    size_t bytes;
};

InvLayout inv_layout(void* mem, int64_t num_keys, int64_t num_edges, int flags) {
    Carver c(mem);
    InvLayout l;
    l.status = c.take<DevStatus>(1);
    l.counts = c.take<relm_mp_plan_counts>(1);
    l.inv = c.take<int32_t>(static_cast<size_t>(num_keys));
    l.snap = SnapOut{nullptr, nullptr, nullptr, nullptr};
    if (flags & RELM_MP_PLAN_SNAPSHOT) {
        const size_t n = static_cast<size_t>(num_edges);
        const size_t tiles = static_cast<size_t>(sort_tiles(num_edges));
        l.snap.keys = c.take<uint32_t>(n);
        l.snap.gathers = c.take<uint32_t>(n);
        l.snap.key_plain = c.take<uint32_t>(tiles);
        l.snap.gather_plain = c.take<uint32_t>(tiles);
    }
    l.bytes = c.used();
    return l;
}


struct CsrLayout {
    DevStatus* status;
    relm_mp_plan_counts* counts;
    int32_t* offsets;
    int32_t* gather_sorted;
    int32_t* hub_key;
    int32_t* hub_chunk_base;
    int32_t* chunk_hub;
    int32_t* multi_hubs;
    int32_t* item_first;
    int32_t* item_short;
    int32_t* short_off;
    int32_t* short_gather;
    uint32_t* snap_keys;   // the sort's narrowed input (edge order) is the plan's snapshot
    uint32_t* snap_gathers;
    uint32_t* snap_plain;  // per sort tile: gathers are the edge ids, snap_gathers not written
    int64_t num_items;
    size_t bytes;
};

CsrLayout csr_layout(void* mem, int64_t num_keys, int64_t num_edges) {
    Carver c(mem);
    CsrLayout l;
    l.status = c.take<DevStatus>(1);
    l.counts = c.take<relm_mp_plan_counts>(1);
    l.offsets = c.take<int32_t>(static_cast<size_t>(num_keys) + 1);
    l.gather_sorted = c.take<int32_t>(static_cast<size_t>(num_edges));
    l.hub_key = c.take<int32_t>(static_cast<size_t>(max_hubs(num_edges)));
    l.hub_chunk_base = c.take<int32_t>(static_cast<size_t>(max_hubs(num_edges)));
    l.chunk_hub = c.take<int32_t>(static_cast<size_t>(max_chunks(num_edges)));
    l.multi_hubs = c.take<int32_t>(static_cast<size_t>(max_hubs(num_edges)));
    l.num_items = item_capacity_for(num_keys);
    l.item_first = c.take<int32_t>(static_cast<size_t>(l.num_items) + 1);
    l.item_short = c.take<int32_t>(static_cast<size_t>(l.num_items) + 1);
    l.short_off = c.take<int32_t>(static_cast<size_t>(num_keys) + 1);
    l.short_gather = c.take<int32_t>(static_cast<size_t>(num_edges));
    l.snap_keys = c.take<uint32_t>(static_cast<size_t>(num_edges));
    l.snap_gathers = c.take<uint32_t>(static_cast<size_t>(num_edges));
    l.snap_plain = c.take<uint32_t>(static_cast<size_t>(sort_tiles(num_edges)));
    l.bytes = c.used();
    return l;
}

struct CsrScratch {
    SortBuffers sort;
    uint32_t* key_index;
    size_t bytes;
};

CsrScratch csr_scratch(void* mem, int64_t num_keys, int64_t num_edges) {
    Carver c(mem);
    CsrScratch l;
    const size_t n = static_cast<size_t>(num_edges);
    l.sort.keys_a = c.take<uint32_t>(n);
    l.sort.vals_a = c.take<uint32_t>(n);
    const size_t hist = sort_hist_words(num_edges);
    l.sort.hist = c.take<uint32_t>(hist);
    l.sort.keys_n = l.sort.vals_n = l.sort.tile_plain = nullptr;  // in the plan (csr_layout)
    l.key_index = c.take<uint32_t>(key_index_words(num_keys));
    l.bytes = c.used();
    return l;
}

size_t hub_partial_upper_bound(int64_t num_edges, int64_t emb, int dtype, int64_t mode) {
    const size_t elem = dtype == RELM_MP_F64 ? 8 : 4;
    return align_up(static_cast<size_t>(max_chunks(num_edges)) * static_cast<size_t>(emb) * elem *
                        (mode == RELM_MP_MODE_LOGSUMEXP ? 2 : 1),
                    256);
}

// Fills the host-side statistics of a validated inverse plan.
void finish_inverse(relm_mp_plan* plan, const DevStatus& host) {
    plan->collisions = static_cast<int64_t>(host.collisions);
    // keys[e] == e for every edge: the map is the identity, which the compute
    // kernels apply without reading inv (one dependent load less per row)
    if (host.key_mismatch == 0) plan->inv = nullptr;
}

int inv_build(const int64_t* keys, int64_t key_bound, const char* key_name, const int64_t* gathers,
              int64_t gather_bound, const char* gather_name, int gather_checked_first,
              int64_t num_edges, int flags, void* plan_mem, size_t plan_bytes, relm_mp_plan* plan,
              bool wait, hipStream_t s) {
    RELM_TRY(check_rows(key_bound, "num_keys"));
    RELM_TRY(check_rows(num_edges, "num_edges"));
    if (gathers != nullptr) RELM_TRY(check_rows(gather_bound, "num_gather"));
    if (flags & ~RELM_MP_PLAN_SNAPSHOT)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: unknown inverse plan flags");
    const InvLayout l = inv_layout(plan_mem, key_bound, num_edges, flags);
    if (plan_mem == nullptr || plan_bytes < l.bytes)
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: inverse plan memory too small");
    HostSlot* hs = nullptr;
    RELM_TRY(host_slot(&hs));
    RELM_TRY(no_pending(hs));
    std::memset(plan, 0, sizeof(*plan));
    plan->kind = RELM_MP_PLAN_INVERSE;
    plan->num_keys = key_bound;
    plan->num_edges = num_edges;
    plan->num_gather = gather_bound;
    plan->inv = l.inv;
    plan->counts = l.counts;
    plan->collisions = -1;
    SnapOut snap = l.snap;
    if (gathers == nullptr) snap.gathers = snap.gather_plain = nullptr;
    plan->snap_keys = reinterpret_cast<const int32_t*>(snap.keys);
    plan->snap_key_plain = snap.key_plain;
    plan->snap_gathers = reinterpret_cast<const int32_t*>(snap.gathers);
    plan->snap_gather_plain = snap.gather_plain;
    RELM_HIP(launch_status_init(l.status, s), "relm_mp status init");
    RELM_HIP(launch_fill_i32(l.inv, key_bound, -1, s), "relm_mp fill");
    RELM_HIP(launch_inv_build(keys, key_bound, gathers, gather_bound, num_edges, l.inv, snap,
                              l.status, s),
             "relm_mp inverse plan kernel");
    int32_t gen = 0;
    RELM_HIP(hs->publish_status(l.status, l.counts, s, &gen), "relm_mp status publish");
    if (!wait) {
        PendingCheck& p = hs->pending;
        p.active = true;
        p.plan_counts = l.counts;
        p.keys = keys;
        p.key_bound = key_bound;
        p.key_name = key_name != nullptr ? key_name : "index";
        p.gathers = gathers;
        p.gather_bound = gather_bound;
        p.gather_name = gather_name != nullptr ? gather_name : "index";
        p.gather_checked_first = gather_checked_first;
        p.gen = gen;
        p.stream = s;
        return RELM_MP_OK;
    }
    RELM_TRY(wait_host_word(hs->status_gen, gen, s, "relm_mp status wait"));
    const DevStatus host = *hs->status;
    RELM_TRY(check_validation(host, keys, key_bound, key_name, gathers, gather_bound, gather_name,
                              gather_checked_first));
    finish_inverse(plan, host);
    return RELM_MP_OK;
}

// Waits for and reports the pending validation of `plan`, if there is one.
int validate_pending(relm_mp_plan* plan) {
    HostSlot* hs = nullptr;
    RELM_TRY(host_slot(&hs));
    PendingCheck& p = hs->pending;
    if (!p.active || p.plan_counts != plan->counts) return RELM_MP_OK;
    p.active = false;
    RELM_TRY(wait_host_word(hs->status_gen, p.gen, p.stream, "relm_mp status wait"));
    const DevStatus host = *hs->status;
    RELM_TRY(check_validation(host, p.keys, p.key_bound, p.key_name.c_str(), p.gathers,
                              p.gather_bound, p.gather_name.c_str(), p.gather_checked_first));
    finish_inverse(plan, host);
    return RELM_MP_OK;
}

// How a build reads its validation status back: through the calling thread's
// pinned host slot (the status is published right after the first sort pass,
// so the host waits only for that), or with a plain copy after the build
// (no host memory of the library's own: the no-allocation entry point).
enum class StatusPath { kPinnedSlot, kStreamCopy };

int csr_build(const int64_t* keys, int64_t key_bound, const char* key_name, const int64_t* gathers,
              int64_t gather_bound, const char* gather_name, int gather_checked_first,
              int64_t num_edges, void* plan_mem, size_t plan_bytes, void* scratch,
              size_t scratch_bytes, relm_mp_plan* plan, bool wait_counts, hipStream_t s,
              StatusPath path = StatusPath::kPinnedSlot) {
    RELM_TRY(check_rows(key_bound, "num_keys"));
    RELM_TRY(check_rows(num_edges, "num_edges"));
    if (gathers != nullptr) RELM_TRY(check_rows(gather_bound, "num_gather"));
    const CsrLayout l = csr_layout(plan_mem, key_bound, num_edges);
    CsrScratch sc = csr_scratch(scratch, key_bound, num_edges);
    sc.sort.keys_n = l.snap_keys;
    sc.sort.vals_n = l.snap_gathers;
    sc.sort.tile_plain = l.snap_plain;
    if (plan_mem == nullptr || plan_bytes < l.bytes)
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: CSR plan memory too small");
    if (scratch == nullptr || scratch_bytes < sc.bytes)
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: CSR scratch memory too small");
    HostSlot* hs = nullptr;
    if (path == StatusPath::kPinnedSlot) {
        RELM_TRY(host_slot(&hs));
        RELM_TRY(no_pending(hs));
    }
    std::memset(plan, 0, sizeof(*plan));
    plan->kind = RELM_MP_PLAN_CSR;
    plan->hub_threshold = kHubThreshold;
    plan->chunk_size = kChunkSize;
    plan->num_keys = key_bound;
    plan->num_edges = num_edges;
    plan->num_gather = gathers != nullptr ? gather_bound : num_edges;
    plan->offsets = l.offsets;
    plan->gather_sorted = l.gather_sorted;
    plan->hub_key = l.hub_key;
    plan->hub_chunk_base = l.hub_chunk_base;
    plan->chunk_hub = l.chunk_hub;
    plan->multi_hubs = l.multi_hubs;
    plan->item_first = l.item_first;
    plan->item_short = l.item_short;
    plan->short_off = l.short_off;
    plan->short_gather = l.short_gather;
    plan->counts = l.counts;
    plan->snap_keys = reinterpret_cast<const int32_t*>(l.snap_keys);
    plan->snap_key_plain = nullptr;
    plan->snap_gathers = gathers != nullptr ? reinterpret_cast<const int32_t*>(l.snap_gathers) : nullptr;
    plan->snap_gather_plain = gathers != nullptr ? l.snap_plain : nullptr;
    plan->max_degree = plan->num_hubs = plan->num_chunks = plan->num_multi_hubs = -1;
    plan->num_items = plan->num_short = -1;
    const SortZero zero = sort_zero_region(sc.sort, num_edges);
    RELM_HIP(launch_status_init(l.status, s, zero.p, zero.n), "relm_mp status init");
    // The validation result is final after the first sort pass: the pass
    // behind it publishes it to the host, and the rest of the build is
    // enqueued before the host waits for it.
    int32_t status_gen = 0;
    if (num_edges > 0) {
        const StatusPublish pub = hs != nullptr ? hs->publish_target(l.status, &status_gen) : StatusPublish{};
        // short_gather is written by the key index after the sort: until
        // then it holds the sort's intermediate keys
        RELM_HIP(sort_by_key(keys, key_bound, gathers, gather_bound, num_edges, sc.sort,
                             reinterpret_cast<uint32_t*>(l.short_gather),
                             reinterpret_cast<uint32_t*>(l.gather_sorted), l.offsets, l.status, s,
                             pub),
                 "relm_mp radix sort");
    } else {
        RELM_HIP(launch_fill_i32(l.offsets, key_bound + 1, 0, s), "relm_mp offsets fill");
        if (hs != nullptr)
            RELM_HIP(hs->publish_status(l.status, nullptr, s, &status_gen), "relm_mp status copy");
    }
    RELM_HIP(launch_key_index(l.offsets, l.gather_sorted, key_bound, sc.key_index, l.hub_key,
                              l.hub_chunk_base, l.multi_hubs, l.chunk_hub, max_hubs(num_edges),
                              max_chunks(num_edges), l.item_first, l.item_short, l.num_items,
                              l.short_off, l.short_gather, l.counts, l.status, s),
             "relm_mp key index kernels");
    DevStatus host{};
    if (hs != nullptr) {
        RELM_TRY(wait_host_word(hs->status_gen, status_gen, s, "relm_mp status wait"));
        host = *hs->status;
    } else {
        RELM_HIP(hipMemcpyAsync(&host, l.status, sizeof(DevStatus), hipMemcpyDeviceToHost, s),
                 "relm_mp status copy");
        RELM_HIP(hipStreamSynchronize(s), "relm_mp status sync");
    }
    RELM_TRY(check_validation(host, keys, key_bound, key_name, gathers, gather_bound, gather_name,
                              gather_checked_first));
    plan->gather_identity = gathers == nullptr || host.gather_mismatch == 0 ? 1 : 0;
    if (wait_counts) RELM_TRY(read_counts(plan, s));
    return RELM_MP_OK;
}

// Device scratch of relm_mp_fanin_reduce_noalloc (plan, sort buffers and hub
// partials of one call), held by every device the library runs on until the
// process ends.
__device__ __align__(256) unsigned char scratch[RELM_MP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
// Calls of one device run one at a time (host side), and each call's work on
// the device waits for the previous call's through an event recorded behind
// it (events hold no device memory).
std::mutex g_noalloc_mu[kMaxDevices];
hipEvent_t g_noalloc_done[kMaxDevices] = {};
bool g_noalloc_recorded[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call on
// that device).
int noalloc_scratch(void** out) {
    int dev = 0;
    RELM_HIP(hipGetDevice(&dev), "relm_mp device query");
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(RELM_MP_ERR_HIP, "relm_mp: device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        RELM_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "relm_mp scratch address");
        if (ptr == nullptr) return set_error(RELM_MP_ERR_HIP, "relm_mp: scratch address is NULL");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return RELM_MP_OK;
}

}  // namespace

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_error(hipError_t err, const char* what) {
    if (err == hipSuccess) return RELM_MP_OK;
    return set_error(RELM_MP_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

}  // namespace relm_mp

using namespace relm_mp;

extern "C" {

const char* relm_mp_last_error(void) { return g_last_error.c_str(); }

const char* relm_mp_build_info(void) {
    static const std::string info = [] {
        char buf[160];
        std::snprintf(buf, sizeof(buf),
                      "hip=%d.%d;arch=gfx950;plans=inverse,csr;hub_threshold=%d;chunk=%d;item=%d",
                      HIP_VERSION_MAJOR, HIP_VERSION_MINOR, kHubThreshold, kChunkSize, kItemSize);
        return std::string(buf);
    }();
    return info.c_str();
}

size_t relm_mp_inv_plan_bytes(int64_t num_keys, int64_t num_edges, int flags) {
    return inv_layout(nullptr, std::max<int64_t>(num_keys, 0), std::max<int64_t>(num_edges, 0),
                      flags)
        .bytes;
}

int relm_mp_inv_plan_build(const int64_t* keys, int64_t key_bound, const char* key_name,
                           const int64_t* gathers, int64_t gather_bound, const char* gather_name,
                           int gather_checked_first, int64_t num_edges, int flags, void* plan_mem,
                           size_t plan_bytes, relm_mp_plan* plan, relm_mp_stream_t stream) {
    return inv_build(keys, key_bound, key_name, gathers, gather_bound, gather_name,
                     gather_checked_first, num_edges, flags, plan_mem, plan_bytes, plan, true,
                     static_cast<hipStream_t>(stream));
}

int relm_mp_inv_plan_build_async(const int64_t* keys, int64_t key_bound, const char* key_name,
                                 const int64_t* gathers, int64_t gather_bound,
                                 const char* gather_name, int gather_checked_first,
                                 int64_t num_edges, int flags, void* plan_mem, size_t plan_bytes,
                                 relm_mp_plan* plan, relm_mp_stream_t stream) {
    return inv_build(keys, key_bound, key_name, gathers, gather_bound, gather_name,
                     gather_checked_first, num_edges, flags, plan_mem, plan_bytes, plan, false,
                     static_cast<hipStream_t>(stream));
}

int relm_mp_rows_scale(int dtype, const void* in, const int64_t* gather, int div_kind,
                       const int32_t* div_offsets, const int64_t* div_values, const void* base,
                       int64_t rows, int64_t emb, void* out, relm_mp_stream_t stream) {
    if (dtype != RELM_MP_F32 && dtype != RELM_MP_F64)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: dtype must be F32 or F64");
    if (rows < 0 || emb < 0 || div_kind < RELM_MP_DIV_NONE || div_kind > RELM_MP_DIV_VALUES)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: bad row scale arguments");
    if (rows > 0 && emb > 0 &&
        (out == nullptr || (div_kind == RELM_MP_DIV_SEGMENT && div_offsets == nullptr) ||
         (div_kind == RELM_MP_DIV_VALUES && div_values == nullptr)))
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: row scale arrays are NULL");
    return compute_rows_scale(dtype, in, gather, div_kind, div_offsets, div_values, base, rows, emb,
                              out, static_cast<hipStream_t>(stream));
}

size_t relm_mp_plan_match_workspace_size(void) { return kMaxMatch * sizeof(int32_t); }

int relm_mp_plan_match(const int64_t* keys, const int64_t* gathers, int64_t n,
                       const relm_mp_plan* const* plans, int32_t num_plans, int32_t* match,
                       void* workspace, size_t workspace_bytes, relm_mp_stream_t stream) {
    if (n < 0 || num_plans < 0 || num_plans > kMaxMatch || (num_plans > 0 && match == nullptr) ||
        (num_plans > 0 && plans == nullptr))
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: bad plan match arguments");
    if (num_plans == 0) return RELM_MP_OK;
    if (n > 0 && keys == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: keys are NULL");
    const relm_mp_plan* cand[kMaxMatch];
    int32_t slot[kMaxMatch];
    int32_t num = 0;
    for (int32_t c = 0; c < num_plans; ++c) {
        const relm_mp_plan* p = plans[c];
        if (p == nullptr || (p->num_edges > 0 && p->snap_keys == nullptr) ||
            (gathers != nullptr && p->num_edges > 0 && p->snap_gathers == nullptr))
            return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                             "relm_mp: plan without the index snapshot to match");
        match[c] = 0;
        if (p->num_edges != n) continue;  // another length: never equal
        if (n == 0) {
            match[c] = 1;
            continue;
        }
        cand[num] = p;
        slot[num++] = c;
    }
    if (num == 0) return RELM_MP_OK;
    if (workspace == nullptr || workspace_bytes < relm_mp_plan_match_workspace_size() ||
        (reinterpret_cast<uintptr_t>(workspace) & 3u) != 0)
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: plan match workspace missing or too small");
    HostSlot* hs = nullptr;
    RELM_TRY(host_slot(&hs));
    hipStream_t s = static_cast<hipStream_t>(stream);
    int32_t* flags = static_cast<int32_t*>(workspace);
    // a new generation per call (the previous one is still in the host word)
    const int32_t gen = static_cast<int32_t>(static_cast<uint32_t>(hs->match_gen) + 1u);
    hs->match_gen = gen;
    RELM_HIP(launch_plan_match(keys, gathers, n, cand, num, flags, gen, hs->match_mapped, s),
             "relm_mp plan match kernel");
    RELM_TRY(wait_host_word(hs->match + kMaxMatch, gen, s, "relm_mp plan match"));
    for (int32_t j = 0; j < num; ++j) match[slot[j]] = hs->match[j] == gen ? 0 : 1;
    return RELM_MP_OK;
}

static int check_film_ranges(const int64_t* range_start, int32_t num_ranges, int64_t rows) {
    if (num_ranges < 1 || num_ranges > kFilmMaxRanges || range_start == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp film: 1 to 16 row ranges expected");
    if (range_start[0] != 0 || range_start[num_ranges] != rows)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp film: the ranges must cover the rows");
    for (int32_t k = 0; k < num_ranges; ++k)
        if (range_start[k + 1] < range_start[k])
            return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp film: the ranges must be ascending");
    if (relm_mp_film_mish_blocks(range_start, num_ranges) > 0x7fffffff)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp film: too many rows");
    return RELM_MP_OK;
}

int64_t relm_mp_film_mish_blocks(const int64_t* range_start, int32_t num_ranges) {
    if (num_ranges < 1 || num_ranges > kFilmMaxRanges || range_start == nullptr) return -1;
    int64_t blocks = 0;
    for (int32_t k = 0; k < num_ranges; ++k) blocks += film_range_blocks(range_start[k + 1] - range_start[k]);
    return blocks;
}

int relm_mp_film_mish(const float* s, int64_t rows, int64_t width, const int64_t* range_start,
                      int32_t num_ranges, const float* gamma, const float* beta, const float* add,
                      float* y, relm_mp_stream_t stream) {
    RELM_TRY(check_rows(rows, "rows"));
    if (width < 0 || width > 0x7fffffff)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp film: width must be in [0, 2^31).");
    RELM_TRY(check_film_ranges(range_start, num_ranges, rows));
    if (rows == 0 || width == 0) return RELM_MP_OK;
    if (s == nullptr || gamma == nullptr || beta == nullptr || y == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp film: NULL array");
    RELM_HIP(launch_film_mish(s, width, range_start, num_ranges, gamma, beta, add, y,
                              static_cast<hipStream_t>(stream)),
             "relm_mp film kernel");
    return RELM_MP_OK;
}

int relm_mp_film_mish_backward(const float* s, const float* dy, int64_t rows, int64_t width,
                               const int64_t* range_start, int32_t num_ranges, const float* gamma,
                               const float* beta, const float* add, float* ds, double* partial,
                               int64_t partial_blocks, relm_mp_stream_t stream) {
    RELM_TRY(check_rows(rows, "rows"));
    if (width < 0 || width > 0x7fffffff)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp film: width must be in [0, 2^31).");
    RELM_TRY(check_film_ranges(range_start, num_ranges, rows));
    if (rows == 0 || width == 0) return RELM_MP_OK;
    if (partial_blocks < relm_mp_film_mish_blocks(range_start, num_ranges))
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp film: partial sums too small");
    if (s == nullptr || dy == nullptr || gamma == nullptr || beta == nullptr || ds == nullptr ||
        partial == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp film: NULL array");
    RELM_HIP(launch_film_mish_backward(s, dy, width, range_start, num_ranges, gamma, beta, add, ds,
                                       partial, static_cast<hipStream_t>(stream)),
             "relm_mp film backward kernel");
    return RELM_MP_OK;
}

int relm_mp_pack_index(const relm_mp_index_part* parts, int32_t num_parts, int64_t* out_a,
                       int64_t* out_b, relm_mp_stream_t stream) {
    if (num_parts < 0 || (num_parts > 0 && parts == nullptr))
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: bad index parts");
    int64_t total = 0;
    for (int32_t i = 0; i < num_parts; ++i) {
        if (parts[i].n < 0 || (parts[i].n > 0 && (parts[i].a == nullptr ||
                                                   (out_b != nullptr && parts[i].b == nullptr))))
            return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: bad index part");
        total += parts[i].n;
    }
    if (total > 0 && out_a == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: output array is NULL");
    RELM_HIP(launch_pack_index(parts, num_parts, out_a, out_b, static_cast<hipStream_t>(stream)),
             "relm_mp pack kernel");
    return RELM_MP_OK;
}

int relm_mp_plan_validate(relm_mp_plan* plan) {
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    return validate_pending(plan);
}

size_t relm_mp_csr_plan_bytes(int64_t num_keys, int64_t num_edges) {
    return csr_layout(nullptr, std::max<int64_t>(num_keys, 0), std::max<int64_t>(num_edges, 0)).bytes;
}

size_t relm_mp_csr_plan_scratch_bytes(int64_t num_keys, int64_t num_edges) {
    return csr_scratch(nullptr, std::max<int64_t>(num_keys, 0), std::max<int64_t>(num_edges, 0)).bytes;
}

int relm_mp_csr_plan_build(const int64_t* keys, int64_t key_bound, const char* key_name,
                           const int64_t* gathers, int64_t gather_bound, const char* gather_name,
                           int gather_checked_first, int64_t num_edges, void* plan_mem,
                           size_t plan_bytes, void* scratch, size_t scratch_bytes,
                           relm_mp_plan* plan, relm_mp_stream_t stream) {
    return csr_build(keys, key_bound, key_name, gathers, gather_bound, gather_name,
                     gather_checked_first, num_edges, plan_mem, plan_bytes, scratch, scratch_bytes,
                     plan, true, static_cast<hipStream_t>(stream));
}

int relm_mp_csr_plan_build_async(const int64_t* keys, int64_t key_bound, const char* key_name,
                                 const int64_t* gathers, int64_t gather_bound,
                                 const char* gather_name, int gather_checked_first,
                                 int64_t num_edges, void* plan_mem, size_t plan_bytes,
                                 void* scratch, size_t scratch_bytes, relm_mp_plan* plan,
                                 relm_mp_stream_t stream) {
    return csr_build(keys, key_bound, key_name, gathers, gather_bound, gather_name,
                     gather_checked_first, num_edges, plan_mem, plan_bytes, scratch, scratch_bytes,
                     plan, false, static_cast<hipStream_t>(stream));
}

int relm_mp_plan_read_counts(relm_mp_plan* plan, relm_mp_stream_t stream) {
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    return read_counts(plan, static_cast<hipStream_t>(stream));
}

size_t relm_mp_plan_compute_scratch_bytes(const relm_mp_plan* plan, int64_t emb, int dtype,
                                          int64_t mode) {
    if (plan == nullptr) return 0;
    return hub_partial_bytes(*plan, emb, dtype, mode);
}

int relm_mp_plan_gather_last(int dtype, const relm_mp_plan* plan, const int64_t* gathers,
                             const void* table, int64_t emb, void* out, relm_mp_stream_t stream) {
    RELM_TRY(check_dtype(dtype));
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    return compute_gather_last(dtype, *plan, gathers, table, emb, out,
                               static_cast<hipStream_t>(stream));
}

// Checks of a grouped row layout over `rows` rows of emb columns.
static int check_grouped(int64_t rows, int64_t emb, int64_t group, int64_t group_stride) {
    if (emb < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "emb must be >= 0.");
    if (group < 1 || group > RELM_MP_MAX_ROWS)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: group must be >= 1");
    if (group_stride < group * emb)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         "relm_mp: group_stride must be at least group * emb");
    if (rows % group != 0)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         "relm_mp: grouped rows must be a multiple of group");
    return RELM_MP_OK;
}

int relm_mp_plan_gather_last_grouped(int dtype, const relm_mp_plan* plan, const int64_t* gathers,
                                     const void* table, int64_t emb, int64_t group,
                                     int64_t group_stride, void* out, relm_mp_stream_t stream) {
    RELM_TRY(check_dtype(dtype));
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    RELM_TRY(check_grouped(plan->num_keys, emb, group, group_stride));
    return compute_gather_last_grouped(dtype, *plan, gathers, table, emb, group, group_stride, out,
                                       static_cast<hipStream_t>(stream));
}

int relm_mp_plan_segment_sum_grouped(int dtype, const relm_mp_plan* plan, const void* table,
                                     int64_t table_rows, int64_t emb, int64_t group,
                                     int64_t group_stride, void* out, void* scratch,
                                     size_t scratch_bytes, relm_mp_stream_t stream) {
    RELM_TRY(check_dtype(dtype));
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    RELM_TRY(check_grouped(table_rows, emb, group, group_stride));
    if (plan->num_gather > table_rows)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         "relm_mp: the plan gathers beyond table_rows");
    return compute_segment_sum_grouped(dtype, *plan, table, emb, group, group_stride, out, scratch,
                                       scratch_bytes, static_cast<hipStream_t>(stream));
}

int relm_mp_plan_segment_reduce(int dtype, const relm_mp_plan* plan, const int64_t* gathers,
                                const void* table, int64_t emb, int64_t mode, void* out,
                                void* scratch, size_t scratch_bytes, relm_mp_stream_t stream) {
    RELM_TRY(check_dtype(dtype));
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    return compute_segment_reduce(dtype, *plan, gathers, table, emb, mode, out, scratch,
                                  scratch_bytes, static_cast<hipStream_t>(stream));
}

int relm_mp_plan_segment_sum_scaled(int dtype, const relm_mp_plan* plan, const void* table,
                                    int64_t emb, int div_kind, const int64_t* div_values,
                                    const void* base, void* out, void* scratch,
                                    size_t scratch_bytes, relm_mp_stream_t stream) {
    RELM_TRY(check_dtype(dtype));
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    if (emb < 0 || div_kind < RELM_MP_DIV_NONE || div_kind > RELM_MP_DIV_VALUES ||
        (div_kind == RELM_MP_DIV_VALUES && div_values == nullptr && plan->num_keys > 0))
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: bad scaled sum arguments");
    if (base != nullptr && base == out && plan->num_keys > 0 && emb > 0)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: base must not alias out");
    return compute_segment_sum_scaled(dtype, *plan, table, emb, div_kind, div_values, base, out,
                                      scratch, scratch_bytes, static_cast<hipStream_t>(stream));
}

int relm_mp_plan_segment_sum_msgdiv(int dtype, const relm_mp_plan* plan, const void* table,
                                    int64_t emb, const int32_t* msg_div_offsets, const void* base,
                                    void* out, void* scratch, size_t scratch_bytes,
                                    relm_mp_stream_t stream) {
    RELM_TRY(check_dtype(dtype));
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    if (emb < 0 || (msg_div_offsets == nullptr && plan->num_keys > 0 && plan->num_edges > 0))
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: bad divided sum arguments");
    if (base != nullptr && base == out && plan->num_keys > 0 && emb > 0)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: base must not alias out");
    return compute_segment_sum_msgdiv(dtype, *plan, table, emb, msg_div_offsets, base, out, scratch,
                                      scratch_bytes, static_cast<hipStream_t>(stream));
}

int relm_mp_plan_logsumexp_backward(int dtype, const relm_mp_plan* plan, const int64_t* gathers,
                                    const void* grad_out, const void* out, const void* rel_flat,
                                    int64_t emb, void* grad_rel, void* scratch,
                                    size_t scratch_bytes, relm_mp_stream_t stream) {
    RELM_TRY(check_dtype(dtype));
    if (plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    return compute_logsumexp_backward(dtype, *plan, gathers, grad_out, out, rel_flat, emb, grad_rel,
                                      scratch, scratch_bytes, static_cast<hipStream_t>(stream));
}

int relm_mp_plan_fanin_backward_by_dst(int dtype, const relm_mp_plan* dst_plan,
                                       const int64_t* dst_idx, int64_t mode,
                                       const void* grad_out, const void* out,
                                       const void* rel_flat, int64_t emb, void* grad_rel,
                                       int64_t rel_rows, relm_mp_stream_t stream) {
    RELM_TRY(check_dtype(dtype));
    RELM_TRY(check_rows(rel_rows, "rel_rows"));
    if (dst_plan == nullptr) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan is NULL");
    if (emb < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "emb must be >= 0.");
    return compute_backward_by_key(dtype, *dst_plan, dst_idx, mode, grad_out, out, rel_flat, emb,
                                   grad_rel, rel_rows, static_cast<hipStream_t>(stream));
}

int relm_mp_plan_fanin_backward_by_src(int dtype, const relm_mp_plan* dst_plan, int64_t mode,
                                       const void* grad_out, const void* out, const void* rel_flat,
                                       int64_t emb, void* grad_rel, int64_t rel_rows, void* inv_mem,
                                       size_t inv_bytes, int map_ready, int64_t* collisions,
                                       relm_mp_stream_t stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    RELM_TRY(check_dtype(dtype));
    RELM_TRY(check_rows(rel_rows, "rel_rows"));
    if (dst_plan == nullptr || collisions == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: plan or collisions is NULL");
    if (emb < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "emb must be >= 0.");
    if (mode != RELM_MP_MODE_SUM && mode != RELM_MP_MODE_LOGSUMEXP)
        return set_error(RELM_MP_ERR_UNSUPPORTED_MODE,
                         "Unsupported fanin_reduce mode. Supported: 0=sum, 1=logsumexp.");
    const relm_mp_plan& fwd = *dst_plan;
    if (fwd.kind != RELM_MP_PLAN_CSR || fwd.snap_gathers == nullptr || fwd.snap_keys == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         "relm_mp: backward by source needs a CSR plan built with a gather array");
    if (rel_rows < fwd.num_gather)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         "relm_mp: backward by source needs rel_rows >= the plan's num_gather");
    *collisions = 0;
    if (rel_rows == 0 || emb == 0) return RELM_MP_OK;
    const InvLayout l = inv_layout(inv_mem, rel_rows, fwd.num_edges, 0);
    if (inv_mem == nullptr || inv_bytes < l.bytes)
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: inverse plan memory too small");
    relm_mp_plan inv{};
    inv.kind = RELM_MP_PLAN_INVERSE;
    inv.num_keys = rel_rows;
    inv.num_edges = fwd.num_edges;
    inv.num_gather = fwd.num_keys;
    inv.inv = l.inv;
    inv.counts = l.counts;
    inv.collisions = -1;
    if (map_ready != 0)  // the map and its device counts from an earlier call
        return compute_backward_by_src(dtype, fwd, inv, mode, grad_out, out, rel_flat, emb, grad_rel, s);
    HostSlot* hs = nullptr;
    RELM_TRY(host_slot(&hs));
    RELM_TRY(no_pending(hs));
    RELM_HIP(launch_status_init(l.status, s), "relm_mp status init");
    // With as many rows as edges every entry of an injective map is written
    // (and a map that is not injective is not used), and the check reads only
    // entries that some edge of this call wrote: no initial fill.
    if (rel_rows != fwd.num_edges) RELM_HIP(launch_fill_i32(l.inv, rel_rows, -1, s), "relm_mp fill");
    RELM_HIP(launch_inv_from_snapshot(fwd.snap_gathers, fwd.snap_gather_plain, fwd.num_edges, rel_rows,
                                      l.inv, l.status, s),
             "relm_mp inverse map kernels");
    int32_t gen = 0;
    RELM_HIP(hs->publish_status(l.status, l.counts, s, &gen), "relm_mp status publish");
    // queued before the host reads the count: the kernels check it on the device
    RELM_TRY(compute_backward_by_src(dtype, fwd, inv, mode, grad_out, out, rel_flat, emb, grad_rel, s));
    RELM_TRY(wait_host_word(hs->status_gen, gen, s, "relm_mp status wait"));
    *collisions = static_cast<int64_t>(hs->status->collisions);
    return RELM_MP_OK;
}

/* ---- op-level entry points -------------------------------------------- */

size_t relm_mp_fanout_scatter_workspace_size(int64_t num_edges, int64_t out_rows) {
    return relm_mp_inv_plan_bytes(out_rows, num_edges, 0);
}

// mp_ops.cpp:3038-3101 and the CPU loop 2815-2836: per edge the reference
// checks src_global_idx before flat_dst.
int relm_mp_fanout_scatter(int dtype, const void* x_cat, int64_t x_rows, int64_t emb,
                           const int64_t* src_global_idx, const int64_t* flat_dst,
                           int64_t num_edges, int64_t out_rows, void* out, void* workspace,
                           size_t workspace_bytes, relm_mp_stream_t stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    RELM_TRY(check_dtype(dtype));
    RELM_TRY(check_rows(out_rows, "out_rows"));
    RELM_TRY(check_rows(x_rows, "x_rows"));
    RELM_TRY(check_rows(num_edges, "num_edges"));
    if (emb < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "emb must be >= 0.");
    if (num_edges == 0 || out_rows == 0)
        return compute_fill(dtype, out, out_rows * emb, 0.0, s);
    relm_mp_plan plan;
    // the gather is enqueued before the host waits for the index check
    RELM_TRY(inv_build(flat_dst, out_rows, "flat_dst", src_global_idx, x_rows, "src_global_idx", 1,
                       num_edges, 0, workspace, workspace_bytes, &plan, false, s));
    const int rc = compute_gather_last(dtype, plan, src_global_idx, x_cat, emb, out, s);
    const int vrc = validate_pending(&plan);
    return vrc != RELM_MP_OK ? vrc : rc;
}

size_t relm_mp_fanout_scatter_backward_workspace_size(int64_t num_edges, int64_t x_rows,
                                                      int64_t emb, int dtype) {
    const size_t plan = relm_mp_csr_plan_bytes(x_rows, num_edges);
    const size_t scratch = std::max(relm_mp_csr_plan_scratch_bytes(x_rows, num_edges),
                                    hub_partial_upper_bound(num_edges, emb, dtype, RELM_MP_MODE_SUM));
    return plan + scratch;
}

// mp_ops.cpp:3103-3166 and the CPU loop 2838-2861 (src checked first).
int relm_mp_fanout_scatter_backward(int dtype, const void* grad_out, int64_t grad_out_rows,
                                    int64_t emb, const int64_t* src_global_idx,
                                    const int64_t* flat_dst, int64_t num_edges, int64_t x_rows,
                                    void* grad_x, void* workspace, size_t workspace_bytes,
                                    relm_mp_stream_t stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    RELM_TRY(check_dtype(dtype));
    RELM_TRY(check_rows(x_rows, "x_rows"));
    RELM_TRY(check_rows(grad_out_rows, "grad_out_rows"));
    RELM_TRY(check_rows(num_edges, "num_edges"));
    if (emb < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "emb must be >= 0.");
    if (num_edges == 0 || x_rows == 0) return compute_fill(dtype, grad_x, x_rows * emb, 0.0, s);
    const size_t need = relm_mp_fanout_scatter_backward_workspace_size(num_edges, x_rows, emb, dtype);
    if (workspace == nullptr || workspace_bytes < need)
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: workspace too small");
    const size_t plan_bytes = relm_mp_csr_plan_bytes(x_rows, num_edges);
    char* scratch = static_cast<char*>(workspace) + plan_bytes;
    relm_mp_plan plan;
    RELM_TRY(csr_build(src_global_idx, x_rows, "src_global_idx", flat_dst, grad_out_rows, "flat_dst",
                       0, num_edges, workspace, plan_bytes, scratch, workspace_bytes - plan_bytes,
                       &plan, false, s));
    return compute_segment_reduce(dtype, plan, nullptr, grad_out, emb, RELM_MP_MODE_SUM, grad_x,
                                  scratch, workspace_bytes - plan_bytes, s);
}

size_t relm_mp_fanin_reduce_workspace_size(int64_t num_edges, int64_t dim_size, int64_t emb,
                                           int dtype) {
    const size_t plan = relm_mp_csr_plan_bytes(dim_size, num_edges);
    const size_t scratch =
        std::max(relm_mp_csr_plan_scratch_bytes(dim_size, num_edges),
                 hub_partial_upper_bound(num_edges, emb, dtype, RELM_MP_MODE_LOGSUMEXP));
    return plan + scratch;
}

// Checks of relm_mp_fanin_reduce's arguments (the workspace aside).
static int fanin_reduce_checks(int dtype, int64_t rel_rows, int64_t emb, int64_t num_edges,
                               int64_t dim_size, int64_t mode) {
    RELM_TRY(check_dtype(dtype));
    RELM_TRY(check_rows(dim_size, "dim_size"));
    RELM_TRY(check_rows(rel_rows, "rel_rows"));
    RELM_TRY(check_rows(num_edges, "num_edges"));
    if (emb < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "emb must be >= 0.");
    if (mode != RELM_MP_MODE_SUM && mode != RELM_MP_MODE_LOGSUMEXP)
        return set_error(RELM_MP_ERR_UNSUPPORTED_MODE,
                         "Unsupported fanin_reduce mode. Supported: 0=sum, 1=logsumexp.");
    return RELM_MP_OK;
}

// The body of relm_mp_fanin_reduce once the workspace is known to suffice.
static int fanin_reduce_run(int dtype, const void* rel_flat, int64_t rel_rows, int64_t emb,
                            const int64_t* flat_src, const int64_t* dst_idx, int64_t num_edges,
                            int64_t dim_size, int64_t mode, void* out, void* workspace,
                            size_t workspace_bytes, hipStream_t s, StatusPath path) {
    const double empty = mode == RELM_MP_MODE_SUM ? 0.0 : -__builtin_huge_val();
    if (num_edges == 0 || dim_size == 0) return compute_fill(dtype, out, dim_size * emb, empty, s);
    const size_t plan_bytes = relm_mp_csr_plan_bytes(dim_size, num_edges);
    char* scratch = static_cast<char*>(workspace) + plan_bytes;
    relm_mp_plan plan;
    RELM_TRY(csr_build(dst_idx, dim_size, "dst_idx", flat_src, rel_rows, "flat_src", 1, num_edges,
                       workspace, plan_bytes, scratch, workspace_bytes - plan_bytes, &plan, false, s,
                       path));
    return compute_segment_reduce(dtype, plan, nullptr, rel_flat, emb, mode, out, scratch,
                                  workspace_bytes - plan_bytes, s);
}

// mp_ops.cpp:3327-3348 (mode router), 3168-3222 (sum), 3005-3036 (logsumexp);
// the sum CPU loop 2863-2886 checks flat_src before dst_idx.
int relm_mp_fanin_reduce(int dtype, const void* rel_flat, int64_t rel_rows, int64_t emb,
                         const int64_t* flat_src, const int64_t* dst_idx, int64_t num_edges,
                         int64_t dim_size, int64_t mode, void* out, void* workspace,
                         size_t workspace_bytes, relm_mp_stream_t stream) {
    RELM_TRY(fanin_reduce_checks(dtype, rel_rows, emb, num_edges, dim_size, mode));
    if (num_edges > 0 && dim_size > 0) {
        const size_t need = relm_mp_fanin_reduce_workspace_size(num_edges, dim_size, emb, dtype);
        if (workspace == nullptr || workspace_bytes < need)
            return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: workspace too small");
    }
    return fanin_reduce_run(dtype, rel_flat, rel_rows, emb, flat_src, dst_idx, num_edges, dim_size,
                            mode, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                            StatusPath::kPinnedSlot);
}

// relm_mp_fanin_reduce on the library's own device scratch: the array below,
// one copy per device.  Host code never passes its name to a kernel or a copy
// (there it names a host-side stand-in); the device address comes from
// hipGetSymbolAddress, looked up once per device with that device current.
int relm_mp_fanin_reduce_noalloc(int dtype, const void* rel_flat, int64_t rel_rows, int64_t emb,
                                 const int64_t* flat_src, const int64_t* dst_idx,
                                 int64_t num_edges, int64_t dim_size, int64_t mode, void* out,
                                 relm_mp_stream_t stream) {
    RELM_TRY(fanin_reduce_checks(dtype, rel_rows, emb, num_edges, dim_size, mode));
    void* ws = nullptr;
    if (num_edges > 0 && dim_size > 0) {
        const size_t need = relm_mp_fanin_reduce_workspace_size(num_edges, dim_size, emb, dtype);
        if (need > static_cast<size_t>(RELM_MP_NOALLOC_SCRATCH_BYTES)) {
            char buf[256];
            std::snprintf(buf, sizeof(buf),
                          "relm_mp_fanin_reduce_noalloc: this call needs %zu bytes of scratch, more "
                          "than the %lld the library reserves per device; use "
                          "relm_mp_fanin_reduce with a workspace",
                          need, static_cast<long long>(RELM_MP_NOALLOC_SCRATCH_BYTES));
            return set_error(RELM_MP_ERR_WORKSPACE, buf);
        }
        RELM_TRY(noalloc_scratch(&ws));
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    int dev = 0;
    RELM_HIP(hipGetDevice(&dev), "relm_mp device query");
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(RELM_MP_ERR_HIP, "relm_mp: device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_noalloc_mu[dev]);
    if (g_noalloc_done[dev] == nullptr)
        RELM_HIP(hipEventCreateWithFlags(&g_noalloc_done[dev], hipEventDisableTiming),
                 "relm_mp noalloc event");
    if (g_noalloc_recorded[dev])
        RELM_HIP(hipStreamWaitEvent(s, g_noalloc_done[dev], 0), "relm_mp noalloc wait");
    const int rc = fanin_reduce_run(dtype, rel_flat, rel_rows, emb, flat_src, dst_idx, num_edges,
                                    dim_size, mode, out, ws,
                                    static_cast<size_t>(RELM_MP_NOALLOC_SCRATCH_BYTES), s,
                                    StatusPath::kStreamCopy);
    // recorded whatever the outcome: kernels of a failed call may still be queued
    const hipError_t rec = hipEventRecord(g_noalloc_done[dev], s);
    if (rec == hipSuccess) g_noalloc_recorded[dev] = true;
    if (rc != RELM_MP_OK) return rc;
    return hip_error(rec, "relm_mp noalloc event record");
}

size_t relm_mp_fanin_reduce_sum_backward_workspace_size(int64_t num_edges, int64_t rel_rows,
                                                        int64_t emb, int dtype) {
    const size_t inv = relm_mp_inv_plan_bytes(rel_rows, num_edges, 0);
    const size_t plan = relm_mp_csr_plan_bytes(rel_rows, num_edges);
    const size_t scratch = std::max(relm_mp_csr_plan_scratch_bytes(rel_rows, num_edges),
                                    hub_partial_upper_bound(num_edges, emb, dtype, RELM_MP_MODE_SUM));
    return inv + plan + scratch;
}

// mp_ops.cpp:3224-3284 and the CPU loop 2888-2911 (flat_src checked first).
int relm_mp_fanin_reduce_sum_backward(int dtype, const void* grad_out, int64_t grad_out_rows,
                                      int64_t emb, const int64_t* flat_src,
                                      const int64_t* dst_idx, int64_t num_edges,
                                      int64_t rel_rows, void* grad_rel, void* workspace,
                                      size_t workspace_bytes, relm_mp_stream_t stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    RELM_TRY(check_dtype(dtype));
    RELM_TRY(check_rows(rel_rows, "rel_rows"));
    RELM_TRY(check_rows(grad_out_rows, "grad_out_rows"));
    RELM_TRY(check_rows(num_edges, "num_edges"));
    if (emb < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "emb must be >= 0.");
    if (num_edges == 0 || rel_rows == 0) return compute_fill(dtype, grad_rel, rel_rows * emb, 0.0, s);
    const size_t need = relm_mp_fanin_reduce_sum_backward_workspace_size(num_edges, rel_rows, emb, dtype);
    if (workspace == nullptr || workspace_bytes < need)
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: workspace too small");
    const size_t inv_bytes = relm_mp_inv_plan_bytes(rel_rows, num_edges, 0);
    relm_mp_plan plan;
    RELM_TRY(inv_build(flat_src, rel_rows, "flat_src", dst_idx, grad_out_rows, "dst_idx", 0,
                       num_edges, 0, workspace, inv_bytes, &plan, true, s));
    if (plan.collisions == 0)
        return compute_gather_last(dtype, plan, dst_idx, grad_out, emb, grad_rel, s);
    char* csr_mem = static_cast<char*>(workspace) + inv_bytes;
    const size_t plan_bytes = relm_mp_csr_plan_bytes(rel_rows, num_edges);
    char* scratch = csr_mem + plan_bytes;
    const size_t scratch_bytes = workspace_bytes - inv_bytes - plan_bytes;
    RELM_TRY(csr_build(flat_src, rel_rows, "flat_src", dst_idx, grad_out_rows, "dst_idx", 0,
                       num_edges, csr_mem, plan_bytes, scratch, scratch_bytes, &plan, false, s));
    return compute_segment_reduce(dtype, plan, nullptr, grad_out, emb, RELM_MP_MODE_SUM, grad_rel,
                                  scratch, scratch_bytes, s);
}

size_t relm_mp_fanin_reduce_logsumexp_backward_workspace_size(int64_t num_edges, int64_t rel_rows,
                                                              int64_t emb, int dtype) {
    return relm_mp_fanin_reduce_sum_backward_workspace_size(num_edges, rel_rows, emb, dtype);
}

// mp_ops.cpp:3286-3325 and the ATen sequence 2981-3003.
int relm_mp_fanin_reduce_logsumexp_backward(int dtype, const void* grad_out, int64_t dim_size,
                                            int64_t emb, const void* rel_flat,
                                            int64_t rel_flat_rows, const int64_t* flat_src,
                                            const int64_t* dst_idx, int64_t num_edges,
                                            const void* out, int64_t rel_rows, void* grad_rel,
                                            void* workspace, size_t workspace_bytes,
                                            relm_mp_stream_t stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    RELM_TRY(check_dtype(dtype));
    RELM_TRY(check_rows(rel_rows, "rel_rows"));
    RELM_TRY(check_rows(rel_flat_rows, "rel_flat rows"));
    RELM_TRY(check_rows(dim_size, "dim_size"));
    RELM_TRY(check_rows(num_edges, "num_edges"));
    if (emb < 0) return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "emb must be >= 0.");
    if (num_edges == 0 || rel_rows == 0) return compute_fill(dtype, grad_rel, rel_rows * emb, 0.0, s);
    const size_t need =
        relm_mp_fanin_reduce_logsumexp_backward_workspace_size(num_edges, rel_rows, emb, dtype);
    if (workspace == nullptr || workspace_bytes < need)
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: workspace too small");
    // A message row is read from rel_flat and its gradient written to grad_rel,
    // so flat_src must index both.
    const int64_t key_bound = std::min(rel_rows, rel_flat_rows);
    // Rows [key_bound, rel_rows) of grad_rel cannot receive messages.
    const size_t elem = dtype == RELM_MP_F64 ? 8 : 4;
    if (key_bound < rel_rows) {
        RELM_TRY(compute_fill(dtype, static_cast<char*>(grad_rel) + key_bound * emb * elem,
                              (rel_rows - key_bound) * emb, 0.0, s));
    }
    const size_t inv_bytes = relm_mp_inv_plan_bytes(rel_rows, num_edges, 0);
    relm_mp_plan plan;
    RELM_TRY(inv_build(flat_src, key_bound, "flat_src", dst_idx, dim_size, "dst_idx", 1, num_edges,
                       0, workspace, inv_bytes, &plan, true, s));
    if (plan.collisions == 0)
        return compute_logsumexp_backward(dtype, plan, dst_idx, grad_out, out, rel_flat, emb,
                                          grad_rel, nullptr, 0, s);
    char* csr_mem = static_cast<char*>(workspace) + inv_bytes;
    const size_t plan_bytes = relm_mp_csr_plan_bytes(rel_rows, num_edges);
    char* scratch = csr_mem + plan_bytes;
    const size_t scratch_bytes = workspace_bytes - inv_bytes - plan_bytes;
    RELM_TRY(csr_build(flat_src, key_bound, "flat_src", dst_idx, dim_size, "dst_idx", 1, num_edges,
                       csr_mem, plan_bytes, scratch, scratch_bytes, &plan, false, s));
    return compute_logsumexp_backward(dtype, plan, nullptr, grad_out, out, rel_flat, emb, grad_rel,
                                      scratch, scratch_bytes, s);
}

}  // extern "C"
