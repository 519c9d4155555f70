// Row kernels of the relational message-passing ops.
//
// Every output row is owned by exactly one "row group" of G lanes (G = 4..64,
// a divisor of the wave), each lane moving V contiguous elements (float4 /
// double2 when the rows allow it); rows wider than G*V are split over
// blockIdx.y slices.  No atomics anywhere: the messages of a key are visited
// in the stable (edge) order of the plan, so every result is deterministic.
//
// CSR plans are reduced in two parts:
//  * segments of at most kHubThreshold messages: k_walk_items.  Key k weighs
//    1 + its short message count and item j holds the keys whose prefix weight
//    lies in [j*kItemSize, (j+1)*kItemSize), so every row group gets a similar
//    amount of work; the group walks its keys in order, each key's messages
//    sequentially in edge order, which makes the fp32 sums bit-identical to the
//    reference's sequential CPU loop.  A workgroup stages the short offsets and
//    gathered indices of its items in LDS first, leaving one memory round trip
//    per batch of message rows.
//  * hubs: k_hub_chunks, one workgroup per chunk of kChunkSize messages; each
//    row group folds a contiguous slice, the slices are folded as a fixed tree.
//    Single-chunk hubs are finished there; the others leave chunk partials that
//    k_hub_combine (one workgroup per hub) folds the same way.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "device_utils.h"
#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kThreads = 256;
// Rows per row group per iteration of the inverse-plan row kernels, the best
// of 1..8 measured: the gather of 16-byte lanes (C3, D = 64; edge order,
// D = 32) keeps 2 rows in flight, of narrower lanes (argument slots of 128
// columns at an 8-byte aligned offset) 8; the logsumexp backward, which
// reads three rows per row, 4.
template <typename T, int V>
constexpr int gather_rows_in_flight() { return sizeof(T) * V >= 16 ? 2 : 8; }
constexpr int kLseRowsInFlight = 4;
constexpr int64_t kMaxBlocksX = 1 << 22;  // keeps blocks * 1024 threads below 2^32
// Largest pair of arrays read into the memory-side cache (256 MB on MI355X)
// ahead of a write-dominated kernel.
constexpr size_t kPrefetchMaxBytes = size_t(256) << 20;

template <int G>
constexpr int batch_rows() {
    return G < 8 ? G : 8;
}

// Element offset of row `row` (a valid row index, below 2^31) of a table of
// D columns: one unsigned 32 x 32 -> 64 multiply instead of a signed 64-bit one.
__device__ __forceinline__ uint64_t row_offset(int64_t row, int64_t D) {
    return static_cast<uint64_t>(static_cast<uint32_t>(row)) *
           static_cast<uint64_t>(static_cast<uint32_t>(D));
}

// Row layouts of a table or an output.  DenseRows: row r at r * D.
// GroupedRows: rows in groups of `group` consecutive rows per line of a wider
// matrix, row r at (r / group) * stride + (r % group) * D - the argument
// columns of a [nodes, width] input matrix with `group` slots per node
// (stride = width, the base pointer at the first argument column).
struct DenseRows {
    __device__ __forceinline__ uint64_t operator()(int64_t row, int64_t D) const {
        return row_offset(row, D);
    }
};

struct GroupedRows {
    uint32_t group;
    uint64_t stride;
    __device__ __forceinline__ uint64_t operator()(int64_t row, int64_t D) const {
        const uint32_t r = static_cast<uint32_t>(row);
        const uint32_t q = r / group;
        return static_cast<uint64_t>(q) * stride +
               static_cast<uint64_t>(r - q * group) * static_cast<uint32_t>(D);
    }
};

template <typename T, int V>
__device__ __forceinline__ void pack_add(Pack<T, V>& a, const Pack<T, V>& b) {
#pragma unroll
    for (int i = 0; i < V; ++i) a.v[i] = a.v[i] + b.v[i];
}

// ---- partial results -----------------------------------------------------

template <typename T, int V>
struct SumPartial {
    Pack<T, V> a;
    static constexpr int kWords = 1;  // Packs per stored partial
    __device__ __forceinline__ static SumPartial identity() { return {pack_fill<T, V>(T(0))}; }
    __device__ __forceinline__ void merge(const SumPartial& o) { pack_add(a, o.a); }
    __device__ __forceinline__ void store(T* p, int64_t D, int64_t col) const { pack_store<T, V>(p + col, a); }
    __device__ __forceinline__ static SumPartial load(const T* p, int64_t D, int64_t col) {
        return {pack_load<T, V>(p + col)};
    }
    __device__ __forceinline__ Pack<T, V> value() const { return a; }
    __device__ __forceinline__ SumPartial shfl_down(int d) const {
        SumPartial r;
#pragma unroll
        for (int i = 0; i < V; ++i) r.a.v[i] = __shfl_down(a.v[i], d, kWave);
        return r;
    }
};

// (m, s): maximum of the messages and the sum of exp(x - m); s is NaN when a
// message was NaN.  Merging rescales both sums to the larger maximum.
template <typename T, int V>
struct LsePartial {
    Pack<T, V> m;
    Pack<T, V> s;
    static constexpr int kWords = 2;
    __device__ __forceinline__ static LsePartial identity() {
        return {pack_fill<T, V>(neg_inf<T>()), pack_fill<T, V>(T(0))};
    }
    __device__ __forceinline__ void merge(const LsePartial& o) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const T M = max_num(m.v[i], o.m.v[i]);
            if (M == neg_inf<T>()) {
                s.v[i] = (s.v[i] != s.v[i]) ? s.v[i] : (o.s.v[i] != o.s.v[i] ? o.s.v[i] : T(0));
            } else {
                s.v[i] = s.v[i] * fast_exp<T>(m.v[i] - M) + o.s.v[i] * fast_exp<T>(o.m.v[i] - M);
            }
            m.v[i] = M;
        }
    }
    __device__ __forceinline__ void store(T* p, int64_t D, int64_t col) const {
        pack_store<T, V>(p + col, m);
        pack_store<T, V>(p + D + col, s);
    }
    __device__ __forceinline__ static LsePartial load(const T* p, int64_t D, int64_t col) {
        return {pack_load<T, V>(p + col), pack_load<T, V>(p + D + col)};
    }
    // Result of a non-empty segment.
    __device__ __forceinline__ Pack<T, V> value() const {
        Pack<T, V> r;
#pragma unroll
        for (int i = 0; i < V; ++i)
            r.v[i] = m.v[i] == neg_inf<T>() ? quiet_nan<T>() : dev_log<T>(s.v[i]) + m.v[i];
        return r;
    }
    __device__ __forceinline__ LsePartial shfl_down(int d) const {
        LsePartial r;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            r.m.v[i] = __shfl_down(m.v[i], d, kWave);
            r.s.v[i] = __shfl_down(s.v[i], d, kWave);
        }
        return r;
    }
};

// ---- ops: what is accumulated per message ----------------------------------

// Sum of table rows.
template <typename T, int V, int U, class Rows = DenseRows>
struct SumOp {
    using Partial = SumPartial<T, V>;
    const T* __restrict__ table;
    int64_t D;
    int64_t col;
    bool colok;
    int64_t lcol;  // column the lane loads: col, or 0 past the row (value unused)
    Pack<T, V> x[U];
    Pack<T, V> acc;
    Rows rows;  // layout of the table rows

    // The walker starts each segment by reset() after storing the previous one.
    static constexpr bool kResetAtEnd = true;
    __device__ __forceinline__ void reset() { acc = pack_fill<T, V>(T(0)); }
    __device__ __forceinline__ void begin(int64_t, bool) { acc = pack_fill<T, V>(T(0)); }
    // Starts a new segment when `head` (branch-free).
    __device__ __forceinline__ void restart(bool head, int64_t) {
#pragma unroll
        for (int i = 0; i < V; ++i) acc.v[i] = head ? T(0) : acc.v[i];
    }
    // Callers pass valid rows past `cnt` (the last valid index repeated, or
    // the next messages), and lanes past the row read its first columns, so
    // every load is unconditional: the compiler keeps all U in flight and
    // waits for each only where it is consumed.  Rows past `cnt` are never
    // accumulated, lanes past the row never stored.
    __device__ __forceinline__ void load(const int32_t (&idx)[U], int) {
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = pack_load<T, V>(table + rows(idx[u], D) + lcol);
    }
    // Rows u >= cnt (or !valid) leave the accumulator as it is: selects, not
    // branches, so the loads stay unconditional.
    __device__ __forceinline__ void consume(int cnt) {
#pragma unroll
        for (int u = 0; u < U; ++u) add(u, u < cnt);
    }
    __device__ __forceinline__ void add(int u, bool valid) {
#pragma unroll
        for (int i = 0; i < V; ++i) acc.v[i] = valid ? acc.v[i] + x[u].v[i] : acc.v[i];
    }
    __device__ __forceinline__ Pack<T, V> result(bool) const { return acc; }
    __device__ __forceinline__ Pack<T, V> empty() const { return pack_fill<T, V>(T(0)); }
    __device__ __forceinline__ Partial partial() const { return {acc}; }
};

// Sum of table rows, each divided by its own row's message count before it
// is added: row g contributes table[g] / d_g, d_g = max(1, div_offsets[g + 1] -
// div_offsets[g]) (the offsets of a CSR plan keyed by the table's rows).  The
// transposed mean of the LGAN aggregations, which divide every gathered
// gradient row by its count and then add (mp_ops.cpp:3548-3557); the counts
// are loaded with the rows, so no divided copy of the table is written.
template <typename T, int V, int U>
struct SumDivOp : SumOp<T, V, U> {
    const int32_t* __restrict__ div_offsets;
    T d[U];

    __device__ __forceinline__ void load(const int32_t (&idx)[U], int cnt) {
        SumOp<T, V, U>::load(idx, cnt);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int32_t n = div_offsets[idx[u] + 1] - div_offsets[idx[u]];
            d[u] = n > 1 ? static_cast<T>(n) : T(1);
        }
    }
    __device__ __forceinline__ void consume(int cnt) {
#pragma unroll
        for (int u = 0; u < U; ++u) add(u, u < cnt);
    }
    __device__ __forceinline__ void add(int u, bool valid) {
#pragma unroll
        for (int i = 0; i < V; ++i)
            this->acc.v[i] = valid ? this->acc.v[i] + this->x[u].v[i] / d[u] : this->acc.v[i];
    }
};

// Logsumexp of table rows as a blocked max-then-sum: per batch the batch
// maximum first, then exp(x - max) summed against the running maximum (s is
// kept relative to m and rescaled when m grows).  Semantics of the reference's
// amax / exp / sum / log sequence: a NaN message makes the result NaN (s
// becomes NaN: through exp(NaN - m), or explicitly while m is still -inf,
// because the maximum ignores NaN), messages that are all -inf give NaN, an
// empty segment -inf.
template <typename T, int V, int U>
struct LseOp {
    using Partial = LsePartial<T, V>;
    const T* __restrict__ table;
    int64_t D;
    int64_t col;
    bool colok;
    int64_t lcol;  // as SumOp::lcol
    Pack<T, V> x[U];
    Pack<T, V> m, s;

    __device__ __forceinline__ void begin(int64_t, bool) {
        m = pack_fill<T, V>(neg_inf<T>());
        s = pack_fill<T, V>(T(0));
    }
    // The walker's segments (reset / add / result) start m at the lowest
    // finite value instead of -inf: a -inf message then gives exp(-inf) = 0
    // with no guard (m - x is never -inf - -inf), and a first finite message
    // still sets s = fma(0, e, 1) = 1 exactly.
    static constexpr bool kResetAtEnd = true;
    __device__ __forceinline__ void reset() {
        m = pack_fill<T, V>(lowest<T>());
        s = pack_fill<T, V>(T(0));
    }
    __device__ __forceinline__ void restart(bool head, int64_t) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
            m.v[i] = head ? lowest<T>() : m.v[i];
            s.v[i] = head ? T(0) : s.v[i];
        }
    }
    // as SumOp::load
    __device__ __forceinline__ void load(const int32_t (&idx)[U], int) {
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = pack_load<T, V>(table + row_offset(idx[u], D) + lcol);
    }
    // Batch maximum, then the rescaled sum; rows u >= cnt are masked by
    // selects (no branch, so the loads stay unconditional).  While the maximum
    // is -inf (messages -inf or NaN only) m stays -inf and a NaN message
    // makes s NaN.
    __device__ __forceinline__ void consume(int cnt) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
            T mb = neg_inf<T>();
#pragma unroll
            for (int u = 0; u < U; ++u) mb = u < cnt ? max_num(mb, x[u].v[i]) : mb;
            const T nm = max_num(m.v[i], mb);
            T acc = s.v[i] * fast_exp<T>(m.v[i] - nm);
            T snan = s.v[i];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                acc = u < cnt ? acc + fast_exp<T>(x[u].v[i] - nm) : acc;
                snan = (u < cnt && x[u].v[i] != x[u].v[i]) ? quiet_nan<T>() : snan;
            }
            const bool fin = nm != neg_inf<T>();
            s.v[i] = fin ? acc : snan;
            m.v[i] = fin ? nm : m.v[i];
        }
    }
    // One message at a time (segments whose batches mix keys): the running
    // maximum only moves up, so each message costs one exp.  An invalid row
    // (past the batch) changes nothing.
    __device__ __forceinline__ void add(int u, bool valid) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
            // exp(-|x - m|) is exp(m - x) when x raises the maximum, exp(x - m)
            // otherwise; m is finite or +inf, so a -inf message adds exp(-inf)
            // = 0 and a NaN message makes s NaN
            const T xv = x[u].v[i];
            const bool up = valid && xv > m.v[i];
            const T d = xv - m.v[i];
            const T e = fast_exp<T>(-fabs(d));
            const T sn = up ? fma(s.v[i], e, T(1)) : s.v[i] + e;
            s.v[i] = valid ? sn : s.v[i];
            m.v[i] = up ? xv : m.v[i];
        }
    }
    // Result of a walked segment.  A +inf message makes the reference's
    // exp(x - max) NaN; so does a NaN message or a segment of -inf only.
    // Those are exactly the cases where log(s) + m is infinite (m = +inf, or
    // s = 0 with m the lowest finite value): otherwise m is finite and
    // 1 <= s <= 65, so m + log(s) cannot round to an infinity.
    __device__ __forceinline__ Pack<T, V> result(bool) const {
        Pack<T, V> r;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const T v = log_add<T>(s.v[i], m.v[i]);
            r.v[i] = __builtin_isinf(v) ? quiet_nan<T>() : v;
        }
        return r;
    }
    __device__ __forceinline__ Pack<T, V> empty() const { return pack_fill<T, V>(neg_inf<T>()); }
    __device__ __forceinline__ Partial partial() const { return Partial{m, s}; }
};

// Logsumexp backward of key r (= a rel row): sum over its messages of
// grad_out[d] * exp(rel[r] - out[d]), d the gathered row, in edge order.
template <typename T, int V, int U>
struct LseBwdOp {
    using Partial = SumPartial<T, V>;
    // a segment starts by loading its key's rel row: restart() at its head
    static constexpr bool kResetAtEnd = false;
    const T* __restrict__ grad_out;
    const T* __restrict__ out;
    const T* __restrict__ rel;
    int64_t D;
    int64_t col;
    bool colok;
    int64_t lcol;  // as SumOp::lcol
    Pack<T, V> g[U], o[U];
    Pack<T, V> xr, acc;

    // key is a valid rel row (hub chunks outside the plan pass row 0)
    __device__ __forceinline__ void begin(int64_t key, bool) {
        acc = pack_fill<T, V>(T(0));
        xr = pack_load<T, V>(rel + key * D + lcol);
    }
    __device__ __forceinline__ void restart(bool head, int64_t key) {
        if (head) begin(key, true);
    }
    // as SumOp::load
    __device__ __forceinline__ void load(const int32_t (&idx)[U], int) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t off = row_offset(idx[u], D) + lcol;
            g[u] = pack_load<T, V>(grad_out + off);
            o[u] = pack_load<T, V>(out + off);
        }
    }
    __device__ __forceinline__ void consume(int cnt) {
#pragma unroll
        for (int u = 0; u < U; ++u) add(u, u < cnt);
    }
    __device__ __forceinline__ void add(int u, bool valid) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const T w = fast_exp<T>(xr.v[i] - o[u].v[i]);
            const T c = g[u].v[i] * w;
            acc.v[i] = valid ? acc.v[i] + c : acc.v[i];
        }
    }
    __device__ __forceinline__ Pack<T, V> result(bool) const { return acc; }
    __device__ __forceinline__ Pack<T, V> empty() const { return pack_fill<T, V>(T(0)); }
    __device__ __forceinline__ Partial partial() const { return {acc}; }
};

// ---- epilogues: applied to each key's result as it is stored ----------------

// Stores the result as is.
// Minimum waves per SIMD asked of the compiler for the walker and the hub
// chunks (HIP's second launch bound), which caps their VGPRs: the fp32 sum and
// logsumexp over dense rows fit 96 VGPRs in the walker (5 waves instead of 4 at
// 116) and 80 in the hub chunks (6 instead of 5 at 93) without spilling; the
// other ops (fp64, grouped rows, the logsumexp backward) would spill, and keep
// the compiler's choice.
template <class Op>
struct WaveFloor {
    static constexpr int walk = 1;
    static constexpr int hub = 1;
};
template <int V, int U>
struct WaveFloor<SumOp<float, V, U, DenseRows>> {
    static constexpr int walk = 5;
    static constexpr int hub = 6;
};
template <int V, int U>
struct WaveFloor<LseOp<float, V, U>> {
    static constexpr int walk = 5;
    static constexpr int hub = 6;
};

struct NoEpilogue {
    template <typename T, int V>
    __device__ __forceinline__ Pack<T, V> operator()(int64_t, const Pack<T, V>& v, int64_t,
                                                     int64_t) const {
        return v;
    }
};

// base[key] + result / d_key, d_key = max(1, segment size) or max(1,
// (T)values[key]) (relm_mp_plan_segment_sum_scaled).  The division and the
// addition round separately; `base` must not alias the output (hub keys are
// written twice).
template <typename T>
struct ScaleEpilogue {
    const T* __restrict__ base;
    int div_kind;
    const int32_t* __restrict__ offsets;
    const int64_t* __restrict__ values;

    template <int V>
    __device__ __forceinline__ Pack<T, V> operator()(int64_t key, const Pack<T, V>& v, int64_t D,
                                                     int64_t col) const {
        Pack<T, V> r = v;
        if (div_kind != RELM_MP_DIV_NONE) {
            T d = T(1);
            if (div_kind == RELM_MP_DIV_SEGMENT) {
                const int32_t n = offsets[key + 1] - offsets[key];
                d = n > 1 ? static_cast<T>(n) : T(1);
            } else {
                const T x = static_cast<T>(values[key]);
                d = x > T(1) ? x : T(1);
            }
#pragma unroll
            for (int i = 0; i < V; ++i) r.v[i] = r.v[i] / d;
        }
        if (base != nullptr) {
            const Pack<T, V> b = pack_load<T, V>(base + key * D + col);
#pragma unroll
            for (int i = 0; i < V; ++i) r.v[i] = b.v[i] + r.v[i];
        }
        return r;
    }
};

// ---- shared walking helpers -------------------------------------------------

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

// ---- kernels -------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(kThreads) void k_fill(T* __restrict__ p, int64_t n, T value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        p[i] = value;
}

// Keys with at most kHubThreshold messages, walked item by item.  A workgroup
// takes R consecutive items, one per row group.  Their keys are consecutive and
// so are their short segments (short_gather leaves the hub segments out), so
// the workgroup first stages its short offsets and gathered row indices in LDS
// with coalesced loads, and labels every staged message with its key (the
// segment heads are marked, then a block-wide running maximum fills the
// labels in).  Keys without short messages (empty segments and hubs) get the
// empty-segment result from a block-wide pass: hub rows are written again by
// the hub kernels, which run after this one on the same stream.  Each group
// then feeds its item's messages in batches of U in edge order; a message
// whose label differs from the previous one restarts the accumulator and one
// whose label differs from the next one stores its key's result - no
// per-key loop, so the row groups of a wave stay in step.
template <typename T, int V, int G, class Op, class Epi>
__global__ __launch_bounds__(kThreads, WaveFloor<Op>::walk) void k_walk_items(
    const int32_t* __restrict__ short_off, const int32_t* __restrict__ short_gather_in,
    const int32_t* __restrict__ gather_sorted, const int32_t* __restrict__ item_first,
    const int32_t* __restrict__ item_short, const relm_mp_plan_counts* __restrict__ pc,
    int64_t num_keys, T* __restrict__ out, Op op, Epi epi) {
    constexpr int R = kThreads / G;
    constexpr int U = batch_rows<G>();
    // R items hold at most R * kItemSize keys and R * kItemSize + kHubThreshold
    // short messages (the last key may weigh up to kHubThreshold + 1)
    constexpr int kKeyCap = R * kItemSize + 2;
    constexpr int kPosCap = R * kItemSize + kHubThreshold + 1;
    constexpr int PI = (kPosCap + kThreads - 1) / kThreads;  // staged positions per thread
    constexpr int KI = (kKeyCap + kThreads - 1) / kThreads;
    // a batch reads U + 1 positions from any message of an item on: the
    // staged range is followed by at least U + 1 padding positions
    static_assert(kThreads * PI >= kPosCap + U + 1, "walker staging leaves no padding");
    constexpr uint16_t kNoLabel = 0xFFFF;  // label of the padding (keys are < kKeyCap)
    static_assert(kKeyCap < kNoLabel, "walker labels fit 16 bits");
    __shared__ int32_t s_off[kKeyCap];
    __shared__ int32_t s_idx[kThreads * PI];   // gathered rows; row 0 as padding
    __shared__ uint16_t s_key[kThreads * PI];  // labels; thread t scans [t * PI, t * PI + PI)
    __shared__ uint32_t s_scan[kThreads / kWave];
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int grp = static_cast<int>(threadIdx.x) / G;
    op.col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    op.colok = op.col < op.D;
    op.lcol = op.colok ? op.col : 0;
    const int64_t D = op.D;
    const int64_t num_items = pc->num_items;
    const int64_t num_short = pc->num_short;
    // a plan without hubs has no separate short-segment copy
    const int32_t* __restrict__ short_gather = pc->num_hubs == 0 ? gather_sorted : short_gather_in;
    // block-uniform loop: every thread reaches the barriers below
    for (int64_t ib = static_cast<int64_t>(blockIdx.x) * R; ib < num_items;
         ib += static_cast<int64_t>(gridDim.x) * R) {
        const int64_t ie = ib + R < num_items ? ib + R : num_items;
        const int64_t bk0 = clamp64(item_first[ib], 0, num_keys);
        const int64_t bk1 = clamp64(item_first[ie], bk0, num_keys);
        const int64_t bs0 = clamp64(item_short[ib], 0, num_short);
        const int64_t bs1 = clamp64(item_short[ie], bs0, num_short);
        const int64_t item = ib + grp;
        int64_t sb = bs1, se = bs1;
        if (item < ie) {
            sb = clamp64(item_short[item], bs0, bs1);
            se = clamp64(item_short[item + 1], sb, bs1);
        }
        // The item construction bounds the workgroup's keys by R * kItemSize and
        // its short messages by R * kItemSize + kHubThreshold; the clamps keep a
        // corrupt plan inside LDS.  All loads are issued before the first write.
        const int nk = static_cast<int>(bk1 - bk0 + 1 < kKeyCap ? bk1 - bk0 + 1 : kKeyCap);
        const int np = static_cast<int>(bs1 - bs0 < kPosCap ? bs1 - bs0 : kPosCap);
        int32_t tk[KI], tp[PI];
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const int i = static_cast<int>(threadIdx.x) + j * kThreads;
            tk[j] = i < nk ? short_off[bk0 + i] : 0;
        }
#pragma unroll
        for (int j = 0; j < PI; ++j) {
            const int i = static_cast<int>(threadIdx.x) + j * kThreads;
            tp[j] = i < np ? short_gather[bs0 + i] : 0;
        }
        __syncthreads();  // the previous round's LDS reads are done
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const int i = static_cast<int>(threadIdx.x) + j * kThreads;
            if (i < nk) s_off[i] = tk[j];
        }
        // labels start at 0; thread t owns positions [t * PI, t * PI + PI).
        // Positions past the staged range read row 0, a valid row of every
        // table the walker reads (it runs only when there are messages).
#pragma unroll
        for (int j = 0; j < PI; ++j) {
            const int i = static_cast<int>(threadIdx.x) + j * kThreads;
            s_idx[i] = i < np ? tp[j] : 0;
            s_key[static_cast<int>(threadIdx.x) * PI + j] = 0;
        }
        __syncthreads();
        // segment heads: the first staged position of each key with short
        // messages carries the key's offset from bk0 (keys with several
        // heads at one position cannot occur: a head needs a message)
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const int i = static_cast<int>(threadIdx.x) + j * kThreads;
            if (i + 1 < nk) {
                const int64_t a = static_cast<int64_t>(s_off[i]) - bs0;
                const int64_t b = static_cast<int64_t>(s_off[i + 1]) - bs0;
                if (b > a && a >= 0 && a < np) s_key[a] = static_cast<uint16_t>(i);
            }
        }
        __syncthreads();
        // running maximum over positions: each position gets its key's label
        {
            uint32_t v[PI];
            uint32_t run = 0;
#pragma unroll
            for (int j = 0; j < PI; ++j) {
                v[j] = s_key[static_cast<int>(threadIdx.x) * PI + j];
                run = v[j] > run ? v[j] : run;
            }
            // exclusive block maximum of the per-thread maxima
            const int lane = lane_id();
            uint32_t x = run;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const uint32_t y = __shfl_up(x, o, kWave);
                if (lane >= o) x = y > x ? y : x;
            }
            if (lane == kWave - 1) s_scan[threadIdx.x / kWave] = x;
            uint32_t before = __shfl_up(x, 1, kWave);
            if (lane == 0) before = 0;
            __syncthreads();
            const int wave = static_cast<int>(threadIdx.x) / kWave;
#pragma unroll
            for (int w = 0; w < kThreads / kWave; ++w) {
                const uint32_t t = s_scan[w];
                if (w < wave) before = t > before ? t : before;
            }
            uint32_t cur = before;
#pragma unroll
            for (int j = 0; j < PI; ++j) {
                cur = v[j] > cur ? v[j] : cur;
                const int at = static_cast<int>(threadIdx.x) * PI + j;
                s_key[at] = at < np ? static_cast<uint16_t>(cur) : kNoLabel;
            }
        }
        __syncthreads();
        // keys without short messages: the empty-segment result
        for (int64_t k = bk0 + grp; k < bk1; k += R) {
            const int i = static_cast<int>(k - bk0 < kKeyCap - 1 ? k - bk0 : kKeyCap - 2);
            if (s_off[i + 1] == s_off[i] && op.colok)
                pack_store_stream<T, V>(out + k * D + op.col, epi(k, op.empty(), D, op.col));
        }
        // the item's messages [sb, se), as staged positions [lb, le)
        const int lb = static_cast<int>(sb - bs0 < np ? sb - bs0 : np);
        const int le = static_cast<int>(se - bs0 < np ? se - bs0 : np);
        // Positions past the item (q + u >= le) hold the next item's messages
        // or the padding: valid rows to load, and labels that differ from
        // the item's last key (items hold whole keys), so a message ends its
        // segment exactly when the next position's label differs.
        if constexpr (Op::kResetAtEnd) op.reset();
        int prev = -1;
        for (int q = lb; q < le; q += U) {
            const int cnt = le - q < U ? le - q : U;
            int32_t idx[U];
            int lab[U + 1];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                idx[u] = s_idx[q + u];
                lab[u] = s_key[q + u];
            }
            lab[U] = s_key[q + U];
            op.load(idx, cnt);
            // Rows past cnt are masked in the arithmetic (no branch around
            // it, so the compiler keeps the loads unconditional and waits
            // for each row only where it is consumed); only a segment's
            // store is under a branch.
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool valid = u < cnt;
                const int64_t key = bk0 + lab[u];
                if constexpr (!Op::kResetAtEnd) {
                    if (valid) op.restart(lab[u] != prev, key);
                }
                op.add(u, valid);
                if (valid && lab[u + 1] != lab[u]) {
                    if (op.colok)
                        pack_store_stream<T, V>(out + row_offset(key, D) + op.col,
                                                epi(key, op.result(true), D, op.col));
                    if constexpr (Op::kResetAtEnd) op.reset();
                }
                prev = valid ? lab[u] : prev;
            }
        }
    }
}

struct HubChunk {
    int64_t key;
    int64_t beg;
    int64_t end;
    int64_t nch;
    bool ok;
};

__device__ __forceinline__ HubChunk hub_chunk(int64_t c, const int32_t* __restrict__ offsets,
                                              const int32_t* __restrict__ hub_key,
                                              const int32_t* __restrict__ hub_chunk_base,
                                              const int32_t* __restrict__ chunk_hub,
                                              int64_t num_hubs, int64_t num_edges) {
    HubChunk hc{0, 0, 0, 0, false};
    const int64_t h = chunk_hub[c];
    if (h < 0 || h >= num_hubs) return hc;
    hc.key = hub_key[h];
    const int64_t j = c - hub_chunk_base[h];
    const int64_t sb = clamp64(offsets[hc.key], 0, num_edges);
    const int64_t se = clamp64(offsets[hc.key + 1], sb, num_edges);
    hc.nch = (se - sb + kChunkSize - 1) / kChunkSize;
    hc.beg = clamp64(sb + j * kChunkSize, sb, se);
    hc.end = clamp64(hc.beg + kChunkSize, hc.beg, se);
    hc.ok = true;
    return hc;
}

// LDS slot of staged chunk position p: one pad word per 32 positions, so the
// row groups of a wave, which read positions a slice length apart, hit
// different banks.
__device__ __forceinline__ int hub_slot(int p) { return p + (p >> 5); }

// One workgroup per hub chunk: the chunk's gathered row indices are staged in
// LDS with coalesced loads, row group g folds slice g of the chunk, the
// slices are folded in order by group 0; a single-chunk hub is finished here.
template <typename T, int V, int G, class Op, class Epi>
__global__ __launch_bounds__(kThreads, WaveFloor<Op>::hub) void k_hub_chunks(
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ gs, int64_t num_edges,
    const int32_t* __restrict__ hub_key, const int32_t* __restrict__ hub_chunk_base,
    const int32_t* __restrict__ chunk_hub, const relm_mp_plan_counts* __restrict__ pc,
    T* __restrict__ partial, T* __restrict__ out, Op op, Epi epi) {
    using Partial = typename Op::Partial;
    constexpr int NG = kThreads / G;
    constexpr int U = batch_rows<G>();
    constexpr int kStage = (kChunkSize + kThreads - 1) / kThreads;  // staged indices per thread
    __shared__ Partial red[kThreads / kWave * G];
    __shared__ int32_t s_gs[kChunkSize + kChunkSize / 32];
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int grp = static_cast<int>(threadIdx.x) / G;
    op.col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    op.colok = op.col < op.D;
    op.lcol = op.colok ? op.col : 0;
    const int64_t D = op.D;
    const int64_t num_hubs = pc->num_hubs;
    const int64_t num_chunks = pc->num_chunks;
    for (int64_t c = blockIdx.x; c < num_chunks; c += gridDim.x) {
        const HubChunk hc =
            hub_chunk(c, offsets, hub_key, hub_chunk_base, chunk_hub, num_hubs, num_edges);
        const int len = hc.ok ? static_cast<int>(hc.end - hc.beg) : 0;  // <= kChunkSize
        {
            int32_t t[kStage];
#pragma unroll
            for (int j = 0; j < kStage; ++j) {
                const int i = static_cast<int>(threadIdx.x) + j * kThreads;
                t[j] = i < len ? gs[hc.beg + i] : 0;
            }
#pragma unroll
            for (int j = 0; j < kStage; ++j) {
                const int i = static_cast<int>(threadIdx.x) + j * kThreads;
                if (i < len) s_gs[hub_slot(i)] = t[j];
            }
        }
        __syncthreads();
        // the chunk's messages split evenly over the row groups in whole
        // batches (a hub of one short chunk still uses every group)
        const int per = ((len + NG * U - 1) / (NG * U)) * U;
        const int lo = min(grp * per, len);
        const int hi = min(lo + per, len);
        op.begin(hc.key, hc.ok && hi > lo);
        for (int q = lo; q < hi; q += U) {
            const int cnt = hi - q < U ? hi - q : U;
            int32_t idx[U];
#pragma unroll
            for (int u = 0; u < U; ++u) idx[u] = s_gs[hub_slot(q + (u < cnt ? u : cnt - 1))];
            op.load(idx, cnt);
            op.consume(cnt);
        }
        // Fold the slices: a shuffle tree over the groups of each wave, then
        // the waves in order.
        Partial pg = hi > lo ? op.partial() : Partial::identity();
        const int gw_idx = (static_cast<int>(threadIdx.x) & (kWave - 1)) / G;
#pragma unroll
        for (int sgrp = 1; sgrp < kWave / G; sgrp <<= 1) {
            const Partial other = pg.shfl_down(sgrp * G);
            if ((gw_idx & (2 * sgrp - 1)) == 0) pg.merge(other);
        }
        if (gw_idx == 0) red[(threadIdx.x / kWave) * G + gl] = pg;
        __syncthreads();
        if (grp == 0 && hc.ok && op.colok) {
            Partial acc = red[gl];
            for (int wv = 1; wv < kThreads / kWave; ++wv) acc.merge(red[wv * G + gl]);
            if (hc.nch == 1)
                pack_store<T, V>(out + hc.key * D + op.col, epi(hc.key, acc.value(), D, op.col));
            else
                acc.store(partial + c * Partial::kWords * D, D, op.col);
        }
        __syncthreads();
    }
}

template <class Partial, typename T, int U>
__device__ __forceinline__ Partial fold_partials(const T* __restrict__ partial, int64_t lo,
                                                 int64_t hi, int64_t D, int64_t col) {
    Partial acc = Partial::identity();
    for (int64_t c0 = lo; c0 < hi; c0 += U) {
        Partial x[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            x[u] = c0 + u < hi ? Partial::load(partial + (c0 + u) * Partial::kWords * D, D, col)
                               : Partial::identity();
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + u < hi) acc.merge(x[u]);
    }
    return acc;
}

// Hubs of more than one chunk: one workgroup per hub.  Row group g folds a
// contiguous range of the hub's chunk partials in chunk order; the group
// results are folded as a fixed tree (shuffles inside a wave, then the waves in
// order), so the result is deterministic.
template <typename T, int V, int G, class Partial, class Epi>
__global__ __launch_bounds__(kThreads) void k_hub_combine(
    int64_t D, const int32_t* __restrict__ hub_key, const int32_t* __restrict__ hub_chunk_base,
    const int32_t* __restrict__ multi_hubs, const relm_mp_plan_counts* __restrict__ pc,
    const T* __restrict__ partial, T* __restrict__ out, Epi epi) {
    constexpr int NG = kThreads / G;
    constexpr int U = batch_rows<G>();
    __shared__ Partial red[kThreads / kWave * G];
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int grp = static_cast<int>(threadIdx.x) / G;
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    const bool colok = col < D;
    const int64_t num_hubs = pc->num_hubs;
    const int64_t num_multi_hubs = pc->num_multi_hubs;
    const int64_t num_chunks = pc->num_chunks;
    for (int64_t bi = blockIdx.x; bi < num_multi_hubs; bi += gridDim.x) {
        const int64_t h = multi_hubs[bi];
        const bool hok = h >= 0 && h < num_hubs;
        const int64_t key = hok ? hub_key[h] : 0;
        // hub slots are in key order and so are their chunks: a hub's chunks
        // end where the next hub's begin
        const int64_t base = hok ? hub_chunk_base[h] : 0;
        const int64_t next = hok && h + 1 < num_hubs ? hub_chunk_base[h + 1] : num_chunks;
        int64_t nch = next - base;
        if (base < 0 || nch < 0 || next > num_chunks) nch = 0;
        const int64_t per = (nch + NG - 1) / NG;
        const int64_t lo = clamp64(grp * per, 0, nch);
        const int64_t hi = clamp64(lo + per, lo, nch);
        Partial pg = colok ? fold_partials<Partial, T, U>(partial, base + lo, base + hi, D, col)
                           : Partial::identity();
        const int gw_idx = (static_cast<int>(threadIdx.x) & (kWave - 1)) / G;
#pragma unroll
        for (int sgrp = 1; sgrp < kWave / G; sgrp <<= 1) {
            const Partial other = pg.shfl_down(sgrp * G);
            if ((gw_idx & (2 * sgrp - 1)) == 0) pg.merge(other);
        }
        if (gw_idx == 0) red[(threadIdx.x / kWave) * G + gl] = pg;
        __syncthreads();
        if (grp == 0 && colok && hok && nch > 0) {
            Partial acc = red[gl];
            for (int wv = 1; wv < kThreads / kWave; ++wv) acc.merge(red[wv * G + gl]);
            pack_store<T, V>(out + key * D + col, epi(key, acc.value(), D, col));
        }
        __syncthreads();
    }
}

// out[r] = table[gathers[inv[r]]] or 0 (inverse plans: fanout forward and
// injective sum backward).  Each row group keeps gather_rows_in_flight<T, V>() rows
// in flight.
// A workgroup takes R * RU consecutive rows at a time (row j * R + group of
// its chunk for the group's j-th row): all resident workgroups stream one
// contiguous region.  (Rows a grid apart instead - RU regions at once, a
// power-of-two distance apart at the bench sizes - ran up to 10% slower.)
// The identity (keys[e] == e for every edge): plans read back by the host
// have inv == NULL; plans still being validated carry the flag in counts.
__device__ __forceinline__ const int32_t* inverse_map(const int32_t* inv,
                                                      const relm_mp_plan_counts* pc) {
    return pc != nullptr && pc->identity != 0 ? nullptr : inv;
}

// The gathered index of edge e (0 <= e < num_edges): the caller's int64
// array, or a plan's int32 snapshot of it (tiles flagged plain hold the edge
// ids and are not stored) - half the index bytes.  fetch() issues the loads,
// value() combines them, so the loads of several edges are in flight at once:
// the snapshot word is read whether or not the tile is plain (it is
// allocated for every edge), and a snapshot without plain flags reads a zero
// word instead of a flag.
__device__ uint32_t g_plain_none = 0u;

struct GathersI64 {
    const int64_t* __restrict__ p;
    struct Raw {
        int64_t v;
    };
    __device__ __forceinline__ Raw fetch(int64_t e) const { return {p[e]}; }
    __device__ __forceinline__ int64_t value(int64_t, const Raw& r) const { return r.v; }
};
struct GathersSnap {
    const int32_t* __restrict__ p;
    const uint32_t* __restrict__ plain;
    struct Raw {
        int32_t v;
        uint32_t flag;
    };
    __device__ __forceinline__ Raw fetch(int64_t e) const {
        const bool has = plain != nullptr;
        const uint32_t* f = has ? plain + e / RELM_MP_SNAP_TILE : &g_plain_none;
        return {p[e], *f};
    }
    __device__ __forceinline__ int64_t value(int64_t e, const Raw& r) const {
        return r.flag != 0u ? e : static_cast<int64_t>(r.v);
    }
};

// Row kernels over inverse plans issue every load of an iteration without a
// branch: a row past num_keys, an edge without a key and an invalid gathered
// index read row 0 / edge 0 instead (the kernels run only with at least one
// edge and one gathered row) and their values are discarded.  With the loads
// under branches the compiler waits for each index before the next.
struct InvRow {
    int64_t key;   // the row, or 0 past num_keys
    bool live;     // key < num_keys
    int64_t g;     // gathered row, or 0
    bool ok;       // the row has an edge whose gathered index is in [0, num_gather)
};

template <int RU, class Src>
__device__ __forceinline__ void inverse_rows(InvRow (&r)[RU], int64_t key0, int64_t stride,
                                             const int32_t* __restrict__ inv, int64_t num_keys,
                                             int64_t num_edges, const Src& gathers,
                                             int64_t num_gather) {
    int64_t e[RU];
#pragma unroll
    for (int j = 0; j < RU; ++j) {
        const int64_t key = key0 + j * stride;
        r[j].live = key < num_keys;
        r[j].key = r[j].live ? key : 0;
    }
    if (inv != nullptr) {
#pragma unroll
        for (int j = 0; j < RU; ++j) {
            const int32_t iv = inv[r[j].key];
            e[j] = r[j].live ? static_cast<int64_t>(iv) : -1;
        }
    } else {
#pragma unroll
        for (int j = 0; j < RU; ++j) e[j] = r[j].live && r[j].key < num_edges ? r[j].key : -1;
    }
    typename Src::Raw raw[RU];
#pragma unroll
    for (int j = 0; j < RU; ++j) {
        const bool has = e[j] >= 0 && e[j] < num_edges;
        e[j] = has ? e[j] : -1;
        raw[j] = gathers.fetch(has ? e[j] : 0);
    }
#pragma unroll
    for (int j = 0; j < RU; ++j) {
        const int64_t d = gathers.value(e[j] >= 0 ? e[j] : 0, raw[j]);
        r[j].ok = e[j] >= 0 && static_cast<uint64_t>(d) < static_cast<uint64_t>(num_gather);
        r[j].g = r[j].ok ? d : 0;
    }
}

template <typename T, int V, int G, class Rows, class Src>
__global__ __launch_bounds__(kThreads) void k_gather_inv(const int32_t* __restrict__ inv_in,
                                                         const relm_mp_plan_counts* __restrict__ pc,
                                                         int64_t num_edges, Src gathers,
                                                         int64_t num_gather,
                                                         const T* __restrict__ table,
                                                         int64_t num_keys, int64_t D,
                                                         T* __restrict__ out, Rows out_rows,
                                                         bool skip_on_collision) {
    constexpr int R = kThreads / G;
    constexpr int RU = gather_rows_in_flight<T, V>();
    // an inverse map built without atomics is only used when no row repeats
    if (skip_on_collision && pc->collisions != 0) return;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    if (col >= D) return;
    const int32_t* inv = inverse_map(inv_in, pc);
    const int64_t chunk = static_cast<int64_t>(R) * RU;
    const int64_t grp = threadIdx.x / G;
    for (int64_t key0 = static_cast<int64_t>(blockIdx.x) * chunk + grp; key0 < num_keys;
         key0 += static_cast<int64_t>(gridDim.x) * chunk) {
        if (num_edges <= 0 || num_gather <= 0) {  // uniform: no row to gather
#pragma unroll
            for (int j = 0; j < RU; ++j)
                if (key0 + j * R < num_keys)
                    pack_store_stream<T, V>(out + out_rows(key0 + j * R, D) + col, pack_fill<T, V>(T(0)));
            continue;
        }
        InvRow r[RU];
        inverse_rows<RU>(r, key0, R, inv, num_keys, num_edges, gathers, num_gather);
        Pack<T, V> v[RU];
#pragma unroll
        for (int j = 0; j < RU; ++j) v[j] = pack_load<T, V>(table + row_offset(r[j].g, D) + col);
#pragma unroll
        for (int j = 0; j < RU; ++j) {
            if (!r[j].ok) v[j] = pack_fill<T, V>(T(0));
            if (r[j].live) pack_store_stream<T, V>(out + out_rows(r[j].key, D) + col, v[j]);
        }
    }
}

// Reads [a, a + na) and [b, b + nb) (16-byte units) and discards the data: a
// read-only pass that leaves the arrays in the memory-side cache for the
// kernel after it.
__global__ __launch_bounds__(kThreads) void k_touch(const uint4* __restrict__ a, int64_t na,
                                                    const uint4* __restrict__ b, int64_t nb) {
    uint32_t acc = 0;
    const int64_t n = na + nb;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const uint4 v = i < na ? a[i] : b[i - na];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    asm volatile("" ::"v"(acc));
}

// Row epilogues of the LGAN aggregations: out[r] = base[r] + in[j] / d_j with
// j = gather[r] (or r), d_j = 1, max(1, segment size j of a CSR plan) or
// max(1, (T)div_values[j]); `in` null reads zeros, `base` null adds nothing.
// The division and the addition round separately, as the reference's
// tensor expressions do.  Each row group keeps gather_rows_in_flight<T, V>()
// rows in flight: the gathered indices of its rows are loaded first, then
// their divisors and rows, without a branch (a row past `rows` reads row 0 of
// every array - the kernel runs only with rows > 0 - and stores nothing).
template <typename T, int V, int G>
__global__ __launch_bounds__(kThreads) void k_rows_scale(
    const T* in, const int64_t* __restrict__ gather, int div_kind,
    const int32_t* __restrict__ div_offsets, const int64_t* __restrict__ div_values,
    const T* base, int64_t rows, int64_t D, T* out) {
    constexpr int R = kThreads / G;
    constexpr int RU = gather_rows_in_flight<T, V>();
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    if (col >= D) return;
    const int64_t chunk = static_cast<int64_t>(R) * RU;
    for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * chunk + threadIdx.x / G; r0 < rows;
         r0 += static_cast<int64_t>(gridDim.x) * chunk) {
        int64_t r[RU], j[RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            r[u] = r0 + u * R;
            const int64_t rc = r[u] < rows ? r[u] : 0;
            j[u] = gather != nullptr ? gather[rc] : rc;
        }
        T d[RU];
        Pack<T, V> x[RU], b[RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            d[u] = T(1);
            if (div_kind == RELM_MP_DIV_SEGMENT) {
                const int32_t n = div_offsets[j[u] + 1] - div_offsets[j[u]];
                d[u] = n > 1 ? static_cast<T>(n) : T(1);
            } else if (div_kind == RELM_MP_DIV_VALUES) {
                const T v = static_cast<T>(div_values[j[u]]);
                d[u] = v > T(1) ? v : T(1);
            }
            x[u] = in != nullptr ? pack_load<T, V>(in + row_offset(j[u], D) + col) : pack_fill<T, V>(T(0));
            if (base != nullptr) b[u] = pack_load<T, V>(base + (r[u] < rows ? r[u] : 0) * D + col);
        }
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            if (div_kind != RELM_MP_DIV_NONE) {
#pragma unroll
                for (int i = 0; i < V; ++i) x[u].v[i] = x[u].v[i] / d[u];
            }
            if (base != nullptr) {
#pragma unroll
                for (int i = 0; i < V; ++i) x[u].v[i] = b[u].v[i] + x[u].v[i];
            }
            if (r[u] < rows) pack_store<T, V>(out + r[u] * D + col, x[u]);
        }
    }
}

// out[k] = table[gather of the last edge of segment k] or 0 (CSR plans).
template <typename T, int V, int G, class Rows>
__global__ __launch_bounds__(kThreads) void k_gather_last_csr(const int32_t* __restrict__ offsets,
                                                              const int32_t* __restrict__ gs,
                                                              int64_t num_edges,
                                                              const T* __restrict__ table,
                                                              int64_t num_keys, int64_t D,
                                                              T* __restrict__ out, Rows out_rows) {
    constexpr int R = kThreads / G;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    if (col >= D) return;
    for (int64_t key = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / G; key < num_keys;
         key += static_cast<int64_t>(gridDim.x) * R) {
        const int64_t b = clamp64(offsets[key], 0, num_edges);
        const int64_t e = clamp64(offsets[key + 1], b, num_edges);
        Pack<T, V> v = pack_fill<T, V>(T(0));
        if (e > b) v = pack_load<T, V>(table + row_offset(gs[e - 1], D) + col);
        pack_store_stream<T, V>(out + out_rows(key, D) + col, v);
    }
}

// Logsumexp backward with an inverse plan (injective keys):
// grad_rel[r] = grad_out[d] * exp(rel[r] - out[d]), d = gathers(inv[r]), or 0.
template <typename T, int V, int G, class Src>
__global__ __launch_bounds__(kThreads) void k_lse_bwd_inv(
    const int32_t* __restrict__ inv_in, const relm_mp_plan_counts* __restrict__ pc,
    int64_t num_edges, Src gathers,
    int64_t num_gather,
    const T* __restrict__ grad_out, const T* __restrict__ out, const T* __restrict__ rel,
    int64_t num_keys, int64_t D, T* __restrict__ grad_rel, bool skip_on_collision) {
    constexpr int R = kThreads / G;
    constexpr int RU = kLseRowsInFlight;
    // an inverse map built without atomics is only used when no row repeats
    if (skip_on_collision && pc->collisions != 0) return;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    if (col >= D) return;
    const int32_t* inv = inverse_map(inv_in, pc);
    const int64_t chunk = static_cast<int64_t>(R) * RU;
    const int64_t grp = threadIdx.x / G;
    for (int64_t key0 = static_cast<int64_t>(blockIdx.x) * chunk + grp; key0 < num_keys;
         key0 += static_cast<int64_t>(gridDim.x) * chunk) {
        if (num_edges <= 0 || num_gather <= 0) {  // uniform: no row to gather
#pragma unroll
            for (int j = 0; j < RU; ++j)
                if (key0 + j * R < num_keys)
                    pack_store_stream<T, V>(grad_rel + (key0 + j * R) * D + col, pack_fill<T, V>(T(0)));
            continue;
        }
        InvRow r[RU];
        inverse_rows<RU>(r, key0, R, inv, num_keys, num_edges, gathers, num_gather);
        Pack<T, V> x[RU], g[RU], o[RU];
#pragma unroll
        for (int j = 0; j < RU; ++j) {
            x[j] = pack_load_stream<T, V>(rel + r[j].key * D + col);
            g[j] = pack_load<T, V>(grad_out + row_offset(r[j].g, D) + col);
            o[j] = pack_load<T, V>(out + row_offset(r[j].g, D) + col);
        }
#pragma unroll
        for (int j = 0; j < RU; ++j) {
            Pack<T, V> res;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const T w = fast_exp<T>(x[j].v[i] - o[j].v[i]);
                const T c = g[j].v[i] * w;
                res.v[i] = r[j].ok ? T(0) + c : T(0);
            }
            if (r[j].live) pack_store_stream<T, V>(grad_rel + r[j].key * D + col, res);
        }
    }
}

// Sum backward of fanin_reduce in edge order when the message rows are a
// permutation of the edges (flat_src injective and rel_rows == num_edges, as a
// count of the inverse map's lost edges - zero - has shown on the device):
// edge e writes its own message row rows(e) whole, grad_rel[rows(e)] =
// grad_out[dsts(e)], so no inverse map is read.  Both index arrays are a
// forward plan's int32 snapshots; all loads of an iteration are issued without
// a branch (an out-of-range index reads row 0 and stores nothing: the kernel
// runs with at least one edge and one destination row).
struct EdgeRow {
    int64_t row;  // message row, or 0
    int64_t d;    // destination row, or 0
    bool ok;
};

template <int RU>
__device__ __forceinline__ void edge_rows(EdgeRow (&r)[RU], int64_t e0, int64_t stride,
                                          int64_t num_edges, const GathersSnap& rows,
                                          int64_t num_rows, const GathersSnap& dsts,
                                          int64_t num_dst) {
    GathersSnap::Raw rr[RU], dr[RU];
    int64_t e[RU];
#pragma unroll
    for (int j = 0; j < RU; ++j) {
        e[j] = e0 + j * stride;
        const int64_t ec = e[j] < num_edges ? e[j] : 0;
        rr[j] = rows.fetch(ec);
        dr[j] = dsts.fetch(ec);
    }
#pragma unroll
    for (int j = 0; j < RU; ++j) {
        const int64_t ec = e[j] < num_edges ? e[j] : 0;
        const int64_t row = rows.value(ec, rr[j]);
        const int64_t d = dsts.value(ec, dr[j]);
        r[j].ok = e[j] < num_edges && static_cast<uint64_t>(row) < static_cast<uint64_t>(num_rows) &&
                  static_cast<uint64_t>(d) < static_cast<uint64_t>(num_dst);
        r[j].row = r[j].ok ? row : 0;
        r[j].d = r[j].ok ? d : 0;
    }
}

template <typename T, int V, int G>
__global__ __launch_bounds__(kThreads) void k_gather_edges(const relm_mp_plan_counts* __restrict__ pc,
                                                           int64_t num_edges, GathersSnap rows,
                                                           int64_t num_rows, GathersSnap dsts,
                                                           int64_t num_dst, const T* __restrict__ table,
                                                           int64_t D, T* __restrict__ out) {
    constexpr int R = kThreads / G;
    constexpr int RU = gather_rows_in_flight<T, V>();
    if (pc->collisions != 0) return;  // not a permutation: the caller takes another path
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    if (col >= D) return;
    const int64_t chunk = static_cast<int64_t>(R) * RU;
    const int64_t grp = threadIdx.x / G;
    for (int64_t e0 = static_cast<int64_t>(blockIdx.x) * chunk + grp; e0 < num_edges;
         e0 += static_cast<int64_t>(gridDim.x) * chunk) {
        EdgeRow r[RU];
        edge_rows<RU>(r, e0, R, num_edges, rows, num_rows, dsts, num_dst);
        Pack<T, V> v[RU];
#pragma unroll
        for (int j = 0; j < RU; ++j) v[j] = pack_load<T, V>(table + row_offset(r[j].d, D) + col);
#pragma unroll
        for (int j = 0; j < RU; ++j)
            if (r[j].ok) pack_store_stream<T, V>(out + row_offset(r[j].row, D) + col, v[j]);
    }
}

// ---- host-side dispatch --------------------------------------------------

struct Geometry {
    int V;
    int G;
    int64_t slices;
};

// Dense rows: the widest of kVecMax, kVecMax / 2 and 1 elements per lane that
// divides D and keeps every row start aligned (rows of an even number of
// floats that is not a multiple of 4 still move 8 bytes per lane).
template <typename T>
Geometry choose_geometry(int64_t D, std::initializer_list<const void*> ptrs) {
    constexpr int kVecMax = 16 / static_cast<int>(sizeof(T));
    int V = kVecMax;
    for (; V > 1; V /= 2) {
        bool ok = D % V == 0;
        for (const void* p : ptrs)
            ok = ok && (p == nullptr || reinterpret_cast<uintptr_t>(p) % (sizeof(T) * V) == 0);
        if (ok) break;
    }
    const int64_t vcols = (D + V - 1) / V;
    int G = 4;
    while (G < vcols && G < 64) G *= 2;
    const int64_t slices = (vcols + G - 1) / G;
    return {V, G, slices};
}

template <typename T, typename F>
int with_geometry(const Geometry& geo, F&& f) {
    auto by_g = [&](auto vt) -> int {
        switch (geo.G) {
            case 4: return f(vt, std::integral_constant<int, 4>{});
            case 8: return f(vt, std::integral_constant<int, 8>{});
            case 16: return f(vt, std::integral_constant<int, 16>{});
            case 32: return f(vt, std::integral_constant<int, 32>{});
            case 64: return f(vt, std::integral_constant<int, 64>{});
            default: break;
        }
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: unsupported row geometry");
    };
    constexpr int kVecMax = 16 / static_cast<int>(sizeof(T));
    if (geo.V == kVecMax) return by_g(std::integral_constant<int, kVecMax>{});
    if constexpr (kVecMax > 2) {
        if (geo.V == kVecMax / 2) return by_g(std::integral_constant<int, kVecMax / 2>{});
    }
    return by_g(std::integral_constant<int, 1>{});
}

// Grouped row layouts (argument slots of a wider matrix): the widest of
// kVecMax, kVecMax / 2 and 1 elements per lane that keeps every row start
// aligned - lines of an odd number of 8-byte pairs still move 8 bytes per lane.
template <typename T>
Geometry choose_grouped_geometry(int64_t D, int64_t stride, std::initializer_list<const void*> ptrs) {
    constexpr int kVecMax = 16 / static_cast<int>(sizeof(T));
    int V = kVecMax;
    for (; V > 1; V /= 2) {
        bool ok = D % V == 0 && stride % V == 0;
        for (const void* p : ptrs)
            ok = ok && (p == nullptr || reinterpret_cast<uintptr_t>(p) % (sizeof(T) * V) == 0);
        if (ok) break;
    }
    const int64_t vcols = (D + V - 1) / V;
    int G = 4;
    while (G < vcols && G < 64) G *= 2;
    return {V, G, (vcols + G - 1) / G};
}

template <typename T, typename F>
int with_grouped_geometry(const Geometry& geo, F&& f) {
    constexpr int kVecMax = 16 / static_cast<int>(sizeof(T));
    auto by_g = [&](auto vt) -> int {
        switch (geo.G) {
            case 4: return f(vt, std::integral_constant<int, 4>{});
            case 8: return f(vt, std::integral_constant<int, 8>{});
            case 16: return f(vt, std::integral_constant<int, 16>{});
            case 32: return f(vt, std::integral_constant<int, 32>{});
            case 64: return f(vt, std::integral_constant<int, 64>{});
            default: break;
        }
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: unsupported row geometry");
    };
    if (geo.V == kVecMax) return by_g(std::integral_constant<int, kVecMax>{});
    if constexpr (kVecMax > 2) {
        if (geo.V == kVecMax / 2) return by_g(std::integral_constant<int, kVecMax / 2>{});
    }
    return by_g(std::integral_constant<int, 1>{});
}

dim3 row_grid(int64_t rows, int G, int64_t slices, int rows_per_group = 1) {
    const int64_t per = static_cast<int64_t>(kThreads / G) * rows_per_group;
    int64_t bx = (rows + per - 1) / per;
    if (bx < 1) bx = 1;
    if (bx > kMaxBlocksX) bx = kMaxBlocksX;
    return dim3(static_cast<unsigned>(bx), static_cast<unsigned>(slices));
}

// Workgroups of `kernel` (kThreads each) resident on the current device at
// once; persistent launches size their grids with it.
int64_t resident_blocks(const void* kernel) {
    static std::mutex mu;
    static std::map<std::pair<const void*, int>, int64_t> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return 2048;
    }
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(kernel, dev);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int cus = 0, per_cu = 0;
    int64_t r = 2048;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0) == hipSuccess &&
        cus > 0 && per_cu > 0)
        r = static_cast<int64_t>(cus) * per_cu;
    else
        (void)hipGetLastError();
    cache.emplace(key, r);
    return r;
}

// Grid of a grid-stride launch over `work` units of `per_block` each, times
// `slices` column slices: one workgroup per unit, at most `rounds` times what
// is resident at once.  Unit costs vary (hub chunks of 65..2048 messages), so
// several rounds of workgroups let the hardware scheduler balance them; the
// workgroups past the actual count (read on the device) exit at once, which
// costs about 1.5 ns each.
dim3 persistent_grid(const void* kernel, int64_t work, int64_t per_block, int64_t slices,
                     int64_t rounds) {
    int64_t bx = (work + per_block - 1) / per_block;
    const int64_t cap =
        std::max<int64_t>(1, rounds * resident_blocks(kernel) / std::max<int64_t>(1, slices));
    bx = std::max<int64_t>(1, std::min(bx, cap));
    return dim3(static_cast<unsigned>(bx), static_cast<unsigned>(slices));
}

// Runs the CSR reduction of `op` (items, hub chunks, hub combines) into out.
// The item, hub and chunk counts are read from plan.counts on the device:
// grids are sized by the host-side counts where the plan has them (>= 0),
// else by the plan's capacities, and capped (persistent_grid).
template <typename T, int V, int G, class Op, class Epi = NoEpilogue>
int run_csr(const relm_mp_plan& plan, const Op& op, int64_t slices, T* partial, T* out,
            hipStream_t s, const Epi& epi = Epi{}) {
    using Partial = typename Op::Partial;
    if (plan.counts == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: CSR plan without counts");
    const int64_t E = plan.num_edges;
    const int64_t items = plan.num_items >= 0 ? plan.num_items : item_capacity_for(plan.num_keys);
    const void* walk = reinterpret_cast<const void*>(&k_walk_items<T, V, G, Op, Epi>);
    hipLaunchKernelGGL((k_walk_items<T, V, G, Op, Epi>),
                       persistent_grid(walk, items, kThreads / G, slices, 4), dim3(kThreads), 0, s,
                       plan.short_off, plan.short_gather, plan.gather_sorted, plan.item_first,
                       plan.item_short, plan.counts, plan.num_keys, out, op, epi);
    int rc = hip_error(hipGetLastError(), "relm_mp item kernel");
    // no hub when the counts say so, or when no segment can be longer than the threshold
    if (rc != RELM_MP_OK || plan.num_hubs == 0 || E <= kHubThreshold) return rc;
    const int64_t chunks = plan.num_chunks >= 0 ? plan.num_chunks : max_chunks(E);
    const void* hub = reinterpret_cast<const void*>(&k_hub_chunks<T, V, G, Op, Epi>);
    hipLaunchKernelGGL((k_hub_chunks<T, V, G, Op, Epi>), persistent_grid(hub, chunks, 1, slices, 8),
                       dim3(kThreads), 0, s, plan.offsets, plan.gather_sorted, plan.num_edges,
                       plan.hub_key, plan.hub_chunk_base, plan.chunk_hub, plan.counts, partial, out,
                       op, epi);
    rc = hip_error(hipGetLastError(), "relm_mp hub chunk kernel");
    // no hub of more than one chunk when the counts say so, or when none fits
    if (rc != RELM_MP_OK || plan.num_multi_hubs == 0 || E <= kChunkSize) return rc;
    const int64_t multi = plan.num_multi_hubs >= 0 ? plan.num_multi_hubs : E / (kChunkSize + 1) + 1;
    const void* comb = reinterpret_cast<const void*>(&k_hub_combine<T, V, G, Partial, Epi>);
    hipLaunchKernelGGL((k_hub_combine<T, V, G, Partial, Epi>),
                       persistent_grid(comb, multi, 1, slices, 8), dim3(kThreads), 0, s,
                       op.D, plan.hub_key, plan.hub_chunk_base,
                       plan.multi_hubs, plan.counts, static_cast<const T*>(partial), out, epi);
    return hip_error(hipGetLastError(), "relm_mp hub combine kernel");
}

// group > 0: the output rows are grouped (GroupedRows{group, group_stride}).
template <typename T>
int gather_last_t(const relm_mp_plan& plan, const int64_t* gathers, const void* table_v,
                  int64_t emb, void* out_v, int64_t group, int64_t group_stride, hipStream_t s,
                  const relm_mp_plan* snap = nullptr, bool skip_on_collision = false) {
    const T* table = static_cast<const T*>(table_v);
    T* out = static_cast<T*>(out_v);
    auto launch = [&](auto vt, auto gt, const Geometry& geo, auto rows) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        using Rows = decltype(rows);
        if (plan.kind == RELM_MP_PLAN_INVERSE) {
            const dim3 grid = row_grid(plan.num_keys, G, geo.slices, gather_rows_in_flight<T, V>());
            if (snap != nullptr) {
                hipLaunchKernelGGL((k_gather_inv<T, V, G, Rows, GathersSnap>), grid, dim3(kThreads), 0, s,
                                   plan.inv, plan.counts, plan.num_edges,
                                   GathersSnap{snap->snap_keys, snap->snap_key_plain}, plan.num_gather,
                                   table, plan.num_keys, emb, out, rows, skip_on_collision);
            } else {
                hipLaunchKernelGGL((k_gather_inv<T, V, G, Rows, GathersI64>), grid, dim3(kThreads), 0, s,
                                   plan.inv, plan.counts, plan.num_edges, GathersI64{gathers},
                                   plan.num_gather, table, plan.num_keys, emb, out, rows, skip_on_collision);
            }
        } else {
            hipLaunchKernelGGL((k_gather_last_csr<T, V, G, Rows>),
                               row_grid(plan.num_keys, G, geo.slices), dim3(kThreads), 0, s,
                               plan.offsets, plan.gather_sorted, plan.num_edges, table,
                               plan.num_keys, emb, out, rows);
        }
        return hip_error(hipGetLastError(), "relm_mp gather kernel");
    };
    if (group > 0) {
        const Geometry geo = choose_grouped_geometry<T>(emb, group_stride, {table, out});
        const GroupedRows rows{static_cast<uint32_t>(group), static_cast<uint64_t>(group_stride)};
        return with_grouped_geometry<T>(
            geo, [&](auto vt, auto gt) -> int { return launch(vt, gt, geo, rows); });
    }
    const Geometry geo = choose_geometry<T>(emb, {table, out});
    return with_geometry<T>(geo,
                            [&](auto vt, auto gt) -> int { return launch(vt, gt, geo, DenseRows{}); });
}

// Sum over each key's segment of table rows in a grouped layout.
template <typename T>
int segment_sum_grouped_t(const relm_mp_plan& plan, const void* table_v, int64_t emb,
                          int64_t group, int64_t group_stride, void* out_v, void* scratch,
                          hipStream_t s) {
    const T* table = static_cast<const T*>(table_v);
    T* out = static_cast<T*>(out_v);
    T* partial = static_cast<T*>(scratch);
    const Geometry geo = choose_grouped_geometry<T>(emb, group_stride, {table, out, partial});
    return with_grouped_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        constexpr int U = batch_rows<G>();
        SumOp<T, V, U, GroupedRows> op{};
        op.table = table;
        op.D = emb;
        op.rows = GroupedRows{static_cast<uint32_t>(group), static_cast<uint64_t>(group_stride)};
        return run_csr<T, V, G>(plan, op, geo.slices, partial, out, s);
    });
}

template <typename T, int MODE>
int segment_reduce_t(const relm_mp_plan& plan, const void* table_v, int64_t emb, void* out_v,
                     void* scratch, hipStream_t s) {
    const T* table = static_cast<const T*>(table_v);
    T* out = static_cast<T*>(out_v);
    T* partial = static_cast<T*>(scratch);
    const Geometry geo = choose_geometry<T>(emb, {table, out, partial});
    return with_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        constexpr int U = batch_rows<G>();
        if constexpr (MODE == RELM_MP_MODE_SUM) {
            SumOp<T, V, U> op{};
            op.table = table;
            op.D = emb;
            return run_csr<T, V, G>(plan, op, geo.slices, partial, out, s);
        } else {
            LseOp<T, V, U> op{};
            op.table = table;
            op.D = emb;
            return run_csr<T, V, G>(plan, op, geo.slices, partial, out, s);
        }
    });
}

template <typename T>
int segment_sum_scaled_t(const relm_mp_plan& plan, const void* table_v, int64_t emb, int div_kind,
                         const int64_t* div_values, const void* base_v, void* out_v, void* scratch,
                         hipStream_t s) {
    const T* table = static_cast<const T*>(table_v);
    const T* base = static_cast<const T*>(base_v);
    T* out = static_cast<T*>(out_v);
    T* partial = static_cast<T*>(scratch);
    const Geometry geo = choose_geometry<T>(emb, {table, base, out, partial});
    return with_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        constexpr int U = batch_rows<G>();
        SumOp<T, V, U> op{};
        op.table = table;
        op.D = emb;
        const ScaleEpilogue<T> epi{base, div_kind, plan.offsets, div_values};
        return run_csr<T, V, G>(plan, op, geo.slices, partial, out, s, epi);
    });
}

template <typename T>
int lse_backward_t(const relm_mp_plan& plan, const int64_t* gathers, const void* grad_out_v,
                   const void* out_v, const void* rel_v, int64_t emb, void* grad_rel_v,
                   void* scratch, hipStream_t s, const relm_mp_plan* snap = nullptr,
                   bool skip_on_collision = false) {
    const T* grad_out = static_cast<const T*>(grad_out_v);
    const T* out = static_cast<const T*>(out_v);
    const T* rel = static_cast<const T*>(rel_v);
    T* grad_rel = static_cast<T*>(grad_rel_v);
    T* partial = static_cast<T*>(scratch);
    const Geometry geo = choose_geometry<T>(emb, {grad_out, out, rel, grad_rel, partial});
    return with_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        constexpr int U = batch_rows<G>();
        if (plan.kind == RELM_MP_PLAN_INVERSE) {
            const dim3 grid = row_grid(plan.num_keys, G, geo.slices, kLseRowsInFlight);
            if (snap != nullptr) {
                hipLaunchKernelGGL((k_lse_bwd_inv<T, V, G, GathersSnap>), grid, dim3(kThreads), 0, s,
                                   plan.inv, plan.counts, plan.num_edges,
                                   GathersSnap{snap->snap_keys, snap->snap_key_plain}, plan.num_gather,
                                   grad_out, out, rel, plan.num_keys, emb, grad_rel, skip_on_collision);
            } else {
                hipLaunchKernelGGL((k_lse_bwd_inv<T, V, G, GathersI64>), grid, dim3(kThreads), 0, s,
                                   plan.inv, plan.counts, plan.num_edges, GathersI64{gathers},
                                   plan.num_gather, grad_out, out, rel, plan.num_keys, emb, grad_rel,
                                   skip_on_collision);
            }
            return hip_error(hipGetLastError(), "relm_mp logsumexp backward kernel");
        }
        LseBwdOp<T, V, U> op{};
        op.grad_out = grad_out;
        op.out = out;
        op.rel = rel;
        op.D = emb;
        return run_csr<T, V, G>(plan, op, geo.slices, partial, grad_rel, s);
    });
}

}  // namespace

size_t hub_partial_bytes(const relm_mp_plan& plan, int64_t emb, int dtype, int64_t mode) {
    if (plan.kind != RELM_MP_PLAN_CSR || plan.num_chunks == 0 || plan.num_edges <= kHubThreshold)
        return 0;
    const size_t elem = dtype == RELM_MP_F64 ? 8 : 4;
    const size_t per = static_cast<size_t>(emb) * elem * (mode == RELM_MP_MODE_LOGSUMEXP ? 2 : 1);
    // counts not read back yet: the capacity of the chunk list
    const int64_t chunks = plan.num_chunks >= 0 ? plan.num_chunks : max_chunks(plan.num_edges);
    return static_cast<size_t>(chunks) * per;
}

int compute_segment_sum_scaled(int dtype, const relm_mp_plan& plan, const void* table,
                               int64_t emb, int div_kind, const int64_t* div_values,
                               const void* base, void* out, void* scratch, size_t scratch_bytes,
                               hipStream_t s) {
    if (plan.num_keys == 0 || emb == 0) return RELM_MP_OK;
    if (plan.kind != RELM_MP_PLAN_CSR)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: scaled sums need a CSR plan");
    if (scratch_bytes < hub_partial_bytes(plan, emb, dtype, RELM_MP_MODE_SUM))
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: hub scratch too small");
    return dtype == RELM_MP_F64
               ? segment_sum_scaled_t<double>(plan, table, emb, div_kind, div_values, base, out,
                                              scratch, s)
               : segment_sum_scaled_t<float>(plan, table, emb, div_kind, div_values, base, out,
                                             scratch, s);
}

template <typename T>
int segment_sum_msgdiv_t(const relm_mp_plan& plan, const void* table_v, int64_t emb,
                         const int32_t* msg_div_offsets, const void* base_v, void* out_v,
                         void* scratch, hipStream_t s) {
    const T* table = static_cast<const T*>(table_v);
    const T* base = static_cast<const T*>(base_v);
    T* out = static_cast<T*>(out_v);
    T* partial = static_cast<T*>(scratch);
    const Geometry geo = choose_geometry<T>(emb, {table, base, out, partial});
    return with_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        constexpr int U = batch_rows<G>();
        SumDivOp<T, V, U> op{};
        op.table = table;
        op.D = emb;
        op.div_offsets = msg_div_offsets;
        const ScaleEpilogue<T> epi{base, RELM_MP_DIV_NONE, plan.offsets, nullptr};
        return run_csr<T, V, G>(plan, op, geo.slices, partial, out, s, epi);
    });
}

int compute_segment_sum_msgdiv(int dtype, const relm_mp_plan& plan, const void* table, int64_t emb,
                               const int32_t* msg_div_offsets, const void* base, void* out,
                               void* scratch, size_t scratch_bytes, hipStream_t s) {
    if (plan.num_keys == 0 || emb == 0) return RELM_MP_OK;
    if (plan.kind != RELM_MP_PLAN_CSR)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: divided sums need a CSR plan");
    if (scratch_bytes < hub_partial_bytes(plan, emb, dtype, RELM_MP_MODE_SUM))
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: hub scratch too small");
    return dtype == RELM_MP_F64
               ? segment_sum_msgdiv_t<double>(plan, table, emb, msg_div_offsets, base, out, scratch, s)
               : segment_sum_msgdiv_t<float>(plan, table, emb, msg_div_offsets, base, out, scratch, s);
}

int compute_fill(int dtype, void* out, int64_t count, double value, hipStream_t s) {
    if (count <= 0) return RELM_MP_OK;
    int64_t blocks = (count + kThreads * 4 - 1) / (kThreads * 4);
    if (blocks > (1 << 20)) blocks = 1 << 20;
    if (dtype == RELM_MP_F64) {
        hipLaunchKernelGGL(k_fill<double>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                           static_cast<double*>(out), count, value);
    } else {
        hipLaunchKernelGGL(k_fill<float>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                           static_cast<float*>(out), count, static_cast<float>(value));
    }
    return hip_error(hipGetLastError(), "relm_mp fill kernel");
}

template <typename T>
int rows_scale_t(const void* in_v, const int64_t* gather, int div_kind, const int32_t* div_offsets,
                 const int64_t* div_values, const void* base_v, int64_t rows, int64_t emb,
                 void* out_v, hipStream_t s) {
    const T* in = static_cast<const T*>(in_v);
    const T* base = static_cast<const T*>(base_v);
    T* out = static_cast<T*>(out_v);
    const Geometry geo = choose_geometry<T>(emb, {in, base, out});
    return with_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        hipLaunchKernelGGL((k_rows_scale<T, V, G>), row_grid(rows, G, geo.slices, gather_rows_in_flight<T, V>()),
                           dim3(kThreads),
                           0, s, in, gather, div_kind, div_offsets, div_values, base, rows, emb,
                           out);
        return hip_error(hipGetLastError(), "relm_mp row scale kernel");
    });
}

int compute_rows_scale(int dtype, const void* in, const int64_t* gather, int div_kind,
                       const int32_t* div_offsets, const int64_t* div_values, const void* base,
                       int64_t rows, int64_t emb, void* out, hipStream_t s) {
    if (rows <= 0 || emb <= 0) return RELM_MP_OK;
    return dtype == RELM_MP_F64
               ? rows_scale_t<double>(in, gather, div_kind, div_offsets, div_values, base, rows,
                                      emb, out, s)
               : rows_scale_t<float>(in, gather, div_kind, div_offsets, div_values, base, rows, emb,
                                     out, s);
}

int compute_gather_last(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                        const void* table, int64_t emb, void* out, hipStream_t s) {
    return compute_gather_last_grouped(dtype, plan, gathers, table, emb, 0, 0, out, s);
}

int compute_gather_last_grouped(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                                const void* table, int64_t emb, int64_t group,
                                int64_t group_stride, void* out, hipStream_t s) {
    if (plan.num_keys == 0 || emb == 0) return RELM_MP_OK;
    if (plan.kind == RELM_MP_PLAN_INVERSE && gathers == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: inverse plans need the gather array");
    return dtype == RELM_MP_F64
               ? gather_last_t<double>(plan, gathers, table, emb, out, group, group_stride, s)
               : gather_last_t<float>(plan, gathers, table, emb, out, group, group_stride, s);
}

int compute_segment_sum_grouped(int dtype, const relm_mp_plan& plan, const void* table,
                                int64_t emb, int64_t group, int64_t group_stride, void* out,
                                void* scratch, size_t scratch_bytes, hipStream_t s) {
    if (plan.num_keys == 0 || emb == 0) return RELM_MP_OK;
    if (plan.kind != RELM_MP_PLAN_CSR)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: grouped sums need a CSR plan");
    if (scratch_bytes < hub_partial_bytes(plan, emb, dtype, RELM_MP_MODE_SUM))
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: hub scratch too small");
    return dtype == RELM_MP_F64
               ? segment_sum_grouped_t<double>(plan, table, emb, group, group_stride, out, scratch, s)
               : segment_sum_grouped_t<float>(plan, table, emb, group, group_stride, out, scratch, s);
}

int compute_segment_reduce(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                           const void* table, int64_t emb, int64_t mode, void* out,
                           void* scratch, size_t scratch_bytes, hipStream_t s) {
    if (plan.num_keys == 0 || emb == 0) return RELM_MP_OK;
    if (mode != RELM_MP_MODE_SUM && mode != RELM_MP_MODE_LOGSUMEXP)
        return set_error(RELM_MP_ERR_UNSUPPORTED_MODE,
                         "Unsupported fanin_reduce mode. Supported: 0=sum, 1=logsumexp.");
    if (plan.kind == RELM_MP_PLAN_INVERSE) {
        if (mode != RELM_MP_MODE_SUM || plan.collisions != 0)
            return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                             "relm_mp: inverse plans reduce only injective keys with mode 0");
        return compute_gather_last(dtype, plan, gathers, table, emb, out, s);
    }
    if (scratch_bytes < hub_partial_bytes(plan, emb, dtype, mode))
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: hub scratch too small");
    if (dtype == RELM_MP_F64) {
        return mode == RELM_MP_MODE_SUM
                   ? segment_reduce_t<double, RELM_MP_MODE_SUM>(plan, table, emb, out, scratch, s)
                   : segment_reduce_t<double, RELM_MP_MODE_LOGSUMEXP>(plan, table, emb, out, scratch, s);
    }
    return mode == RELM_MP_MODE_SUM
               ? segment_reduce_t<float, RELM_MP_MODE_SUM>(plan, table, emb, out, scratch, s)
               : segment_reduce_t<float, RELM_MP_MODE_LOGSUMEXP>(plan, table, emb, out, scratch, s);
}

int compute_logsumexp_backward(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                               const void* grad_out, const void* out, const void* rel_flat,
                               int64_t emb, void* grad_rel, void* scratch, size_t scratch_bytes,
                               hipStream_t s) {
    if (plan.num_keys == 0 || emb == 0) return RELM_MP_OK;
    if (plan.kind == RELM_MP_PLAN_INVERSE) {
        if (plan.collisions != 0)
            return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                             "relm_mp: inverse plans reduce only injective keys");
        if (gathers == nullptr)
            return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                             "relm_mp: inverse plans need the gather array");
    } else if (scratch_bytes < hub_partial_bytes(plan, emb, dtype, RELM_MP_MODE_SUM)) {
        return set_error(RELM_MP_ERR_WORKSPACE, "relm_mp: hub scratch too small");
    }
    return dtype == RELM_MP_F64
               ? lse_backward_t<double>(plan, gathers, grad_out, out, rel_flat, emb, grad_rel, scratch, s)
               : lse_backward_t<float>(plan, gathers, grad_out, out, rel_flat, emb, grad_rel, scratch, s);
}

// The edge-order sum backward over a forward plan's snapshots
// (k_gather_edges); `counts` carries the inverse map's lost-edge count.
template <typename T>
int sum_backward_edges_t(const relm_mp_plan& fwd, const relm_mp_plan_counts* counts,
                         const void* grad_out_v, int64_t emb, void* grad_rel_v, hipStream_t s) {
    const T* grad_out = static_cast<const T*>(grad_out_v);
    T* grad_rel = static_cast<T*>(grad_rel_v);
    const int64_t E = fwd.num_edges;
    const GathersSnap rows{fwd.snap_gathers, fwd.snap_gather_plain};
    const GathersSnap dsts{fwd.snap_keys, fwd.snap_key_plain};
    const Geometry geo = choose_geometry<T>(emb, {grad_out, grad_rel});
    return with_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        hipLaunchKernelGGL((k_gather_edges<T, V, G>), row_grid(E, G, geo.slices, gather_rows_in_flight<T, V>()),
                           dim3(kThreads), 0, s, counts, E, rows, E, dsts, fwd.num_keys, grad_out, emb,
                           grad_rel);
        return hip_error(hipGetLastError(), "relm_mp edge-order sum backward kernel");
    });
}

int compute_backward_by_src(int dtype, const relm_mp_plan& dst_plan, const relm_mp_plan& inv_plan,
                            int64_t mode, const void* grad_out, const void* out,
                            const void* rel_flat, int64_t emb, void* grad_rel, hipStream_t s) {
    if (inv_plan.num_keys == 0 || emb == 0) return RELM_MP_OK;
    if (mode != RELM_MP_MODE_SUM && mode != RELM_MP_MODE_LOGSUMEXP)
        return set_error(RELM_MP_ERR_UNSUPPORTED_MODE,
                         "Unsupported fanin_reduce mode. Supported: 0=sum, 1=logsumexp.");
    // Rows in order through the inverse map, each row's destination from the
    // forward plan's int32 snapshot of dst_idx.  The sum backward with as many
    // message rows as edges (a flat_src without repeats - the device skips the
    // kernel otherwise - is then a permutation) runs in edge order instead, each
    // edge writing its own row whole, with no map to read: C2 in the callers'
    // layout 1.486 against 1.515 ms per step.  The logsumexp backward, which
    // also reads every message row, keeps the rows in order: in edge order the
    // callers' layout reads and writes every other row per sweep (1.802
    // against 1.777 ms).
    const bool by_edges = mode == RELM_MP_MODE_SUM && inv_plan.num_keys == dst_plan.num_edges;
    const relm_mp_plan* snap = &dst_plan;
    if (mode == RELM_MP_MODE_SUM) {
        // as the edge-order sum backward: grad_out and the destinations read
        // into the memory-side cache first when they fit
        const size_t elem = dtype == RELM_MP_F64 ? 8 : 4;
        const size_t tb = static_cast<size_t>(dst_plan.num_keys) * static_cast<size_t>(emb) * elem;
        const size_t ib = static_cast<size_t>(dst_plan.num_edges) * sizeof(int32_t);
        if (tb + ib <= kPrefetchMaxBytes && tb % 16 == 0 && ib % 16 == 0 &&
            (reinterpret_cast<uintptr_t>(grad_out) | reinterpret_cast<uintptr_t>(dst_plan.snap_keys)) % 16 == 0) {
            const int64_t units = static_cast<int64_t>((tb + ib) / 16);
            const int64_t blocks = std::min<int64_t>((units + kThreads * 8 - 1) / (kThreads * 8), 4096);
            hipLaunchKernelGGL(k_touch, dim3(static_cast<unsigned>(std::max<int64_t>(blocks, 1))),
                               dim3(kThreads), 0, s, static_cast<const uint4*>(grad_out),
                               static_cast<int64_t>(tb / 16), reinterpret_cast<const uint4*>(dst_plan.snap_keys),
                               static_cast<int64_t>(ib / 16));
            const int rc = hip_error(hipGetLastError(), "relm_mp prefetch kernel");
            if (rc != RELM_MP_OK) return rc;
        }
        if (by_edges)
            return dtype == RELM_MP_F64
                       ? sum_backward_edges_t<double>(dst_plan, inv_plan.counts, grad_out, emb, grad_rel, s)
                       : sum_backward_edges_t<float>(dst_plan, inv_plan.counts, grad_out, emb, grad_rel, s);
        return dtype == RELM_MP_F64
                   ? gather_last_t<double>(inv_plan, nullptr, grad_out, emb, grad_rel, 0, 0, s, snap, true)
                   : gather_last_t<float>(inv_plan, nullptr, grad_out, emb, grad_rel, 0, 0, s, snap, true);
    }
    return dtype == RELM_MP_F64
               ? lse_backward_t<double>(inv_plan, nullptr, grad_out, out, rel_flat, emb, grad_rel, nullptr, s, snap, true)
               : lse_backward_t<float>(inv_plan, nullptr, grad_out, out, rel_flat, emb, grad_rel, nullptr, s, snap, true);
}

int compute_backward_by_key(int dtype, const relm_mp_plan& plan, const int64_t* dst_idx,
                            int64_t mode, const void* grad_out, const void* out,
                            const void* rel_flat, int64_t emb, void* grad_rel, int64_t rel_rows,
                            hipStream_t s) {
    if (plan.kind != RELM_MP_PLAN_CSR || plan.gather_identity == 0)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         "relm_mp: backward by key needs a CSR plan whose gathered rows are the identity");
    if (mode != RELM_MP_MODE_SUM && mode != RELM_MP_MODE_LOGSUMEXP)
        return set_error(RELM_MP_ERR_UNSUPPORTED_MODE,
                         "Unsupported fanin_reduce mode. Supported: 0=sum, 1=logsumexp.");
    if (plan.num_edges > rel_rows)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT,
                         "relm_mp: backward by key needs num_edges <= rel_rows");
    if (dst_idx == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: dst_idx is NULL");
    // Message row e belongs to edge e alone, so the backward runs in edge
    // order over the identity inverse plan: rel_flat / grad_rel stream through
    // in order, the destination rows are gathered (rows >= num_edges get 0).
    // This beat walking the plan's segments, whose row writes scatter.
    relm_mp_plan ident{};
    ident.kind = RELM_MP_PLAN_INVERSE;
    ident.num_keys = rel_rows;
    ident.num_edges = plan.num_edges;
    ident.num_gather = plan.num_keys;
    // the destinations as the forward's plan keeps them (int32 snapshot, when
    // it keeps one): half the index bytes of dst_idx
    const relm_mp_plan* snap = plan.snap_keys != nullptr ? &plan : nullptr;
    if (rel_rows == 0 || emb == 0) return RELM_MP_OK;
    if (mode == RELM_MP_MODE_SUM) {
        // The sum backward writes every message row and reads only the
        // destination rows and dst_idx.  HBM sustains a pure write stream far
        // better than one with reads interleaved (C2: 0.40 ms against 0.62 ms
        // per launch when grad_out and dst_idx were not cached), so when both
        // fit the memory-side cache they are read into it first.
        const size_t elem = dtype == RELM_MP_F64 ? 8 : 4;
        const size_t tb = static_cast<size_t>(plan.num_keys) * static_cast<size_t>(emb) * elem;
        const void* idx = snap != nullptr ? static_cast<const void*>(plan.snap_keys) : dst_idx;
        const size_t ib = static_cast<size_t>(plan.num_edges) * (snap != nullptr ? sizeof(int32_t) : sizeof(int64_t));
        if (tb + ib <= kPrefetchMaxBytes && tb % 16 == 0 && ib % 16 == 0 &&
            (reinterpret_cast<uintptr_t>(grad_out) | reinterpret_cast<uintptr_t>(idx)) % 16 == 0) {
            const int64_t units = static_cast<int64_t>((tb + ib) / 16);
            const int64_t blocks = std::min<int64_t>((units + kThreads * 8 - 1) / (kThreads * 8), 4096);
            hipLaunchKernelGGL(k_touch, dim3(static_cast<unsigned>(std::max<int64_t>(blocks, 1))),
                               dim3(kThreads), 0, s, static_cast<const uint4*>(grad_out),
                               static_cast<int64_t>(tb / 16), static_cast<const uint4*>(idx),
                               static_cast<int64_t>(ib / 16));
            const int rc = hip_error(hipGetLastError(), "relm_mp prefetch kernel");
            if (rc != RELM_MP_OK) return rc;
        }
        return dtype == RELM_MP_F64
                   ? gather_last_t<double>(ident, dst_idx, grad_out, emb, grad_rel, 0, 0, s, snap)
                   : gather_last_t<float>(ident, dst_idx, grad_out, emb, grad_rel, 0, 0, s, snap);
    }
    return dtype == RELM_MP_F64
               ? lse_backward_t<double>(ident, dst_idx, grad_out, out, rel_flat, emb, grad_rel, nullptr, s, snap)
               : lse_backward_t<float>(ident, dst_idx, grad_out, out, rel_flat, emb, grad_rel, nullptr, s, snap);
}

}  // namespace relm_mp
