// Row kernels of the relational message-passing ops.
//
// Every output row is written exactly once by one "row group" of G lanes
// (G = 4..64, a divisor of the wave), each lane moving V contiguous elements
// (float4 / double2 when the rows allow it).  Rows wider than G*V are split
// over blockIdx.y slices.  No atomics: a key's messages are visited in the
// stable (edge) order of the plan, so results are deterministic and, for
// segments up to kHubThreshold messages, the fp32 sums are bit-identical to a
// sequential loop in edge order.  Longer segments ("hubs") are cut into chunks
// of kChunkSize messages; chunk partials are combined in chunk order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "device_utils.h"
#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kThreads = 256;
constexpr int64_t kMaxBlocksX = 1 << 22;  // keeps blocks * 256 threads below 2^32

template <int G>
constexpr int batch_rows() {
    return G < 8 ? G : 8;
}

struct Span {
    int64_t beg;
    int64_t end;
};

__device__ __forceinline__ Span segment(const int32_t* __restrict__ offsets, int64_t key,
                                        int64_t num_edges) {
    int64_t b = offsets[key];
    int64_t e = offsets[key + 1];
    b = b < 0 ? 0 : (b > num_edges ? num_edges : b);
    e = e < b ? b : (e > num_edges ? num_edges : e);
    return {b, e};
}

// ---- accumulators --------------------------------------------------------

template <typename T, int V>
struct SumAcc {
    Pack<T, V> acc;
    __device__ __forceinline__ void init() { acc = pack_fill<T, V>(T(0)); }
    template <int U>
    __device__ __forceinline__ void batch(const Pack<T, V> (&x)[U], int valid) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u < valid) {
#pragma unroll
                for (int i = 0; i < V; ++i) acc.v[i] = acc.v[i] + x[u].v[i];
            }
        }
    }
};

// Blocked max-then-sum: per batch of rows, the batch maximum first, then the
// exponentials against the running maximum.  s is kept relative to m; while
// m is -inf, s stays 0.
template <typename T, int V>
struct LseAcc {
    Pack<T, V> m;
    Pack<T, V> s;
    __device__ __forceinline__ void init() {
        m = pack_fill<T, V>(neg_inf<T>());
        s = pack_fill<T, V>(T(0));
    }
    template <int U>
    __device__ __forceinline__ void batch(const Pack<T, V> (&x)[U], int valid) {
#pragma unroll
        for (int i = 0; i < V; ++i) {
            T mb = neg_inf<T>();
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (u < valid) mb = max_nan(mb, x[u].v[i]);
            const T nm = max_nan(m.v[i], mb);
            if (nm != neg_inf<T>()) {
                T acc = s.v[i] * dev_exp<T>(m.v[i] - nm);
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (u < valid) acc = acc + dev_exp<T>(x[u].v[i] - nm);
                s.v[i] = acc;
                m.v[i] = nm;
            }
        }
    }
};

// grad_out[d] * exp(x_r - out[d]) accumulated in edge order.
template <typename T, int V>
struct LseBwdAcc {
    Pack<T, V> acc;
    Pack<T, V> xr;
    __device__ __forceinline__ void init() { acc = pack_fill<T, V>(T(0)); }
    template <int U>
    __device__ __forceinline__ void batch2(const Pack<T, V> (&g)[U], const Pack<T, V> (&o)[U],
                                           int valid) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u < valid) {
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    const T w = dev_exp<T>(xr.v[i] - o[u].v[i]);
                    const T c = g[u].v[i] * w;
                    acc.v[i] = acc.v[i] + c;
                }
            }
        }
    }
};

template <typename T, int V>
__device__ __forceinline__ Pack<T, V> lse_finish(const LseAcc<T, V>& a, bool nonempty) {
    Pack<T, V> r;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        if (!nonempty) {
            r.v[i] = neg_inf<T>();
        } else if (a.m.v[i] == neg_inf<T>()) {
            r.v[i] = quiet_nan<T>();  // every message is -inf: exp(-inf - -inf) is NaN
        } else {
            r.v[i] = dev_log<T>(a.s.v[i]) + a.m.v[i];
        }
    }
    return r;
}

// Visits positions [beg, end) of `gs` in order, in batches of U rows of
// `table` (row index = gs[pos]); lanes of the group load the batch's indices
// cooperatively and broadcast them with a group shuffle.
template <typename T, int V, int G, typename Acc>
__device__ __forceinline__ void reduce_rows(Acc& acc, const int32_t* __restrict__ gs, int64_t beg,
                                            int64_t end, const T* __restrict__ table, int64_t D,
                                            int64_t col, bool colok, int gl) {
    constexpr int U = batch_rows<G>();
    for (int64_t i = beg; i < end; i += G) {
        const int cnt = static_cast<int>(end - i < G ? end - i : G);
        const int32_t my = gl < cnt ? gs[i + gl] : 0;
        for (int t0 = 0; t0 < cnt; t0 += U) {
            Pack<T, V> x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int32_t g = __shfl(my, t0 + u, G);
                if (t0 + u < cnt && colok)
                    x[u] = pack_load<T, V>(table + static_cast<int64_t>(g) * D + col);
                else
                    x[u] = pack_fill<T, V>(T(0));
            }
            if (colok) acc.template batch<U>(x, cnt - t0);
        }
    }
}

template <typename T, int V, int G>
__device__ __forceinline__ void reduce_rows_lse_bwd(LseBwdAcc<T, V>& acc,
                                                    const int32_t* __restrict__ gs, int64_t beg,
                                                    int64_t end, const T* __restrict__ grad_out,
                                                    const T* __restrict__ out, int64_t D,
                                                    int64_t col, bool colok, int gl) {
    constexpr int U = batch_rows<G>();
    for (int64_t i = beg; i < end; i += G) {
        const int cnt = static_cast<int>(end - i < G ? end - i : G);
        const int32_t my = gl < cnt ? gs[i + gl] : 0;
        for (int t0 = 0; t0 < cnt; t0 += U) {
            Pack<T, V> g[U], o[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int32_t d = __shfl(my, t0 + u, G);
                if (t0 + u < cnt && colok) {
                    const int64_t off = static_cast<int64_t>(d) * D + col;
                    g[u] = pack_load<T, V>(grad_out + off);
                    o[u] = pack_load<T, V>(out + off);
                } else {
                    g[u] = pack_fill<T, V>(T(0));
                    o[u] = pack_fill<T, V>(T(0));
                }
            }
            if (colok) acc.template batch2<U>(g, o, cnt - t0);
        }
    }
}

// ---- kernels -------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(kThreads) void k_fill(T* __restrict__ p, int64_t n, T value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        p[i] = value;
}

// out[r] = table[gathers[inv[r]]] or 0 (inverse plans: fanout forward and
// injective sum backward).
template <typename T, int V, int G>
__global__ __launch_bounds__(kThreads) void k_gather_inv(const int32_t* __restrict__ inv,
                                                         const int64_t* __restrict__ gathers,
                                                         int64_t num_gather,
                                                         const T* __restrict__ table,
                                                         int64_t num_keys, int64_t D,
                                                         T* __restrict__ out) {
    constexpr int R = kThreads / G;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    if (col >= D) return;
    for (int64_t key = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / G; key < num_keys;
         key += static_cast<int64_t>(gridDim.x) * R) {
        const int32_t e = inv[key];
        Pack<T, V> v = pack_fill<T, V>(T(0));
        if (e >= 0) {
            const int64_t g = gathers[e];
            if (static_cast<uint64_t>(g) < static_cast<uint64_t>(num_gather))
                v = pack_load<T, V>(table + g * D + col);
        }
        pack_store_stream<T, V>(out + key * D + col, v);
    }
}

// out[k] = table[gather of the last edge of segment k] or 0 (CSR plans).
template <typename T, int V, int G>
__global__ __launch_bounds__(kThreads) void k_gather_last_csr(const int32_t* __restrict__ offsets,
                                                              const int32_t* __restrict__ gs,
                                                              int64_t num_edges,
                                                              const T* __restrict__ table,
                                                              int64_t num_keys, int64_t D,
                                                              T* __restrict__ out) {
    constexpr int R = kThreads / G;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    if (col >= D) return;
    for (int64_t key = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / G; key < num_keys;
         key += static_cast<int64_t>(gridDim.x) * R) {
        const Span sp = segment(offsets, key, num_edges);
        Pack<T, V> v = pack_fill<T, V>(T(0));
        if (sp.end > sp.beg) v = pack_load<T, V>(table + static_cast<int64_t>(gs[sp.end - 1]) * D + col);
        pack_store_stream<T, V>(out + key * D + col, v);
    }
}

// Segments with at most kHubThreshold messages: one row group per key, the
// messages in edge order.
template <typename T, int V, int G, int MODE>
__global__ __launch_bounds__(kThreads) void k_segment_short(const int32_t* __restrict__ offsets,
                                                            const int32_t* __restrict__ gs,
                                                            int64_t num_edges,
                                                            const T* __restrict__ table,
                                                            int64_t num_keys, int64_t D,
                                                            T* __restrict__ out) {
    constexpr int R = kThreads / G;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    const bool colok = col < D;
    for (int64_t key = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / G; key < num_keys;
         key += static_cast<int64_t>(gridDim.x) * R) {
        const Span sp = segment(offsets, key, num_edges);
        if (sp.end - sp.beg > kHubThreshold) continue;
        if constexpr (MODE == RELM_MP_MODE_SUM) {
            SumAcc<T, V> acc;
            acc.init();
            reduce_rows<T, V, G>(acc, gs, sp.beg, sp.end, table, D, col, colok, gl);
            if (colok) pack_store_stream<T, V>(out + key * D + col, acc.acc);
        } else {
            LseAcc<T, V> acc;
            acc.init();
            reduce_rows<T, V, G>(acc, gs, sp.beg, sp.end, table, D, col, colok, gl);
            if (colok)
                pack_store_stream<T, V>(out + key * D + col, lse_finish<T, V>(acc, sp.end > sp.beg));
        }
    }
}

struct HubChunk {
    int64_t key;
    int64_t beg;
    int64_t end;
    bool ok;
};

__device__ __forceinline__ HubChunk hub_chunk(int64_t c, const int32_t* __restrict__ offsets,
                                              const int32_t* __restrict__ hub_key,
                                              const int32_t* __restrict__ hub_chunk_base,
                                              const int32_t* __restrict__ chunk_hub,
                                              int64_t num_hubs, int64_t num_edges) {
    HubChunk hc{0, 0, 0, false};
    const int64_t h = chunk_hub[c];
    if (h < 0 || h >= num_hubs) return hc;
    hc.key = hub_key[h];
    const int64_t j = c - hub_chunk_base[h];
    const Span sp = segment(offsets, hc.key, num_edges);
    hc.beg = sp.beg + j * kChunkSize;
    if (hc.beg < sp.beg) hc.beg = sp.beg;
    if (hc.beg > sp.end) hc.beg = sp.end;
    hc.end = hc.beg + kChunkSize < sp.end ? hc.beg + kChunkSize : sp.end;
    hc.ok = true;
    return hc;
}

// Hub chunk partials: sum -> partial[c][D]; logsumexp -> (m, s) in
// partial[c][0:D], partial[c][D:2D]; logsumexp backward -> sum.
template <typename T, int V, int G, int MODE>
__global__ __launch_bounds__(kThreads) void k_hub_partial(
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ gs, int64_t num_edges,
    const T* __restrict__ table, int64_t D, const int32_t* __restrict__ hub_key,
    const int32_t* __restrict__ hub_chunk_base, const int32_t* __restrict__ chunk_hub,
    int64_t num_hubs, int64_t num_chunks, T* __restrict__ partial) {
    constexpr int R = kThreads / G;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    const bool colok = col < D;
    for (int64_t c = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / G; c < num_chunks;
         c += static_cast<int64_t>(gridDim.x) * R) {
        const HubChunk hc =
            hub_chunk(c, offsets, hub_key, hub_chunk_base, chunk_hub, num_hubs, num_edges);
        const int64_t beg = hc.ok ? hc.beg : 0;
        const int64_t end = hc.ok ? hc.end : 0;
        if constexpr (MODE == RELM_MP_MODE_SUM) {
            SumAcc<T, V> acc;
            acc.init();
            reduce_rows<T, V, G>(acc, gs, beg, end, table, D, col, colok, gl);
            if (colok) pack_store<T, V>(partial + c * D + col, acc.acc);
        } else {
            LseAcc<T, V> acc;
            acc.init();
            reduce_rows<T, V, G>(acc, gs, beg, end, table, D, col, colok, gl);
            if (colok) {
                pack_store<T, V>(partial + c * 2 * D + col, acc.m);
                pack_store<T, V>(partial + c * 2 * D + D + col, acc.s);
            }
        }
    }
}

// Combines the chunk partials of one hub per block, in chunk order: group g
// folds a contiguous range of chunks, then group results are folded in group
// order.
template <typename T, int V, int G, int MODE>
__global__ __launch_bounds__(kThreads) void k_hub_combine(const int32_t* __restrict__ offsets,
                                                          int64_t num_edges, int64_t D,
                                                          const int32_t* __restrict__ hub_key,
                                                          const int32_t* __restrict__ hub_chunk_base,
                                                          int64_t num_hubs, int64_t num_chunks,
                                                          const T* __restrict__ partial,
                                                          T* __restrict__ out) {
    constexpr int NG = kThreads / G;
    __shared__ Pack<T, V> red_a[kThreads];
    __shared__ Pack<T, V> red_b[kThreads];
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int grp = static_cast<int>(threadIdx.x) / G;
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    const bool colok = col < D;
    for (int64_t h = blockIdx.x; h < num_hubs; h += gridDim.x) {
        const int64_t key = hub_key[h];
        const Span sp = segment(offsets, key, num_edges);
        const int64_t nch_all = (sp.end - sp.beg + kChunkSize - 1) / kChunkSize;
        int64_t base = hub_chunk_base[h];
        int64_t nch = nch_all;
        if (base < 0) base = 0;
        if (base + nch > num_chunks) nch = num_chunks - base > 0 ? num_chunks - base : 0;
        const int64_t per = (nch + NG - 1) / NG;
        const int64_t lo = grp * per < nch ? grp * per : nch;
        const int64_t hi = lo + per < nch ? lo + per : nch;
        if constexpr (MODE == RELM_MP_MODE_SUM) {
            Pack<T, V> acc = pack_fill<T, V>(T(0));
            if (colok) {
                for (int64_t c = lo; c < hi; ++c) {
                    const Pack<T, V> x = pack_load<T, V>(partial + (base + c) * D + col);
#pragma unroll
                    for (int i = 0; i < V; ++i) acc.v[i] = acc.v[i] + x.v[i];
                }
            }
            red_a[threadIdx.x] = acc;
            __syncthreads();
            if (grp == 0 && colok) {
                Pack<T, V> tot = pack_fill<T, V>(T(0));
                for (int g = 0; g < NG; ++g) {
                    const Pack<T, V> x = red_a[g * G + gl];
#pragma unroll
                    for (int i = 0; i < V; ++i) tot.v[i] = tot.v[i] + x.v[i];
                }
                pack_store<T, V>(out + key * D + col, tot);
            }
            __syncthreads();
        } else {
            Pack<T, V> M = pack_fill<T, V>(neg_inf<T>());
            Pack<T, V> S = pack_fill<T, V>(T(0));
            if (colok) {
                for (int64_t c = lo; c < hi; ++c) {
                    const Pack<T, V> m = pack_load<T, V>(partial + (base + c) * 2 * D + col);
#pragma unroll
                    for (int i = 0; i < V; ++i) M.v[i] = max_nan(M.v[i], m.v[i]);
                }
                for (int64_t c = lo; c < hi; ++c) {
                    const Pack<T, V> m = pack_load<T, V>(partial + (base + c) * 2 * D + col);
                    const Pack<T, V> s = pack_load<T, V>(partial + (base + c) * 2 * D + D + col);
#pragma unroll
                    for (int i = 0; i < V; ++i)
                        if (M.v[i] != neg_inf<T>())
                            S.v[i] = S.v[i] + s.v[i] * dev_exp<T>(m.v[i] - M.v[i]);
                }
            }
            red_a[threadIdx.x] = M;
            red_b[threadIdx.x] = S;
            __syncthreads();
            if (grp == 0 && colok) {
                Pack<T, V> MM = pack_fill<T, V>(neg_inf<T>());
                for (int g = 0; g < NG; ++g) {
                    const Pack<T, V> m = red_a[g * G + gl];
#pragma unroll
                    for (int i = 0; i < V; ++i) MM.v[i] = max_nan(MM.v[i], m.v[i]);
                }
                Pack<T, V> SS = pack_fill<T, V>(T(0));
                for (int g = 0; g < NG; ++g) {
                    const Pack<T, V> m = red_a[g * G + gl];
                    const Pack<T, V> s = red_b[g * G + gl];
#pragma unroll
                    for (int i = 0; i < V; ++i)
                        if (MM.v[i] != neg_inf<T>())
                            SS.v[i] = SS.v[i] + s.v[i] * dev_exp<T>(m.v[i] - MM.v[i]);
                }
                Pack<T, V> r;
#pragma unroll
                for (int i = 0; i < V; ++i)
                    r.v[i] = MM.v[i] == neg_inf<T>() ? quiet_nan<T>() : dev_log<T>(SS.v[i]) + MM.v[i];
                pack_store<T, V>(out + key * D + col, r);
            }
            __syncthreads();
        }
    }
}

// Logsumexp backward with an inverse plan (injective keys):
// grad_rel[r] = grad_out[d] * exp(rel[r] - out[d]), d = gathers[inv[r]], or 0.
template <typename T, int V, int G>
__global__ __launch_bounds__(kThreads) void k_lse_bwd_inv(
    const int32_t* __restrict__ inv, const int64_t* __restrict__ gathers, int64_t num_gather,
    const T* __restrict__ grad_out, const T* __restrict__ out, const T* __restrict__ rel,
    int64_t num_keys, int64_t D, T* __restrict__ grad_rel) {
    constexpr int R = kThreads / G;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    if (col >= D) return;
    for (int64_t key = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / G; key < num_keys;
         key += static_cast<int64_t>(gridDim.x) * R) {
        const int32_t e = inv[key];
        Pack<T, V> r = pack_fill<T, V>(T(0));
        if (e >= 0) {
            const int64_t d = gathers[e];
            if (static_cast<uint64_t>(d) < static_cast<uint64_t>(num_gather)) {
                const Pack<T, V> x = pack_load<T, V>(rel + key * D + col);
                const Pack<T, V> g = pack_load<T, V>(grad_out + d * D + col);
                const Pack<T, V> o = pack_load<T, V>(out + d * D + col);
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    const T w = dev_exp<T>(x.v[i] - o.v[i]);
                    const T c = g.v[i] * w;
                    r.v[i] = T(0) + c;
                }
            }
        }
        pack_store_stream<T, V>(grad_rel + key * D + col, r);
    }
}

// Logsumexp backward with a CSR plan keyed by flat_src: short segments.
template <typename T, int V, int G>
__global__ __launch_bounds__(kThreads) void k_lse_bwd_short(
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ gs, int64_t num_edges,
    const T* __restrict__ grad_out, const T* __restrict__ out, const T* __restrict__ rel,
    int64_t num_keys, int64_t D, T* __restrict__ grad_rel) {
    constexpr int R = kThreads / G;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    const bool colok = col < D;
    for (int64_t key = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / G; key < num_keys;
         key += static_cast<int64_t>(gridDim.x) * R) {
        const Span sp = segment(offsets, key, num_edges);
        if (sp.end - sp.beg > kHubThreshold) continue;
        LseBwdAcc<T, V> acc;
        acc.init();
        acc.xr = pack_fill<T, V>(T(0));
        if (colok && sp.end > sp.beg) acc.xr = pack_load<T, V>(rel + key * D + col);
        reduce_rows_lse_bwd<T, V, G>(acc, gs, sp.beg, sp.end, grad_out, out, D, col, colok, gl);
        if (colok) pack_store_stream<T, V>(grad_rel + key * D + col, acc.acc);
    }
}

template <typename T, int V, int G>
__global__ __launch_bounds__(kThreads) void k_lse_bwd_hub_partial(
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ gs, int64_t num_edges,
    const T* __restrict__ grad_out, const T* __restrict__ out, const T* __restrict__ rel,
    int64_t D, const int32_t* __restrict__ hub_key, const int32_t* __restrict__ hub_chunk_base,
    const int32_t* __restrict__ chunk_hub, int64_t num_hubs, int64_t num_chunks,
    T* __restrict__ partial) {
    constexpr int R = kThreads / G;
    const int gl = static_cast<int>(threadIdx.x) & (G - 1);
    const int64_t col = static_cast<int64_t>(blockIdx.y) * (G * V) + static_cast<int64_t>(gl) * V;
    const bool colok = col < D;
    for (int64_t c = static_cast<int64_t>(blockIdx.x) * R + threadIdx.x / G; c < num_chunks;
         c += static_cast<int64_t>(gridDim.x) * R) {
        const HubChunk hc =
            hub_chunk(c, offsets, hub_key, hub_chunk_base, chunk_hub, num_hubs, num_edges);
        LseBwdAcc<T, V> acc;
        acc.init();
        acc.xr = pack_fill<T, V>(T(0));
        if (colok && hc.ok) acc.xr = pack_load<T, V>(rel + hc.key * D + col);
        reduce_rows_lse_bwd<T, V, G>(acc, gs, hc.ok ? hc.beg : 0, hc.ok ? hc.end : 0, grad_out,
                                     out, D, col, colok, gl);
        if (colok) pack_store<T, V>(partial + c * D + col, acc.acc);
    }
}

// ---- host-side dispatch --------------------------------------------------

struct Geometry {
    int V;
    int G;
    int64_t slices;
};

template <typename T>
Geometry choose_geometry(int64_t D, std::initializer_list<const void*> ptrs) {
    constexpr int kVecMax = 16 / static_cast<int>(sizeof(T));
    int V = kVecMax;
    if (D % V != 0) V = 1;
    for (const void* p : ptrs) {
        if (p != nullptr && reinterpret_cast<uintptr_t>(p) % (sizeof(T) * V) != 0) V = 1;
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
    return by_g(std::integral_constant<int, 1>{});
}

dim3 row_grid(int64_t rows, int G, int64_t slices) {
    const int64_t per = kThreads / G;
    int64_t bx = (rows + per - 1) / per;
    if (bx < 1) bx = 1;
    if (bx > kMaxBlocksX) bx = kMaxBlocksX;
    return dim3(static_cast<unsigned>(bx), static_cast<unsigned>(slices));
}

template <typename T>
int gather_last_t(const relm_mp_plan& plan, const int64_t* gathers, const void* table_v,
                  int64_t emb, void* out_v, hipStream_t s) {
    const T* table = static_cast<const T*>(table_v);
    T* out = static_cast<T*>(out_v);
    const Geometry geo = choose_geometry<T>(emb, {table, out});
    return with_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        const dim3 grid = row_grid(plan.num_keys, G, geo.slices);
        if (plan.kind == RELM_MP_PLAN_INVERSE) {
            hipLaunchKernelGGL((k_gather_inv<T, V, G>), grid, dim3(kThreads), 0, s, plan.inv,
                               gathers, plan.num_gather, table, plan.num_keys, emb, out);
        } else {
            hipLaunchKernelGGL((k_gather_last_csr<T, V, G>), grid, dim3(kThreads), 0, s,
                               plan.offsets, plan.gather_sorted, plan.num_edges, table,
                               plan.num_keys, emb, out);
        }
        return hip_error(hipGetLastError(), "relm_mp gather kernel");
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
        hipLaunchKernelGGL((k_segment_short<T, V, G, MODE>), row_grid(plan.num_keys, G, geo.slices),
                           dim3(kThreads), 0, s, plan.offsets, plan.gather_sorted, plan.num_edges,
                           table, plan.num_keys, emb, out);
        int rc = hip_error(hipGetLastError(), "relm_mp segment kernel");
        if (rc != RELM_MP_OK || plan.num_hubs == 0) return rc;
        hipLaunchKernelGGL((k_hub_partial<T, V, G, MODE>), row_grid(plan.num_chunks, G, geo.slices),
                           dim3(kThreads), 0, s, plan.offsets, plan.gather_sorted, plan.num_edges,
                           table, emb, plan.hub_key, plan.hub_chunk_base, plan.chunk_hub,
                           plan.num_hubs, plan.num_chunks, partial);
        rc = hip_error(hipGetLastError(), "relm_mp hub partial kernel");
        if (rc != RELM_MP_OK) return rc;
        const unsigned hb = static_cast<unsigned>(std::min<int64_t>(plan.num_hubs, kMaxBlocksX));
        hipLaunchKernelGGL((k_hub_combine<T, V, G, MODE>), dim3(hb, static_cast<unsigned>(geo.slices)),
                           dim3(kThreads), 0, s, plan.offsets, plan.num_edges, emb, plan.hub_key,
                           plan.hub_chunk_base, plan.num_hubs, plan.num_chunks,
                           static_cast<const T*>(partial), out);
        return hip_error(hipGetLastError(), "relm_mp hub combine kernel");
    });
}

template <typename T>
int lse_backward_t(const relm_mp_plan& plan, const int64_t* gathers, const void* grad_out_v,
                   const void* out_v, const void* rel_v, int64_t emb, void* grad_rel_v,
                   void* scratch, hipStream_t s) {
    const T* grad_out = static_cast<const T*>(grad_out_v);
    const T* out = static_cast<const T*>(out_v);
    const T* rel = static_cast<const T*>(rel_v);
    T* grad_rel = static_cast<T*>(grad_rel_v);
    T* partial = static_cast<T*>(scratch);
    const Geometry geo = choose_geometry<T>(emb, {grad_out, out, rel, grad_rel, partial});
    return with_geometry<T>(geo, [&](auto vt, auto gt) -> int {
        constexpr int V = decltype(vt)::value;
        constexpr int G = decltype(gt)::value;
        const dim3 grid = row_grid(plan.num_keys, G, geo.slices);
        if (plan.kind == RELM_MP_PLAN_INVERSE) {
            hipLaunchKernelGGL((k_lse_bwd_inv<T, V, G>), grid, dim3(kThreads), 0, s, plan.inv,
                               gathers, plan.num_gather, grad_out, out, rel, plan.num_keys, emb,
                               grad_rel);
            return hip_error(hipGetLastError(), "relm_mp logsumexp backward kernel");
        }
        hipLaunchKernelGGL((k_lse_bwd_short<T, V, G>), grid, dim3(kThreads), 0, s, plan.offsets,
                           plan.gather_sorted, plan.num_edges, grad_out, out, rel, plan.num_keys,
                           emb, grad_rel);
        int rc = hip_error(hipGetLastError(), "relm_mp logsumexp backward kernel");
        if (rc != RELM_MP_OK || plan.num_hubs == 0) return rc;
        hipLaunchKernelGGL((k_lse_bwd_hub_partial<T, V, G>), row_grid(plan.num_chunks, G, geo.slices),
                           dim3(kThreads), 0, s, plan.offsets, plan.gather_sorted, plan.num_edges,
                           grad_out, out, rel, emb, plan.hub_key, plan.hub_chunk_base,
                           plan.chunk_hub, plan.num_hubs, plan.num_chunks, partial);
        rc = hip_error(hipGetLastError(), "relm_mp logsumexp backward hub kernel");
        if (rc != RELM_MP_OK) return rc;
        const unsigned hb = static_cast<unsigned>(std::min<int64_t>(plan.num_hubs, kMaxBlocksX));
        hipLaunchKernelGGL((k_hub_combine<T, V, G, RELM_MP_MODE_SUM>),
                           dim3(hb, static_cast<unsigned>(geo.slices)), dim3(kThreads), 0, s,
                           plan.offsets, plan.num_edges, emb, plan.hub_key, plan.hub_chunk_base,
                           plan.num_hubs, plan.num_chunks, static_cast<const T*>(partial),
                           grad_rel);
        return hip_error(hipGetLastError(), "relm_mp logsumexp backward combine kernel");
    });
}

}  // namespace

size_t hub_partial_bytes(const relm_mp_plan& plan, int64_t emb, int dtype, int64_t mode) {
    if (plan.kind != RELM_MP_PLAN_CSR || plan.num_chunks == 0) return 0;
    const size_t elem = dtype == RELM_MP_F64 ? 8 : 4;
    const size_t per = static_cast<size_t>(emb) * elem * (mode == RELM_MP_MODE_LOGSUMEXP ? 2 : 1);
    return static_cast<size_t>(plan.num_chunks) * per;
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

int compute_gather_last(int dtype, const relm_mp_plan& plan, const int64_t* gathers,
                        const void* table, int64_t emb, void* out, hipStream_t s) {
    if (plan.num_keys == 0 || emb == 0) return RELM_MP_OK;
    if (plan.kind == RELM_MP_PLAN_INVERSE && gathers == nullptr)
        return set_error(RELM_MP_ERR_INVALID_ARGUMENT, "relm_mp: inverse plans need the gather array");
    return dtype == RELM_MP_F64 ? gather_last_t<double>(plan, gathers, table, emb, out, s)
                                : gather_last_t<float>(plan, gathers, table, emb, out, s);
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

}  // namespace relm_mp
