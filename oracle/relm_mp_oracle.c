/*
 * relm_mp_oracle.c - CPU restatement of relmo's message-passing ops, used ONLY
 * as a checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline.
 * Nothing in the product (relmo_amd/) links, loads or calls this file.
 *
 * Every function restates the reference CPU lane of
 * maichmueller/relmo src/_ops/mp/mp_ops.cpp (file:line given per function):
 * sequential loops in edge order, single-threaded, bounds-checked with the
 * reference's check order.  fp32 arithmetic is plain IEEE (built with
 * -ffp-contract=off), so the sum paths reproduce the reference's bits.
 *
 * Bounds errors return ORACLE_BAD_INDEX and fill *bad (which array, edge,
 * value, bound) instead of throwing.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_BAD_INDEX 2

typedef struct oracle_bad {
    int32_t which; /* 0: first index array argument, 1: second */
    int32_t pad;
    int64_t edge;
    int64_t value;
    int64_t bound;
} oracle_bad;

static int bad_index(oracle_bad* bad, int which, int64_t e, int64_t v, int64_t bound) {
    if (bad) {
        bad->which = which;
        bad->edge = e;
        bad->value = v;
        bad->bound = bound;
    }
    return ORACLE_BAD_INDEX;
}

static int in_bounds(int64_t v, int64_t n) { return v >= 0 && v < n; }

/* NaN-propagating maximum: ATen's scatter_reduce "amax" keeps a NaN once seen. */
static float max_nan_f(float a, float b) { return (isnan(b) || b > a) ? b : a; }
static double max_nan_d(double a, double b) { return (isnan(b) || b > a) ? b : a; }

/* ---- mp_ops.cpp:2815-2836 fanout_scatter_cpu_kernel --------------------
 * out zero-filled; for e in order: check src (x_rows) then dst (out_rows);
 * copy x[src[e]] to out[dst[e]] (the last edge wins on duplicates). */
#define DEF_FANOUT(T, S)                                                                        \
    int oracle_fanout_scatter_##S(const T* x, int64_t x_rows, int64_t emb, const int64_t* src, \
                                  const int64_t* dst, int64_t n, int64_t out_rows, T* out,      \
                                  oracle_bad* bad) {                                            \
        memset(out, 0, (size_t)(out_rows * emb) * sizeof(T));                                   \
        for (int64_t e = 0; e < n; ++e) {                                                       \
            const int64_t s = src[e], d = dst[e];                                               \
            if (!in_bounds(s, x_rows)) return bad_index(bad, 0, e, s, x_rows);                  \
            if (!in_bounds(d, out_rows)) return bad_index(bad, 1, e, d, out_rows);              \
            memcpy(out + d * emb, x + s * emb, (size_t)emb * sizeof(T));                        \
        }                                                                                       \
        return ORACLE_OK;                                                                       \
    }
DEF_FANOUT(float, f32)
DEF_FANOUT(double, f64)

/* Shared accumulate loop: out[w[e]] += in[r[e]] in edge order, checking the
 * write index w first (mp_ops.cpp:2838-2861, 2888-2911) or the read index r
 * first (mp_ops.cpp:2863-2886).  which=0 names the r array, 1 the w array. */
#define DEF_ACCUM(T, S)                                                                         \
    static int accumulate_##S(const T* in, int64_t in_rows, const int64_t* r, const int64_t* w, \
                              int64_t n, int64_t out_rows, int64_t emb, T* out,                 \
                              int read_first, int r_which, oracle_bad* bad) {                   \
        memset(out, 0, (size_t)(out_rows * emb) * sizeof(T));                                   \
        for (int64_t e = 0; e < n; ++e) {                                                       \
            const int64_t ri = r[e], wi = w[e];                                                 \
            if (read_first) {                                                                   \
                if (!in_bounds(ri, in_rows)) return bad_index(bad, r_which, e, ri, in_rows);    \
                if (!in_bounds(wi, out_rows)) return bad_index(bad, 1 - r_which, e, wi, out_rows); \
            } else {                                                                            \
                if (!in_bounds(wi, out_rows)) return bad_index(bad, 1 - r_which, e, wi, out_rows); \
                if (!in_bounds(ri, in_rows)) return bad_index(bad, r_which, e, ri, in_rows);    \
            }                                                                                   \
            const T* src_row = in + ri * emb;                                                   \
            T* dst_row = out + wi * emb;                                                        \
            for (int64_t k = 0; k < emb; ++k) dst_row[k] += src_row[k];                         \
        }                                                                                       \
        return ORACLE_OK;                                                                       \
    }
DEF_ACCUM(float, f32)
DEF_ACCUM(double, f64)

/* ---- mp_ops.cpp:2838-2861 fanout_scatter_backward_cpu_kernel ------------
 * grad_x[src[e]] += grad_out[dst[e]]; src checked before dst.
 * which: 0 = src_global_idx, 1 = flat_dst. */
#define DEF_FANOUT_BWD(T, S)                                                                        \
    int oracle_fanout_scatter_backward_##S(const T* grad_out, int64_t grad_out_rows, int64_t emb,  \
                                           const int64_t* src, const int64_t* dst, int64_t n,      \
                                           int64_t x_rows, T* grad_x, oracle_bad* bad) {           \
        /* read index = dst (which 1), write index = src (which 0) */                              \
        return accumulate_##S(grad_out, grad_out_rows, dst, src, n, x_rows, emb, grad_x, 0, 1, bad); \
    }
DEF_FANOUT_BWD(float, f32)
DEF_FANOUT_BWD(double, f64)

/* ---- mp_ops.cpp:2863-2886 fanin_reduce_sum_cpu_kernel --------------------
 * out[dst[e]] += rel[flat_src[e]]; flat_src checked before dst_idx.
 * which: 0 = flat_src, 1 = dst_idx. */
#define DEF_FANIN_SUM(T, S)                                                                     \
    int oracle_fanin_reduce_sum_##S(const T* rel, int64_t rel_rows, int64_t emb,                \
                                    const int64_t* flat_src, const int64_t* dst, int64_t n,     \
                                    int64_t dim_size, T* out, oracle_bad* bad) {                \
        return accumulate_##S(rel, rel_rows, flat_src, dst, n, dim_size, emb, out, 1, 0, bad);  \
    }
DEF_FANIN_SUM(float, f32)
DEF_FANIN_SUM(double, f64)

/* ---- mp_ops.cpp:2888-2911 fanin_reduce_sum_backward_cpu_kernel -----------
 * grad_rel[flat_src[e]] += grad_out[dst[e]]; flat_src checked before dst_idx.
 * which: 0 = flat_src, 1 = dst_idx. */
#define DEF_FANIN_SUM_BWD(T, S)                                                                     \
    int oracle_fanin_reduce_sum_backward_##S(const T* grad_out, int64_t grad_out_rows, int64_t emb, \
                                             const int64_t* flat_src, const int64_t* dst,           \
                                             int64_t n, int64_t rel_rows, T* grad_rel,              \
                                             oracle_bad* bad) {                                     \
        /* read index = dst (which 1), write index = flat_src (which 0) */                          \
        return accumulate_##S(grad_out, grad_out_rows, dst, flat_src, n, rel_rows, emb, grad_rel, \
                              0, 1, bad);                                                           \
    }
DEF_FANIN_SUM_BWD(float, f32)
DEF_FANIN_SUM_BWD(double, f64)

/* ---- mp_ops.cpp:3019-3035 fanin_reduce_logsumexp (CPU ATen sequence) -----
 * m = full(-inf); m[dst[e]] = amax(m, rel[src[e]]) (NaN propagates);
 * s[dst[e]] += exp(rel[src[e]] - m[dst[e]]) in edge order; out = log(s) + m.
 * Empty rows: log(0) + -inf = -inf.  which: 0 = flat_src, 1 = dst_idx. */
#define DEF_FANIN_LSE(T, S, EXP, LOG, MAXN)                                                         \
    int oracle_fanin_reduce_logsumexp_##S(const T* rel, int64_t rel_rows, int64_t emb,              \
                                          const int64_t* flat_src, const int64_t* dst, int64_t n,   \
                                          int64_t dim_size, T* out, oracle_bad* bad) {              \
        const size_t cells = (size_t)(dim_size * emb);                                              \
        T* m = (T*)malloc((cells ? cells : 1) * sizeof(T));                                         \
        T* s = (T*)calloc(cells ? cells : 1, sizeof(T));                                            \
        if (!m || !s) {                                                                             \
            free(m);                                                                                \
            free(s);                                                                                \
            return -1;                                                                              \
        }                                                                                           \
        for (size_t i = 0; i < cells; ++i) m[i] = -(T)INFINITY;                                     \
        for (int64_t e = 0; e < n; ++e) {                                                           \
            const int64_t si = flat_src[e], d = dst[e];                                             \
            if (!in_bounds(si, rel_rows) || !in_bounds(d, dim_size)) {                              \
                free(m);                                                                            \
                free(s);                                                                            \
                return in_bounds(si, rel_rows) ? bad_index(bad, 1, e, d, dim_size)                  \
                                               : bad_index(bad, 0, e, si, rel_rows);                \
            }                                                                                       \
            for (int64_t k = 0; k < emb; ++k)                                                       \
                m[d * emb + k] = MAXN(m[d * emb + k], rel[si * emb + k]);                           \
        }                                                                                           \
        for (int64_t e = 0; e < n; ++e) {                                                           \
            const int64_t si = flat_src[e], d = dst[e];                                             \
            for (int64_t k = 0; k < emb; ++k) {                                                     \
                const T w = EXP(rel[si * emb + k] - m[d * emb + k]);                                \
                s[d * emb + k] = s[d * emb + k] + w;                                                \
            }                                                                                       \
        }                                                                                           \
        for (size_t i = 0; i < cells; ++i) out[i] = LOG(s[i]) + m[i];                               \
        free(m);                                                                                    \
        free(s);                                                                                    \
        return ORACLE_OK;                                                                           \
    }
DEF_FANIN_LSE(float, f32, expf, logf, max_nan_f)
DEF_FANIN_LSE(double, f64, exp, log, max_nan_d)

/* ---- mp_ops.cpp:2981-3003 fanin_reduce_logsumexp_backward_fallback -------
 * grad_rel = zeros; grad_rel[flat_src[e]] += grad_out[d] * exp(rel[flat_src[e]] - out[d])
 * in edge order, d = dst_idx[e].  which: 0 = flat_src, 1 = dst_idx. */
#define DEF_FANIN_LSE_BWD(T, S, EXP)                                                                 \
    int oracle_fanin_reduce_logsumexp_backward_##S(                                                  \
        const T* grad_out, int64_t dim_size, int64_t emb, const T* rel, int64_t rel_flat_rows,       \
        const int64_t* flat_src, const int64_t* dst, int64_t n, const T* out, int64_t rel_rows,      \
        T* grad_rel, oracle_bad* bad) {                                                              \
        memset(grad_rel, 0, (size_t)(rel_rows * emb) * sizeof(T));                                   \
        const int64_t key_bound = rel_rows < rel_flat_rows ? rel_rows : rel_flat_rows;               \
        for (int64_t e = 0; e < n; ++e) {                                                            \
            const int64_t si = flat_src[e], d = dst[e];                                              \
            if (!in_bounds(si, key_bound)) return bad_index(bad, 0, e, si, key_bound);               \
            if (!in_bounds(d, dim_size)) return bad_index(bad, 1, e, d, dim_size);                   \
            for (int64_t k = 0; k < emb; ++k) {                                                      \
                const T w = EXP(rel[si * emb + k] - out[d * emb + k]);                               \
                const T c = grad_out[d * emb + k] * w;                                               \
                grad_rel[si * emb + k] = grad_rel[si * emb + k] + c;                                 \
            }                                                                                        \
        }                                                                                            \
        return ORACLE_OK;                                                                            \
    }
DEF_FANIN_LSE_BWD(float, f32, expf)
DEF_FANIN_LSE_BWD(double, f64, exp)

/* ---- float64 truth of the fp32 ops -----------------------------------------
 * Same reductions with every fp32 input widened to double and accumulated in
 * double, plus the per-cell sum of |terms| (the conditioning of each output),
 * used to bound the rounding error of long fp32 segments. */
void oracle_segment_sum_truth(const float* table, int64_t emb, const int64_t* read_idx,
                              const int64_t* write_idx, int64_t n, int64_t out_rows, double* sum,
                              double* abs_sum) {
    memset(sum, 0, (size_t)(out_rows * emb) * sizeof(double));
    memset(abs_sum, 0, (size_t)(out_rows * emb) * sizeof(double));
    for (int64_t e = 0; e < n; ++e) {
        const float* r = table + read_idx[e] * emb;
        double* o = sum + write_idx[e] * emb;
        double* a = abs_sum + write_idx[e] * emb;
        for (int64_t k = 0; k < emb; ++k) {
            o[k] += (double)r[k];
            a[k] += fabs((double)r[k]);
        }
    }
}

/* Logsumexp of fp32 messages in double: max first, then sum of exp in double. */
void oracle_fanin_logsumexp_truth(const float* rel, int64_t emb, const int64_t* flat_src,
                                  const int64_t* dst, int64_t n, int64_t dim_size, double* out) {
    const size_t cells = (size_t)(dim_size * emb);
    double* m = (double*)malloc((cells ? cells : 1) * sizeof(double));
    double* s = (double*)calloc(cells ? cells : 1, sizeof(double));
    for (size_t i = 0; i < cells; ++i) m[i] = -INFINITY;
    for (int64_t e = 0; e < n; ++e)
        for (int64_t k = 0; k < emb; ++k) {
            double* mm = m + dst[e] * emb + k;
            *mm = max_nan_d(*mm, (double)rel[flat_src[e] * emb + k]);
        }
    for (int64_t e = 0; e < n; ++e)
        for (int64_t k = 0; k < emb; ++k)
            s[dst[e] * emb + k] += exp((double)rel[flat_src[e] * emb + k] - m[dst[e] * emb + k]);
    for (size_t i = 0; i < cells; ++i) out[i] = log(s[i]) + m[i];
    free(m);
    free(s);
}

/* ---- index preprocessing ----------------------------------------------------
 * Stable CSR by key (the definition the GPU plan must reproduce bit-exactly):
 * offsets = exclusive cumsum of bincount(keys, minlength=num_keys);
 * perm = edge ids in stable key order (edge order inside each key).
 * Returns ORACLE_BAD_INDEX for a key outside [0, num_keys). */
int oracle_csr_build(const int64_t* keys, int64_t n, int64_t num_keys, int32_t* offsets,
                     int32_t* perm, oracle_bad* bad) {
    memset(offsets, 0, (size_t)(num_keys + 1) * sizeof(int32_t));
    for (int64_t e = 0; e < n; ++e) {
        if (!in_bounds(keys[e], num_keys)) return bad_index(bad, 0, e, keys[e], num_keys);
        offsets[keys[e] + 1] += 1;
    }
    for (int64_t k = 0; k < num_keys; ++k) offsets[k + 1] += offsets[k];
    int32_t* cursor = (int32_t*)malloc((size_t)(num_keys ? num_keys : 1) * sizeof(int32_t));
    if (!cursor) return -1;
    memcpy(cursor, offsets, (size_t)num_keys * sizeof(int32_t));
    for (int64_t e = 0; e < n; ++e) perm[cursor[keys[e]]++] = (int32_t)e;
    free(cursor);
    return ORACLE_OK;
}

/* Inverse map: inv[k] = largest edge with key k, or -1; returns the number of
 * edges whose key an earlier edge already had (keys assumed in range). */
int64_t oracle_inverse_build(const int64_t* keys, int64_t n, int64_t num_keys, int32_t* inv) {
    int64_t collisions = 0;
    for (int64_t k = 0; k < num_keys; ++k) inv[k] = -1;
    for (int64_t e = 0; e < n; ++e) {
        if (inv[keys[e]] >= 0) ++collisions;
        inv[keys[e]] = (int32_t)e;
    }
    return collisions;
}
