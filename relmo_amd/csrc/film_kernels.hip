// FiLM step of a central MLP with its Mish activation, fused:
//
//   y = mish(beta[k] + gamma[k] * (s + add[k]))   for the rows of range k,
//
// where the rows of one range share their gamma / beta / add rows (the rows of
// one predicate: the condition and the slot mask are constant per predicate).
// One pass over s replaces torch's add, addcmul, Mish and the concatenation of
// the per-range results; the backward reads s and the upstream gradient once,
// writes ds and leaves per-block column sums of du * (s + add) and du (du the
// gradient at the Mish input), in fp64, for the per-range gamma / beta
// gradients.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device_utils.h"
#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kMaxThreads = 1024;
constexpr int kMaxRanges = RELM_MP_FILM_MAX_RANGES;
constexpr int kRowsPerBlock = RELM_MP_FILM_ROWS_PER_BLOCK;

// Range k covers rows [start[k], start[k + 1]); its blocks of kRowsPerBlock
// rows are blocks [first_block[k], first_block[k + 1]) of the grid, so no
// block spans two ranges.
struct FilmRanges {
    int64_t start[kMaxRanges + 1];
    int64_t first_block[kMaxRanges + 1];
    int num;
};

// Mish and its derivative in the fp32 formulation of PyTorch's own Mish
// kernels (torch.nn.functional.mish and its backward on ROCm):
//   mish(u)         = u * tanh(log1p(exp(u)))
//   dy * mish'(u)   = dy * (t + u * sigmoid(u) * (1 - t * t)),  t = tanh(log1p(exp(u))),
// with the two multiply-adds of the derivative fused as torch's build fuses
// them, the accurate expf / log1pf / tanhf and IEEE division.  Together with
// the affine step b + g * (s + a) rounded as torch's addcmul rounds it, the
// fused step computes exactly what torch's FiLM and Mish ops compute, bit for
// bit (checked against them on the GPU).  The weight gradient of the Linear
// before the FiLM step is a sum over all rows with large cancellation; its
// rounding error moves by a factor of three with the last bit of a few rows'
// gradients, so a different (even more accurate) formulation leaves the
// models' gradients at a different fp32 error than the torch lane's.
// At u >= 10 that formulation has t = 1 exactly (log1p(exp(u)) > 10, whose
// tanh rounds to 1), so mish(u) = u and the gradient is dy; at u <= -104
// exp(u) is 0 in fp32, so t = 0: mish(u) = u * 0 and the gradient dy * +0.  The shortcuts
// skip the transcendental calls there and give the same bits (tested over
// dense sweeps of both ranges against torch).
constexpr float kMishOne = 10.0f;
constexpr float kMishZero = -104.0f;

__device__ __forceinline__ float mish(float u) {
    if (u >= kMishOne) return u;
    if (u <= kMishZero) return u * 0.0f;
    return u * tanhf(log1pf(expf(u)));
}

__device__ __forceinline__ float mish_backward(float dy, float u) {
    if (u >= kMishOne) return dy;
    if (u <= kMishZero) return dy * 0.0f;  // fma(u * 0, 1, 0) = +0 in the full formula
    const float sg = 1.0f / (1.0f + expf(-u));
    const float t = tanhf(log1pf(expf(u)));
    return dy * fmaf(u * sg, fmaf(-t, t, 1.0f), t);
}

template <int V>
using Vec = Pack<float, V>;

// The block's rows and its range: blocks of a range are consecutive.
struct BlockRows {
    int k;
    int64_t r0;
    int64_t r1;
};

__device__ __forceinline__ BlockRows block_rows(const FilmRanges& R) {
    const int64_t b = blockIdx.x;
    int k = 0;
#pragma unroll
    for (int q = 1; q < kMaxRanges; ++q)
        if (q < R.num && b >= R.first_block[q]) k = q;
    const int64_t r0 = R.start[k] + (b - R.first_block[k]) * kRowsPerBlock;
    const int64_t r1 = min(r0 + kRowsPerBlock, R.start[k + 1]);
    return {k, r0, r1};
}

// Thread layout of both kernels: `phases` groups of `units` threads (one per
// column unit of V floats); thread t owns unit t % units and, within the
// workgroup's block of rows, the rows r0 + p, r0 + p + phases, ... (p = t /
// units).  Several phases keep the lanes busy where a row has fewer units
// than the workgroup threads (C5: 199 pairs of floats per row, 5 phases over
// 1024 threads); with one phase the threads loop over the units instead (rows
// wider than the workgroup).  A thread keeps its columns, so the backward's
// column sums need no atomics.
struct FilmLayout {
    int units;   // column units per row
    int phases;  // row phases
};

template <int V>
__global__ __launch_bounds__(kMaxThreads) void k_film_mish(const float* __restrict__ s,
                                                           int64_t width, FilmRanges R, FilmLayout L,
                                                           const float* __restrict__ gamma,
                                                           const float* __restrict__ beta,
                                                           const float* __restrict__ add,
                                                           float* __restrict__ y) {
    const BlockRows br = block_rows(R);
    const int t = static_cast<int>(threadIdx.x);
    const int ph = L.phases > 1 ? t / L.units : 0;
    if (ph >= L.phases) return;
    const int step = L.phases;
    for (int64_t c = L.phases > 1 ? t % L.units : t; c < L.units; c += L.phases > 1 ? L.units : blockDim.x) {
        const int64_t col = c * V;
        const Vec<V> g = pack_load<float, V>(gamma + br.k * width + col);
        const Vec<V> b = pack_load<float, V>(beta + br.k * width + col);
        const Vec<V> a = add != nullptr ? pack_load<float, V>(add + br.k * width + col)
                                        : pack_fill<float, V>(0.0f);
        int64_t r = br.r0 + ph;
        for (; r + 3 * step < br.r1; r += 4 * step) {
            Vec<V> x[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) x[j] = pack_load_stream<float, V>(s + (r + j * step) * width + col);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                Vec<V> o;
#pragma unroll
                for (int i = 0; i < V; ++i) o.v[i] = mish(b.v[i] + g.v[i] * (x[j].v[i] + a.v[i]));
                pack_store_stream<float, V>(y + (r + j * step) * width + col, o);
            }
        }
        for (; r < br.r1; r += step) {
            const Vec<V> x = pack_load_stream<float, V>(s + r * width + col);
            Vec<V> o;
#pragma unroll
            for (int i = 0; i < V; ++i) o.v[i] = mish(b.v[i] + g.v[i] * (x.v[i] + a.v[i]));
            pack_store_stream<float, V>(y + r * width + col, o);
        }
    }
}

// ds = dy * mish'(u) * gamma; partial[block][0][col] = sum over the block's
// rows of du * (s + add), partial[block][1][col] = sum of du, du = dy *
// mish'(u), each term rounded to fp32 and added in fp64: by each thread over
// its rows in row order, then the phases in order.  The block sums stay fp64
// (the caller adds a range's blocks in fp64 and rounds once), so a per-range
// sum over tens of thousands of rows carries only the rounding of its terms.
// With several phases, `lds` holds phases * units * V * 2 doubles.
template <int V>
__global__ __launch_bounds__(kMaxThreads) void k_film_mish_backward(
    const float* __restrict__ s, const float* __restrict__ dy, int64_t width, FilmRanges R,
    FilmLayout L, const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ add, float* __restrict__ ds, double* __restrict__ partial) {
    extern __shared__ double lds[];
    const BlockRows br = block_rows(R);
    const int t = static_cast<int>(threadIdx.x);
    const int ph = L.phases > 1 ? t / L.units : 0;
    const int step = L.phases;
    double* __restrict__ part = partial + static_cast<int64_t>(blockIdx.x) * 2 * width;
    const bool active = ph < L.phases;
    for (int64_t c = L.phases > 1 ? t % L.units : t; active && c < L.units;
         c += L.phases > 1 ? L.units : blockDim.x) {
        const int64_t col = c * V;
        const Vec<V> g = pack_load<float, V>(gamma + br.k * width + col);
        const Vec<V> b = pack_load<float, V>(beta + br.k * width + col);
        const Vec<V> a = add != nullptr ? pack_load<float, V>(add + br.k * width + col)
                                        : pack_fill<float, V>(0.0f);
        double sum_t[V], sum_u[V];
#pragma unroll
        for (int i = 0; i < V; ++i) sum_t[i] = sum_u[i] = 0.0;
        auto stp = [&](const Vec<V>& x, const Vec<V>& d, int64_t r) {
            Vec<V> o;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const float tt = x.v[i] + a.v[i];
                const float du = mish_backward(d.v[i], b.v[i] + g.v[i] * tt);
                o.v[i] = du * g.v[i];
                sum_t[i] += static_cast<double>(du * tt);
                sum_u[i] += static_cast<double>(du);
            }
            pack_store_stream<float, V>(ds + r * width + col, o);
        };
        int64_t r = br.r0 + ph;
        for (; r + 3 * step < br.r1; r += 4 * step) {
            Vec<V> x[4], d[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[j] = pack_load_stream<float, V>(s + (r + j * step) * width + col);
                d[j] = pack_load_stream<float, V>(dy + (r + j * step) * width + col);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) stp(x[j], d[j], r + j * step);
        }
        for (; r < br.r1; r += step)
            stp(pack_load_stream<float, V>(s + r * width + col),
                pack_load_stream<float, V>(dy + r * width + col), r);
        if (L.phases > 1) {
            // this thread's sums into LDS: [phase][unit][V] for t, then for u
            double* lt = lds + (static_cast<int64_t>(ph) * L.units + c) * V;
            double* lu = lt + static_cast<int64_t>(L.phases) * L.units * V;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                lt[i] = sum_t[i];
                lu[i] = sum_u[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < V; ++i) {
                part[col + i] = sum_t[i];
                part[width + col + i] = sum_u[i];
            }
        }
    }
    if (L.phases > 1) {
        __syncthreads();
        // phase 0's threads add the phases in order
        if (active && ph == 0) {
            const int c = t;
            const int64_t col = static_cast<int64_t>(c) * V;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                double at = 0.0, au = 0.0;
                for (int p = 0; p < L.phases; ++p) {
                    const double* lt = lds + (static_cast<int64_t>(p) * L.units + c) * V;
                    at += lt[i];
                    au += lt[static_cast<int64_t>(L.phases) * L.units * V + i];
                }
                part[col + i] = at;
                part[width + col + i] = au;
            }
        }
    }
}

// Floats per lane: 4 where the width and every table are 16-byte aligned,
// else 2 where they are 8-byte aligned, else 1.
int film_vec(int64_t width, std::initializer_list<const void*> ptrs) {
    for (int v : {4, 2}) {
        bool ok = width % v == 0;
        for (const void* p : ptrs) ok = ok && (p == nullptr || reinterpret_cast<uintptr_t>(p) % (4 * v) == 0);
        if (ok) return v;
    }
    return 1;
}

FilmRanges film_ranges(const int64_t* range_start, int32_t num_ranges) {
    FilmRanges R{};
    int64_t blocks = 0;
    for (int k = 0; k < num_ranges; ++k) {
        R.start[k] = range_start[k];
        R.first_block[k] = blocks;
        blocks += film_range_blocks(range_start[k + 1] - range_start[k]);
    }
    for (int k = num_ranges; k <= kMaxRanges; ++k) {
        R.start[k] = range_start[num_ranges];
        R.first_block[k] = blocks;
    }
    R.num = num_ranges;
    return R;
}

// Most phases whose threads fit one workgroup (at most kMaxPhases), and the
// workgroup size: a multiple of the wave.  Narrow rows take many phases, so
// that a block of kRowsPerBlock rows still fills a workgroup (rows of 32
// floats: 16 column pairs x 64 phases of 8 rows each).  With 4 floats per
// lane the phases' threads stay within 768, so that the backward's fp64
// phase sums (phases * units * V * 16 bytes) fit 48 KB of LDS.
constexpr int kMaxPhases = 64;
FilmLayout film_layout(int64_t units, int V) {
    const int64_t cap = V >= 4 ? 768 : kMaxThreads;
    FilmLayout L{static_cast<int>(units), 1};
    if (units <= cap / 2) L.phases = static_cast<int>(std::min<int64_t>(kMaxPhases, cap / units));
    return L;
}

int film_threads(const FilmLayout& L) {
    const int n = L.units * L.phases;
    return std::min(kMaxThreads, (n + 63) / 64 * 64);
}

size_t film_lds_bytes(const FilmLayout& L, int V) {
    return L.phases > 1 ? static_cast<size_t>(L.phases) * L.units * V * 2 * sizeof(double) : 0;
}

}  // namespace

hipError_t launch_film_mish(const float* s, int64_t width, const int64_t* range_start,
                            int32_t num_ranges, const float* gamma, const float* beta,
                            const float* add, float* y, hipStream_t st) {
    const FilmRanges R = film_ranges(range_start, num_ranges);
    const int64_t blocks = R.first_block[kMaxRanges];
    if (blocks == 0 || width == 0) return hipSuccess;
    const int V = film_vec(width, {s, gamma, beta, add, y});
    const FilmLayout L = film_layout(width / V, V);
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(film_threads(L)), 0, st, s,
                           width, R, L, gamma, beta, add, y);
    };
    if (V == 4) launch(k_film_mish<4>);
    else if (V == 2) launch(k_film_mish<2>);
    else launch(k_film_mish<1>);
    return hipGetLastError();
}

hipError_t launch_film_mish_backward(const float* s, const float* dy, int64_t width,
                                     const int64_t* range_start, int32_t num_ranges,
                                     const float* gamma, const float* beta, const float* add,
                                     float* ds, double* partial, hipStream_t st) {
    const FilmRanges R = film_ranges(range_start, num_ranges);
    const int64_t blocks = R.first_block[kMaxRanges];
    if (blocks == 0 || width == 0) return hipSuccess;
    const int V = film_vec(width, {s, dy, gamma, beta, add, ds, partial});
    const FilmLayout L = film_layout(width / V, V);
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(film_threads(L)),
                           film_lds_bytes(L, V), st, s, dy, width, R, L, gamma, beta, add, ds, partial);
    };
    if (V == 4) launch(k_film_mish_backward<4>);
    else if (V == 2) launch(k_film_mish_backward<2>);
    else launch(k_film_mish_backward<1>);
    return hipGetLastError();
}

}  // namespace relm_mp
