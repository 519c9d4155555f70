// FiLM step of a central MLP with its Mish activation, fused:
//
//   y = mish(beta[k] + gamma[k] * (s + add[k]))   for the rows of range k,
//
// where the rows of one range share their gamma / beta / add rows (the rows of
// one predicate: the condition and the slot mask are constant per predicate).
// One pass over s replaces torch's add, addcmul, Mish and the concatenation of
// the per-range results; the backward reads s and the upstream gradient once,
// writes ds and leaves per-block column sums of du * (s + add) and du (du the
// gradient at the Mish input) for the per-range gamma / beta gradients.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device_utils.h"
#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kThreads = 256;
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

// Mish and its derivative through n = e^u (e^u + 2): tanh(softplus(u)) =
// n / (n + 2), and d/du [u tanh(softplus(u))] = n / (n + 2) + 4 u e^u (1 +
// e^u) / (n + 2)^2.  Above u = 20, tanh(softplus(u)) is 1 in fp32.
__device__ __forceinline__ float mish(float u) {
    if (u > 20.0f) return u;
    const float e = __expf(u);
    const float n = e * (e + 2.0f);
    return u * n * __builtin_amdgcn_rcpf(n + 2.0f);
}

__device__ __forceinline__ float mish_grad(float u) {
    if (u > 20.0f) return 1.0f;
    const float e = __expf(u);
    const float n = e * (e + 2.0f);
    const float r = __builtin_amdgcn_rcpf(n + 2.0f);
    return n * r + 4.0f * u * e * (1.0f + e) * r * r;
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

// One workgroup per block of rows; thread t handles column units t, t + 256,
// ... (V floats each) of every row of the block.
template <int V>
__global__ __launch_bounds__(kThreads) void k_film_mish(const float* __restrict__ s,
                                                         int64_t width, FilmRanges R,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta,
                                                         const float* __restrict__ add,
                                                         float* __restrict__ y) {
    const BlockRows br = block_rows(R);
    const int64_t units = width / V;
    for (int64_t c = threadIdx.x; c < units; c += kThreads) {
        const int64_t col = c * V;
        const Vec<V> g = pack_load<float, V>(gamma + br.k * width + col);
        const Vec<V> b = pack_load<float, V>(beta + br.k * width + col);
        const Vec<V> a = add != nullptr ? pack_load<float, V>(add + br.k * width + col)
                                        : pack_fill<float, V>(0.0f);
        int64_t r = br.r0;
        for (; r + 4 <= br.r1; r += 4) {
            Vec<V> x[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) x[j] = pack_load_stream<float, V>(s + (r + j) * width + col);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                Vec<V> o;
#pragma unroll
                for (int i = 0; i < V; ++i) o.v[i] = mish(b.v[i] + g.v[i] * (x[j].v[i] + a.v[i]));
                pack_store_stream<float, V>(y + (r + j) * width + col, o);
            }
        }
        for (; r < br.r1; ++r) {
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
// mish'(u), each term rounded to fp32 and added in row order in fp64 (the
// sum of a block is rounded once: a per-range sum over tens of thousands of
// rows keeps about the accuracy of a tree reduction).
template <int V>
__global__ __launch_bounds__(kThreads) void k_film_mish_backward(
    const float* __restrict__ s, const float* __restrict__ dy, int64_t width, FilmRanges R,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ add, float* __restrict__ ds, float* __restrict__ partial) {
    const BlockRows br = block_rows(R);
    const int64_t units = width / V;
    float* __restrict__ part = partial + static_cast<int64_t>(blockIdx.x) * 2 * width;
    for (int64_t c = threadIdx.x; c < units; c += kThreads) {
        const int64_t col = c * V;
        const Vec<V> g = pack_load<float, V>(gamma + br.k * width + col);
        const Vec<V> b = pack_load<float, V>(beta + br.k * width + col);
        const Vec<V> a = add != nullptr ? pack_load<float, V>(add + br.k * width + col)
                                        : pack_fill<float, V>(0.0f);
        double sum_t[V], sum_u[V];
#pragma unroll
        for (int i = 0; i < V; ++i) sum_t[i] = sum_u[i] = 0.0;
        auto step = [&](const Vec<V>& x, const Vec<V>& d, int64_t r) {
            Vec<V> o;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const float t = x.v[i] + a.v[i];
                const float du = d.v[i] * mish_grad(b.v[i] + g.v[i] * t);
                o.v[i] = du * g.v[i];
                sum_t[i] += static_cast<double>(du * t);
                sum_u[i] += static_cast<double>(du);
            }
            pack_store_stream<float, V>(ds + r * width + col, o);
        };
        int64_t r = br.r0;
        for (; r + 4 <= br.r1; r += 4) {
            Vec<V> x[4], d[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[j] = pack_load_stream<float, V>(s + (r + j) * width + col);
                d[j] = pack_load_stream<float, V>(dy + (r + j) * width + col);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) step(x[j], d[j], r + j);
        }
        for (; r < br.r1; ++r)
            step(pack_load_stream<float, V>(s + r * width + col),
                 pack_load_stream<float, V>(dy + r * width + col), r);
        Vec<V> pt, pu;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            pt.v[i] = static_cast<float>(sum_t[i]);
            pu.v[i] = static_cast<float>(sum_u[i]);
        }
        pack_store<float, V>(part + col, pt);
        pack_store<float, V>(part + width + col, pu);
    }
}

int film_vec(int64_t width, std::initializer_list<const void*> ptrs) {
    if (width % 2 != 0) return 1;
    for (const void* p : ptrs)
        if (p != nullptr && reinterpret_cast<uintptr_t>(p) % 8 != 0) return 1;
    return 2;
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

}  // namespace

hipError_t launch_film_mish(const float* s, int64_t width, const int64_t* range_start,
                            int32_t num_ranges, const float* gamma, const float* beta,
                            const float* add, float* y, hipStream_t st) {
    const FilmRanges R = film_ranges(range_start, num_ranges);
    const int64_t blocks = R.first_block[kMaxRanges];
    if (blocks == 0 || width == 0) return hipSuccess;
    if (film_vec(width, {s, gamma, beta, add, y}) == 2)
        hipLaunchKernelGGL(k_film_mish<2>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st, s,
                           width, R, gamma, beta, add, y);
    else
        hipLaunchKernelGGL(k_film_mish<1>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st, s,
                           width, R, gamma, beta, add, y);
    return hipGetLastError();
}

hipError_t launch_film_mish_backward(const float* s, const float* dy, int64_t width,
                                     const int64_t* range_start, int32_t num_ranges,
                                     const float* gamma, const float* beta, const float* add,
                                     float* ds, float* partial, hipStream_t st) {
    const FilmRanges R = film_ranges(range_start, num_ranges);
    const int64_t blocks = R.first_block[kMaxRanges];
    if (blocks == 0 || width == 0) return hipSuccess;
    if (film_vec(width, {s, dy, gamma, beta, add, ds, partial}) == 2)
        hipLaunchKernelGGL(k_film_mish_backward<2>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                           st, s, dy, width, R, gamma, beta, add, ds, partial);
    else
        hipLaunchKernelGGL(k_film_mish_backward<1>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                           st, s, dy, width, R, gamma, beta, add, ds, partial);
    return hipGetLastError();
}

}  // namespace relm_mp
