// Weight and bias gradients of a Linear with few columns over many rows:
//
//   dw[o][i] = sum_r g[r][o] * x[r][i],   db[o] = sum_r g[r][o]
//
// for g [M, O] (the gradient at the Linear's output) and x [M, I] (its input),
// O and I at most 96, M up to millions (the relation MLPs of a RelationalGNN
// step reduce over all atoms).  A library GEMM walks all of M in a few output
// tiles for such shapes; here each wave reduces its own run of rows with the
// fp32 matrix cores (v_mfma_f32_32x32x2f32: two rows per instruction into a
// 32 x 32 tile of dw), every workgroup stores one partial, and two more
// kernels add the partials up in workgroup order: a fixed summation order, so
// the result is the same on every run.
//
// Operand layout of v_mfma_f32_32x32x2f32 (one block): lane l supplies
// A[l % 32][l / 32] and B[l / 32][l % 32]; accumulator register j of lane l
// holds D[8 (j / 4) + 4 (l / 32) + j % 4][l % 32].  With A = g^T (row o of
// the tile, k = the row of g) and B = x, lane l loads g[r + l / 32][o0 + l %
// 32] and x[r + l / 32][i0 + l % 32]: two rows of 128 contiguous bytes per
// operand and instruction.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.h"

namespace relm_mp {

namespace {

constexpr int kWgThreads = 256;
constexpr int kWgWaves = kWgThreads / 64;
constexpr int kMaxTiles = 3;  // O, I <= 96

// Row pairs per iteration: the loads of the next iteration are issued before
// this one's products, so 2 * U row pairs of operands are in flight per wave.
template <int TO, int TI>
constexpr int wgrad_unroll() { return TO * TI <= 4 ? 8 : 4; }

typedef float v16f __attribute__((ext_vector_type(16)));

// Row (within a 32 x 32 tile) of accumulator register j of lane l.
__device__ __forceinline__ int acc_row(int lane, int j) { return 8 * (j / 4) + 4 * (lane / 32) + (j % 4); }

// Work of the four waves of a workgroup: with T = TO * TI output tiles of
// 32 x 32, T < 4 tiles are each taken by 4 / T waves over disjoint quarters or
// halves of the workgroup's rows (T = 3: three waves, one idle); T >= 4 tiles
// are dealt out to the waves (tile t to wave t % 4) over all of its rows, so
// that a wave holds at most three accumulators.
template <int T>
constexpr int wgrad_subsets() { return T == 1 ? 4 : (T == 2 ? 2 : 1); }

// Partial of workgroup b: O * I entries of dw (row-major), then O of db.
template <int TO, int TI>
__global__ __launch_bounds__(kWgThreads) void k_linear_wgrad(const float* __restrict__ g, int64_t ldg,
                                                             const float* __restrict__ x, int64_t ldx,
                                                             int64_t M, int O, int I, int64_t rows_per_wg,
                                                             float* __restrict__ partial) {
    constexpr int T = TO * TI;
    constexpr int S = wgrad_subsets<T>();
    constexpr int MT = S > 1 ? 1 : (T + kWgWaves - 1) / kWgWaves;  // tiles per wave
    constexpr int U = wgrad_unroll<TO, TI>();
    __shared__ float red[S > 1 ? (S - 1) * T * 1024 + (S - 1) * TO * 32 : 1];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int sub = S > 1 ? wave / T : 0;
    const int64_t per = rows_per_wg / S;  // even
    const int64_t r_begin = static_cast<int64_t>(blockIdx.x) * rows_per_wg + sub * per;
    const int64_t r_end = min(M, r_begin + per);

    // this wave's tiles: t_k = first + k * 4 (S == 1) or the single t = wave % T
    const int first = S > 1 ? wave % T : wave;
    int to_k[MT], ti_k[MT];
    bool own[MT], o_ok[MT], i_ok[MT];
#pragma unroll
    for (int k = 0; k < MT; ++k) {
        const int t = first + k * kWgWaves;
        own[k] = (S > 1 ? wave < S * T : true) && t < T;
        to_k[k] = own[k] ? t / TI : 0;
        ti_k[k] = own[k] ? t % TI : 0;
        o_ok[k] = own[k] && to_k[k] * 32 + col < O;
        i_ok[k] = own[k] && ti_k[k] * 32 + col < I;
    }
    v16f acc[MT];
    float bsum[MT];
#pragma unroll
    for (int k = 0; k < MT; ++k) {
        acc[k] = v16f{};
        bsum[k] = 0.0f;
    }

    float a[U][MT], b[U][MT];
    auto load = [&](int64_t r0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t row = r0 + 2 * u + half;
            const bool rv = row < r_end;
#pragma unroll
            for (int k = 0; k < MT; ++k) {
                a[u][k] = rv && o_ok[k] ? g[row * ldg + to_k[k] * 32 + col] : 0.0f;
                b[u][k] = rv && i_ok[k] ? x[row * ldx + ti_k[k] * 32 + col] : 0.0f;
            }
        }
    };
    load(r_begin);
    for (int64_t r0 = r_begin; r0 < r_end; r0 += 2 * U) {
        float ca[U][MT], cb[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < MT; ++k) {
                ca[u][k] = a[u][k];
                cb[u][k] = b[u][k];
            }
        if (r0 + 2 * U < r_end) load(r0 + 2 * U);  // next iteration's rows, in flight meanwhile
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < MT; ++k) {
                bsum[k] += ca[u][k];
                acc[k] = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[u][k], cb[u][k], acc[k], 0, 0, 0);
            }
    }
    // bias of o-tile to_k: kept by the wave of tile (to_k, 0); the two halves
    // of the wave hold alternate rows
#pragma unroll
    for (int k = 0; k < MT; ++k) bsum[k] += __shfl_xor(bsum[k], 32, 64);

    if constexpr (S > 1) {
        // waves of the later row subsets leave their tiles in LDS; the first
        // subset's wave adds them in subset order
        if (sub > 0 && wave < S * T) {
            float* dst = red + ((sub - 1) * T + first) * 1024 + lane * 16;
#pragma unroll
            for (int j = 0; j < 16; ++j) dst[j] = acc[0][j];
            if (ti_k[0] == 0 && lane < 32) red[(S - 1) * T * 1024 + ((sub - 1) * TO + to_k[0]) * 32 + lane] = bsum[0];
        }
        __syncthreads();
        if (sub == 0) {
            for (int q = 1; q < S; ++q) {
                const float* src = red + ((q - 1) * T + first) * 1024 + lane * 16;
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[0][j] += src[j];
                if (ti_k[0] == 0) bsum[0] += red[(S - 1) * T * 1024 + ((q - 1) * TO + to_k[0]) * 32 + col];
            }
        }
    }
    // the owning waves store the workgroup's partial in row-major order
    float* out = partial + static_cast<int64_t>(blockIdx.x) * (static_cast<int64_t>(O) * I + O);
    if (sub == 0) {
#pragma unroll
        for (int k = 0; k < MT; ++k) {
            if (!own[k]) continue;
            const int i = ti_k[k] * 32 + col;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int o = to_k[k] * 32 + acc_row(lane, j);
                if (o < O && i < I) out[static_cast<int64_t>(o) * I + i] = acc[k][j];
            }
            if (ti_k[k] == 0 && lane < 32 && to_k[k] * 32 + lane < O)
                out[static_cast<int64_t>(O) * I + to_k[k] * 32 + lane] = bsum[k];
        }
    }
}

constexpr int kSumGroup = 32;  // partials added per thread in the first summing pass

// First pass: sums[q][e] = partial[32 q][e] + ... + partial[32 q + 31][e] (in
// that order; blockIdx.y = q), so that many threads share the adding up.
__global__ __launch_bounds__(kWgThreads) void k_linear_wgrad_group(const float* __restrict__ partial,
                                                                   int64_t wgs, int64_t n,
                                                                   float* __restrict__ sums) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kWgThreads + threadIdx.x;
    if (e >= n) return;
    const int64_t b0 = static_cast<int64_t>(blockIdx.y) * kSumGroup;
    float v[kSumGroup];
#pragma unroll
    for (int k = 0; k < kSumGroup; ++k) v[k] = b0 + k < wgs ? partial[(b0 + k) * n + e] : 0.0f;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kSumGroup; ++k) s += v[k];
    sums[static_cast<int64_t>(blockIdx.y) * n + e] = s;
}

// dw[o][i] (row stride ldw) and db[o]: the group sums added in group order.
__global__ __launch_bounds__(kWgThreads) void k_linear_wgrad_sum(const float* __restrict__ sums,
                                                                 int64_t groups, int O, int I,
                                                                 float* __restrict__ dw, int64_t ldw,
                                                                 float* __restrict__ db) {
    const int64_t n = static_cast<int64_t>(O) * I + O;
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kWgThreads + threadIdx.x;
    if (e >= n) return;
    float s = 0.0f;
    for (int64_t q = 0; q < groups; ++q) s += sums[q * n + e];
    if (e < static_cast<int64_t>(O) * I) {
        dw[(e / I) * ldw + e % I] = s;
    } else if (db != nullptr) {
        db[e - static_cast<int64_t>(O) * I] = s;
    }
}

// Workgroups: about 32 row pairs per wave, at most 2048 workgroups (fewer for
// wide outputs, whose partials cost more to write and add up).
int64_t wgrad_wgs(int64_t M, int64_t O, int64_t I) {
    const int64_t rows = 2 * 32 * kWgWaves;
    const int64_t cap = O * I <= 32 * 32 ? 2048 : (O * I <= 64 * 64 ? 1024 : 512);
    return std::max<int64_t>(1, std::min<int64_t>(cap, (M + rows - 1) / rows));
}

}  // namespace

// Partials of every workgroup, then the sums of the groups of kSumGroup.
size_t linear_wgrad_scratch_bytes(int64_t M, int64_t O, int64_t I) {
    const int64_t wgs = wgrad_wgs(M, O, I);
    const int64_t groups = (wgs + kSumGroup - 1) / kSumGroup;
    return static_cast<size_t>(wgs + groups) * static_cast<size_t>(O * I + O) * sizeof(float);
}

bool linear_wgrad_supported(int64_t O, int64_t I) {
    return O >= 1 && I >= 1 && O <= kMaxTiles * 32 && I <= kMaxTiles * 32;
}

hipError_t launch_linear_wgrad(const float* g, int64_t ldg, const float* x, int64_t ldx, int64_t M,
                               int64_t O, int64_t I, float* dw, int64_t ldw, float* db, float* scratch,
                               hipStream_t s) {
    const int64_t wgs = wgrad_wgs(M, O, I);
    // rows per workgroup: a multiple of 2 * waves, covering M
    const int64_t step = 2 * kWgWaves;
    const int64_t rows_per_wg = ((M + wgs - 1) / wgs + step - 1) / step * step;
    const int to = static_cast<int>((O + 31) / 32), ti = static_cast<int>((I + 31) / 32);
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(wgs)), dim3(kWgThreads), 0, s, g, ldg, x, ldx,
                           M, static_cast<int>(O), static_cast<int>(I), rows_per_wg, scratch);
    };
    switch (to * 4 + ti) {
        case 1 * 4 + 1: launch(k_linear_wgrad<1, 1>); break;
        case 1 * 4 + 2: launch(k_linear_wgrad<1, 2>); break;
        case 1 * 4 + 3: launch(k_linear_wgrad<1, 3>); break;
        case 2 * 4 + 1: launch(k_linear_wgrad<2, 1>); break;
        case 2 * 4 + 2: launch(k_linear_wgrad<2, 2>); break;
        case 2 * 4 + 3: launch(k_linear_wgrad<2, 3>); break;
        case 3 * 4 + 1: launch(k_linear_wgrad<3, 1>); break;
        case 3 * 4 + 2: launch(k_linear_wgrad<3, 2>); break;
        case 3 * 4 + 3: launch(k_linear_wgrad<3, 3>); break;
        default: return hipErrorInvalidValue;
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int64_t n = O * I + O;
    const int64_t groups = (wgs + kSumGroup - 1) / kSumGroup;
    float* sums = scratch + wgs * n;
    const unsigned eblocks = static_cast<unsigned>((n + kWgThreads - 1) / kWgThreads);
    hipLaunchKernelGGL(k_linear_wgrad_group, dim3(eblocks, static_cast<unsigned>(groups)), dim3(kWgThreads), 0, s,
                       scratch, wgs, n, sums);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_linear_wgrad_sum, dim3(eblocks), dim3(kWgThreads), 0, s, sums, groups,
                       static_cast<int>(O), static_cast<int>(I), dw, ldw, db);
    return hipGetLastError();
}

}  // namespace relm_mp
