// Device helpers for gfx950 (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace relm_mp {

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

__device__ __forceinline__ unsigned long long lanemask_lt() {
    return (1ull << lane_id()) - 1ull;
}

// The dispatcher hands workgroups to the 8 XCDs round robin (workgroup b to
// XCD b % 8).  xcd_tile maps workgroup b to a tile so that each XCD works
// through one contiguous range of tiles: neighbouring tiles then share an L2,
// where the partial lines they write at the seams of their output ranges
// merge.  A bijection of [0, ntiles).
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t ntiles) {
    constexpr int64_t kXcds = 8;
    const int64_t q = ntiles / kXcds, r = ntiles % kXcds;
    const int64_t x = b % kXcds;
    return x * q + (x < r ? x : r) + b / kXcds;
}

// Lanes of the wave whose `digit` (of BITS bits) equals this lane's, among
// the lanes in `active`.  One ballot per bit; each bit keeps the lanes whose
// ballot bit agrees with this lane's digit bit, peers &= ~(ballot ^ bitmask):
// a sign-extending bit extract, a compare and one v_bitop3 per 32-bit half.
// v_bitop3's table is indexed by (src0, src1, src2) bits; with src0 = 0xF0,
// src1 = 0xCC, src2 = 0xAA, src0 & ~(src1 ^ src2) = 0x90.
template <int BITS>
__device__ __forceinline__ unsigned long long match_digit(uint32_t digit,
                                                          unsigned long long active) {
    uint32_t lo = static_cast<uint32_t>(active);
    uint32_t hi = static_cast<uint32_t>(active >> 32);
#pragma unroll
    for (int b = 0; b < BITS; ++b) {
        // all ones if bit b of the digit is set, else zero
        const int32_t sm = __builtin_amdgcn_sbfe(static_cast<int32_t>(digit), b, 1);
        const unsigned long long m = __ballot(sm < 0);
        lo = __builtin_amdgcn_bitop3_b32(lo, static_cast<uint32_t>(m), static_cast<uint32_t>(sm), 0x90);
        hi = __builtin_amdgcn_bitop3_b32(hi, static_cast<uint32_t>(m >> 32), static_cast<uint32_t>(sm),
                                         0x90);
    }
    return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// Row-vector of V elements moved as one aligned load / store.
template <typename T, int V>
struct alignas(sizeof(T) * V) Pack {
    T v[V];
};

template <typename T, int V>
__device__ __forceinline__ Pack<T, V> pack_fill(T x) {
    Pack<T, V> p;
#pragma unroll
    for (int i = 0; i < V; ++i) p.v[i] = x;
    return p;
}

template <typename T, int V>
__device__ __forceinline__ Pack<T, V> pack_load(const T* ptr) {
    return *reinterpret_cast<const Pack<T, V>*>(ptr);
}

template <typename T, int V>
__device__ __forceinline__ void pack_store(T* ptr, const Pack<T, V>& p) {
    *reinterpret_cast<Pack<T, V>*>(ptr) = p;
}

// Streaming load: rows read once, kept out of the way of reused rows in L2.
template <typename T, int V>
__device__ __forceinline__ Pack<T, V> pack_load_stream(const T* ptr) {
    Pack<T, V> p;
#pragma unroll
    for (int i = 0; i < V; ++i) p.v[i] = __builtin_nontemporal_load(ptr + i);
    return p;
}

// Streaming store: the written rows are not re-read by this kernel.
template <typename T, int V>
__device__ __forceinline__ void pack_store_stream(T* ptr, const Pack<T, V>& p) {
#pragma unroll
    for (int i = 0; i < V; ++i) __builtin_nontemporal_store(p.v[i], ptr + i);
}

// Maximum that propagates NaN like ATen's amax (a NaN operand wins).
template <typename T>
__device__ __forceinline__ T max_nan(T a, T b) {
    return (b > a || b != b) ? b : a;
}

template <typename T>
__device__ __forceinline__ T dev_exp(T x);
template <>
__device__ __forceinline__ float dev_exp<float>(float x) { return expf(x); }
template <>
__device__ __forceinline__ double dev_exp<double>(double x) { return exp(x); }

// exp on the hardware exp2 unit (v_exp_f32 of x * log2(e)); relative error
// grows like |x| * 2^-24, far inside the logsumexp tolerance.  The double
// version stays the accurate libm-equivalent exp.
template <typename T>
__device__ __forceinline__ T fast_exp(T x);
template <>
__device__ __forceinline__ float fast_exp<float>(float x) { return __expf(x); }
template <>
__device__ __forceinline__ double fast_exp<double>(double x) { return exp(x); }

// Maximum that ignores NaN operands (v_max_f32); NaN is tracked separately.
template <typename T>
__device__ __forceinline__ T max_num(T a, T b) { return fmax(a, b); }

template <typename T>
__device__ __forceinline__ T dev_log(T x);
// Callers take the log of a sum of exp terms one of which is exp(0) = 1, so
// x >= 1 (or NaN, or +inf): the hardware log2 (v_log_f32, ~1 ulp on normal
// inputs) times ln 2, without the denormal range reduction and the
// extra-precision ln 2 product of logf (which __logf also expands to).
template <>
__device__ __forceinline__ float dev_log<float>(float x) {
    return __builtin_amdgcn_logf(x) * 0.693147180559945309f;
}
template <>
__device__ __forceinline__ double dev_log<double>(double x) { return log(x); }

// log(s) + m: for float one rounding of log2(s) * ln 2 + m (the hardware
// log2, then a fused multiply-add); for double the accurate log.
template <typename T>
__device__ __forceinline__ T log_add(T s, T m) { return log(s) + m; }
template <>
__device__ __forceinline__ float log_add<float>(float s, float m) {
    return __builtin_fmaf(__builtin_amdgcn_logf(s), 0.693147180559945309f, m);
}

template <typename T>
__device__ __forceinline__ T neg_inf() { return -__builtin_huge_val(); }
template <>
__device__ __forceinline__ float neg_inf<float>() { return -__builtin_huge_valf(); }

// Lowest finite value.
template <typename T>
__device__ __forceinline__ T lowest() { return -__DBL_MAX__; }
template <>
__device__ __forceinline__ float lowest<float>() { return -__FLT_MAX__; }

template <typename T>
__device__ __forceinline__ T quiet_nan() { return __builtin_nan(""); }
template <>
__device__ __forceinline__ float quiet_nan<float>() { return __builtin_nanf(""); }

// Inclusive scan over one wave.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t x) {
    const int lane = lane_id();
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, kWave);
        if (lane >= o) x += y;
    }
    return x;
}

// Inclusive scan over a block of NT threads (NT a multiple of 64).  `lds` holds
// NT/64 words.  Returns the inclusive prefix; `total` receives the block sum.
template <int NT>
__device__ __forceinline__ uint32_t block_inclusive_scan(uint32_t x, uint32_t* lds,
                                                         uint32_t& total) {
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    x = wave_inclusive_scan(x);
    if (lane_id() == kWave - 1) lds[wave] = x;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NT / kWave; ++w) {
        const uint32_t t = lds[w];
        if (w < wave) pre += t;
        tot += t;
    }
    __syncthreads();
    total = tot;
    return x + pre;
}

// Exclusive maximum scan over a block of NT threads (NT a multiple of 64):
// the maximum of x over the threads before this one, 0 for thread 0.  `lds`
// holds NT/64 words.
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_max(uint32_t x, uint32_t* lds) {
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = lane_id();
    uint32_t incl = x;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o, kWave);
        if (lane >= o) incl = max(incl, y);
    }
    if (lane == kWave - 1) lds[wave] = incl;
    uint32_t ex = __shfl_up(incl, 1, kWave);
    if (lane == 0) ex = 0;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NT / kWave; ++w)
        if (w < wave) ex = max(ex, lds[w]);
    __syncthreads();
    return ex;
}

}  // namespace relm_mp
