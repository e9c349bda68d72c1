// Shared helpers for the gfx950 kernels behind the mathbrain C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "mathbrain_hip.h"

namespace mb {

// ---- error reporting ---------------------------------------------------------------------

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

// Returns MB_OK or the launch error as a positive hipError_t code.
int check_launch(const char* what);

#define MB_REQUIRE(cond, ...)                                         \
    do {                                                              \
        if (!(cond)) return ::mb::fail(MB_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
    } while (0)

// ---- small device utilities -----------------------------------------------------------------

__host__ __device__ inline int next_pow2(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

__host__ __device__ inline int ceil_log2(int v) {
    int b = 0;
    while ((1 << b) < v) ++b;
    return b;
}

// rho^steps for integer steps >= 0, to within ~2 ulp of a correctly rounded powf:
// log2(rho) is carried as a float pair (hi + lo) and the rounding error of
// steps*hi is recovered with an fma, so that the exponent keeps full precision
// even for steps in the thousands.
__device__ inline float pow_steps(float l2hi, float l2lo, int steps) {
    if (steps == 0) return 1.0f;
    const float s = (float)steps;
    const float p = s * l2hi;
    float r = exp2f(p);
    if (__builtin_isfinite(p)) {
        const float e = __builtin_fmaf(s, l2hi, -p) + s * l2lo;
        r = r * __builtin_fmaf(e, 0.69314718055994530942f, 1.0f);
    }
    return r;
}

// Splits log2(rho) into a float pair, in double precision.
__device__ inline void log2_split(float rho, float& hi, float& lo) {
    const double l = log2((double)rho);
    hi = (float)l;
    lo = __builtin_isfinite(l) ? (float)(l - (double)hi) : 0.0f;
}

// Exclusive scan of one int per thread over a whole block (blockDim.x a multiple of 64,
// at most 1024).  `scratch` holds >= 16 ints of LDS.  Returns the exclusive prefix and
// writes the block total to `total`.
__device__ inline int block_exclusive_scan(int v, int* scratch, int& total) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nwaves = blockDim.x >> 6;
    int incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        int w = lane < nwaves ? scratch[lane] : 0;
        int wi = w;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            int o = __shfl_up(wi, d, 64);
            if (lane >= d) wi += o;
        }
        if (lane < nwaves) scratch[16 + lane] = wi - w;  // exclusive wave offsets
        if (lane == nwaves - 1) scratch[32] = wi;
    }
    __syncthreads();
    const int res = scratch[16 + wave] + incl - v;
    total = scratch[32];
    __syncthreads();
    return res;
}

// In-place ascending bitonic sort of n (power of two) keys in LDS by the whole block.
template <typename T>
__device__ inline void block_bitonic_sort(T* s, int n) {
    const int half = n >> 1;
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < half; i += blockDim.x) {
                const int lo = 2 * j * (i / j) + (i % j);
                const int hi = lo + j;
                const bool up = (lo & k) == 0;
                const T a = s[lo];
                const T b = s[hi];
                if ((a > b) == up) {
                    s[lo] = b;
                    s[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

}  // namespace mb
