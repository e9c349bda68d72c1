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

// Streaming stores (global_store ... nt) for outputs that no later access of the same kernel
// reads: the lines leave the L2 early instead of staying dirty there, so the write-back at
// the kernel's end has less to do.
typedef float f32x4v __attribute__((ext_vector_type(4)));
__device__ inline void st_stream(float* dst, float v) { __builtin_nontemporal_store(v, dst); }
__device__ inline void st_stream4(float* dst, float4 v) {
    const f32x4v q = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(q, reinterpret_cast<f32x4v*>(dst));
}

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

// Inclusive prefix sum over the 64 lanes of a wave on DPP: shifts by 1, 2, 4 and 8 lanes
// inside each row of 16 (lanes shifted in from outside the row add 0), then lane 15's sum
// broadcast into rows 1 and 3 and lane 31's into rows 2 and 3.  No LDS traffic.
__device__ inline int wave_inclusive_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}

// Exclusive scan of one int per thread over a whole block (blockDim.x a multiple of 64,
// at most 1024).  `scratch` holds >= 33 ints of LDS.  Returns the exclusive prefix and
// writes the block total to `total`.
__device__ inline int block_exclusive_scan(int v, int* scratch, int& total) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nwaves = blockDim.x >> 6;
    const int incl = wave_inclusive_scan(v);
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const int w = lane < nwaves ? scratch[lane] : 0;
        const int wi = wave_inclusive_scan(w);
        if (lane < nwaves) scratch[16 + lane] = wi - w;  // exclusive wave offsets
        if (lane == nwaves - 1) scratch[32] = wi;
    }
    __syncthreads();
    const int res = scratch[16 + wave] + incl - v;
    total = scratch[32];
    __syncthreads();
    return res;
}

// Stable LSD radix sort, by 8-bit digits of bits [sh0, sh0 + nbits), of the L keys in
// a[0:L) (the block's LDS), using b[0:L) and cnt[4 * blockDim.x] ints of LDS as scratch.
// blockDim.x is a multiple of 64 and L <= 64 * MAXR * (blockDim.x / 64).  Wave w owns a
// contiguous run of the input; a lane's rank among the equal digits of its 64-key round
// comes from eight ballots, the wave's running count per digit lives in cnt[digit][w],
// and one block scan over cnt (digit-major) turns the counts into stable offsets.
// Returns the buffer that holds the sorted keys (a or b).
template <int MAXR, typename T>
__device__ T* block_radix_sort(T* a, T* b, int* cnt, int L, int sh0, int nbits) {
    const int nw = blockDim.x >> 6;
    const int w = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int C = ((L + nw - 1) / nw + 63) & ~63;  // keys per wave
    const int rounds = C >> 6;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int sh = sh0; sh < sh0 + nbits; sh += 8) {
        for (int d = lane; d < 256; d += 64) cnt[d * nw + w] = 0;
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        T kk[MAXR];
        int rk[MAXR], dg[MAXR];
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
            if (r >= rounds) break;
            const int e = w * C + r * 64 + lane;
            const bool valid = e < L;
            const T key = valid ? a[e] : T(0);
            const int dig = (int)((key >> sh) & T(255));
            uint64_t m = __ballot(valid);
#pragma unroll
            for (int bit = 0; bit < 8; ++bit) {
                const bool on = (dig >> bit) & 1;
                const uint64_t bl = __ballot(valid && on);
                m &= on ? bl : ~bl;
            }
            const int base = valid ? cnt[dig * nw + w] : 0;
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
            if (valid && (m & below) == 0) cnt[dig * nw + w] = base + __popcll(m);
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
            kk[r] = key;
            rk[r] = base + __popcll(m & below);
            dg[r] = dig;
        }
        __syncthreads();
        // exclusive scan of cnt in (digit, wave) order: 4 entries per thread
        int* c4 = cnt + 4 * threadIdx.x;
        const int v0 = c4[0], v1 = c4[1], v2 = c4[2], v3 = c4[3];
        int total;
        const int off = block_exclusive_scan(v0 + v1 + v2 + v3, cnt + 4 * blockDim.x, total);
        c4[0] = off;
        c4[1] = off + v0;
        c4[2] = off + v0 + v1;
        c4[3] = off + v0 + v1 + v2;
        __syncthreads();
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
            if (r >= rounds) break;
            const int e = w * C + r * 64 + lane;
            if (e < L) b[cnt[dg[r] * nw + w] + rk[r]] = kk[r];
        }
        __syncthreads();
        T* t = a;
        a = b;
        b = t;
    }
    return a;
}

}  // namespace mb
