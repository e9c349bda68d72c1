// RMSNorm forward and backward on gfx950.
//
// Replaces RMSNorm.forward (mathbrain/model.py:11-19) and the autograd graph torch builds
// for it (pow, mean, add, rsqrt, two broadcast multiplies forward, about twice as many
// kernels backward) with one read of each row per pass:
//   forward   r = rsqrt(mean(x^2) + eps),  y = w * (x * r)      (the reference's order)
//   backward  dx = r (w dy) - (r^3 / D) x sum_d(w dy x),   dw = sum_rows dy (x r)
// One wave per row (lane l holds columns l, l + 64, ...); the backward walks rows with a
// grid stride, keeps its dw partial sums in registers, reduces them over the workgroup in
// LDS and adds them to dw with one atomic per column and workgroup.
#include "common.h"

#include <algorithm>

namespace mb {
namespace {

constexpr int kRmsThreads = 256;  // four rows (waves) per workgroup
constexpr int kRmsMaxD = 1024;
constexpr int kRmsBwdBlocks = 512;

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int PER>
__global__ void __launch_bounds__(kRmsThreads)
rms_fwd_kernel(const float* __restrict__ x, const float* __restrict__ w, int64_t rows, int D,
               float eps, float* __restrict__ y, float* __restrict__ rstd) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kRmsThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;  // the row is uniform across the wave
    const float* xr = x + row * D;
    float v[PER];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        v[i] = d < D ? xr[d] : 0.f;
        ss = __builtin_fmaf(v[i], v[i], ss);
    }
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)D + eps);
    float* yr = y + row * D;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        if (d < D) yr[d] = w[d] * (v[i] * r);
    }
    if (lane == 0) rstd[row] = r;
}

template <int PER>
__global__ void __launch_bounds__(kRmsThreads)
rms_bwd_kernel(const float* __restrict__ x, const float* __restrict__ w,
               const float* __restrict__ dy, const float* __restrict__ rstd, int64_t rows, int D,
               float* __restrict__ dx, float* __restrict__ dw) {
    __shared__ float part[kRmsThreads / 64][kRmsMaxD];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t nwaves = (int64_t)gridDim.x * (kRmsThreads / 64);
    float wv[PER], acc[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        wv[i] = d < D ? w[d] : 0.f;
        acc[i] = 0.f;
    }
    const float invD = 1.0f / (float)D;
    // rows are software-pipelined: the next row's loads are issued before this row's math
    int64_t row = (int64_t)blockIdx.x * (kRmsThreads / 64) + wave;
    float xn[PER], gn[PER], rn = 0.f;
    auto fetch = [&](int64_t rr) {
        const bool okr = rr < rows;
        const float* xr = x + (okr ? rr : 0) * D;
        const float* gr = dy + (okr ? rr : 0) * D;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int d = lane + 64 * i;
            const bool ok = okr && d < D;
            xn[i] = ok ? xr[d] : 0.f;
            gn[i] = ok ? gr[d] : 0.f;
        }
        rn = okr ? rstd[rr] : 0.f;
    };
    fetch(row);
    for (; row < rows; row += nwaves) {
        float xv[PER], gv[PER];
        const float r = rn;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            xv[i] = xn[i];
            gv[i] = gn[i];
        }
        fetch(row + nwaves);
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i) dot = __builtin_fmaf(wv[i] * gv[i], xv[i], dot);
        dot = wave_sum(dot);
        const float c = r * r * r * invD * dot;
        float* dxr = dx + row * D;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int d = lane + 64 * i;
            if (d < D) dxr[d] = r * (wv[i] * gv[i]) - c * xv[i];
            acc[i] = __builtin_fmaf(gv[i], xv[i] * r, acc[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        if (d < D) part[wave][d] = acc[i];
    }
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += kRmsThreads) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < kRmsThreads / 64; ++k) s += part[k][d];
        atomicAdd(dw + d, s);
    }
}

__global__ void rms_zero_kernel(float* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0.f;
}

int rms_per(int D) {
    const int need = (D + 63) / 64;
    return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : 16;
}

}  // namespace
}  // namespace mb

using namespace mb;

extern "C" int mb_rmsnorm_fwd(const float* x, const float* w, int64_t rows, int D, float eps,
                              float* y, float* rstd, void* stream) {
    MB_REQUIRE(rows >= 0, "mb_rmsnorm_fwd: rows=%lld < 0", (long long)rows);
    if (D < 1 || D > kRmsMaxD)
        return fail(MB_ERR_UNSUPPORTED, "mb_rmsnorm_fwd: D=%d (supported: 1..%d)", D, kRmsMaxD);
    if (rows == 0) return MB_OK;
    MB_REQUIRE(x && w && y && rstd, "mb_rmsnorm_fwd: null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    const int64_t blocks = (rows + kRmsThreads / 64 - 1) / (kRmsThreads / 64);
    MB_REQUIRE(blocks <= 0x7fffffff, "mb_rmsnorm_fwd: rows=%lld too many", (long long)rows);
    const dim3 grid((unsigned)blocks), blk(kRmsThreads);
    switch (rms_per(D)) {
        case 1: hipLaunchKernelGGL(rms_fwd_kernel<1>, grid, blk, 0, st, x, w, rows, D, eps, y, rstd); break;
        case 2: hipLaunchKernelGGL(rms_fwd_kernel<2>, grid, blk, 0, st, x, w, rows, D, eps, y, rstd); break;
        case 4: hipLaunchKernelGGL(rms_fwd_kernel<4>, grid, blk, 0, st, x, w, rows, D, eps, y, rstd); break;
        case 8: hipLaunchKernelGGL(rms_fwd_kernel<8>, grid, blk, 0, st, x, w, rows, D, eps, y, rstd); break;
        default: hipLaunchKernelGGL(rms_fwd_kernel<16>, grid, blk, 0, st, x, w, rows, D, eps, y, rstd); break;
    }
    return check_launch("mb_rmsnorm_fwd");
}

extern "C" int mb_rmsnorm_bwd(const float* x, const float* w, const float* dy, const float* rstd,
                              int64_t rows, int D, float* dx, float* dw, void* stream) {
    MB_REQUIRE(rows >= 0, "mb_rmsnorm_bwd: rows=%lld < 0", (long long)rows);
    if (D < 1 || D > kRmsMaxD)
        return fail(MB_ERR_UNSUPPORTED, "mb_rmsnorm_bwd: D=%d (supported: 1..%d)", D, kRmsMaxD);
    MB_REQUIRE(dw, "mb_rmsnorm_bwd: null dw");
    hipStream_t st = (hipStream_t)stream;
    // dw is accumulated with atomics: cleared here with a fill kernel (no memset)
    hipLaunchKernelGGL(rms_zero_kernel, dim3((D + 255) / 256), dim3(256), 0, st, dw, D);
    if (rows == 0) return check_launch("mb_rmsnorm_bwd");
    MB_REQUIRE(x && w && dy && rstd && dx, "mb_rmsnorm_bwd: null pointer argument");
    // two workgroups per CU, each walking rows with a grid stride: every workgroup adds its
    // D column sums to dw at the end, so more workgroups mean more atomics on the same D
    // addresses (2048 workgroups: 65 us at 28 672 x 512, most of it those atomics)
    const int64_t want = (rows + kRmsThreads / 64 - 1) / (kRmsThreads / 64);
    const dim3 grid((unsigned)std::min<int64_t>(want, kRmsBwdBlocks)), blk(kRmsThreads);
    switch (rms_per(D)) {
        case 1: hipLaunchKernelGGL(rms_bwd_kernel<1>, grid, blk, 0, st, x, w, dy, rstd, rows, D, dx, dw); break;
        case 2: hipLaunchKernelGGL(rms_bwd_kernel<2>, grid, blk, 0, st, x, w, dy, rstd, rows, D, dx, dw); break;
        case 4: hipLaunchKernelGGL(rms_bwd_kernel<4>, grid, blk, 0, st, x, w, dy, rstd, rows, D, dx, dw); break;
        case 8: hipLaunchKernelGGL(rms_bwd_kernel<8>, grid, blk, 0, st, x, w, dy, rstd, rows, D, dx, dw); break;
        default: hipLaunchKernelGGL(rms_bwd_kernel<16>, grid, blk, 0, st, x, w, dy, rstd, rows, D, dx, dw); break;
    }
    return check_launch("mb_rmsnorm_bwd");
}
