// SwiGLU gate product, forward and backward, on gfx950.
//
// Replaces the elementwise part of SwiGLU.forward (mathbrain/model.py:21-29),
// F.silu(w1(x)) * w3(x), and its autograd backward (torch's silu, mul, mul-backward and
// silu-backward passes) with one pass per direction over the two projections a = w1(x),
// b = w3(x):
//   forward   m  = SiLU(a) * b
//   backward  da = dm * b * SiLU'(a),  db = dm * SiLU(a),   SiLU'(a) = s (1 + a (1 - s))
// with s = sigmoid(a), evaluated in fp32 and rounded once to the storage type (fp32 or
// bf16; under autocast the projections are bf16).  Each thread handles 8 consecutive
// elements (one 16-byte load of bf16, 32 bytes of fp32) with a grid stride; a ragged tail
// goes element by element.
#include "common.h"

#include <algorithm>

namespace mb {
namespace {

constexpr int kSwiThreads = 256;
constexpr int kSwiPer = 8;

typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));

__device__ inline float ld(const float* p, int64_t i) { return p[i]; }
__device__ inline float ld(const __bf16* p, int64_t i) { return (float)p[i]; }
__device__ inline void st(float* p, int64_t i, float v) { p[i] = v; }
__device__ inline void st(__bf16* p, int64_t i, float v) { p[i] = (__bf16)v; }

// Eight consecutive elements starting at a multiple of 8 (16- or 32-byte aligned: the
// tensors are contiguous allocations), as one vector load / store.
__device__ inline void ld8(const float* p, int64_t i, float (&v)[kSwiPer]) {
    const f32x8 x = *reinterpret_cast<const f32x8*>(p + i);
#pragma unroll
    for (int e = 0; e < kSwiPer; ++e) v[e] = x[e];
}
__device__ inline void ld8(const __bf16* p, int64_t i, float (&v)[kSwiPer]) {
    const bf16x8v x = *reinterpret_cast<const bf16x8v*>(p + i);
#pragma unroll
    for (int e = 0; e < kSwiPer; ++e) v[e] = (float)x[e];
}
__device__ inline void st8(float* p, int64_t i, const float (&v)[kSwiPer]) {
    f32x8 x;
#pragma unroll
    for (int e = 0; e < kSwiPer; ++e) x[e] = v[e];
    *reinterpret_cast<f32x8*>(p + i) = x;
}
__device__ inline void st8(__bf16* p, int64_t i, const float (&v)[kSwiPer]) {
    bf16x8v x;
#pragma unroll
    for (int e = 0; e < kSwiPer; ++e) x[e] = (__bf16)v[e];
    *reinterpret_cast<bf16x8v*>(p + i) = x;
}

__device__ inline float sigmoid_f(float a) { return 1.0f / (1.0f + __expf(-a)); }

template <class T>
__global__ void __launch_bounds__(kSwiThreads)
swiglu_fwd_kernel(const T* __restrict__ a, const T* __restrict__ b, int64_t n, T* __restrict__ m) {
    const int64_t stride = (int64_t)gridDim.x * kSwiThreads * kSwiPer;
    for (int64_t i0 = ((int64_t)blockIdx.x * kSwiThreads + threadIdx.x) * kSwiPer; i0 < n; i0 += stride) {
        float av[kSwiPer], bv[kSwiPer], mv[kSwiPer];
        const bool whole = i0 + kSwiPer <= n;
        if (whole) {
            ld8(a, i0, av);
            ld8(b, i0, bv);
        } else {
#pragma unroll
            for (int e = 0; e < kSwiPer; ++e) {
                const bool ok = i0 + e < n;
                av[e] = ok ? ld(a, i0 + e) : 0.f;
                bv[e] = ok ? ld(b, i0 + e) : 0.f;
            }
        }
#pragma unroll
        for (int e = 0; e < kSwiPer; ++e) mv[e] = av[e] * sigmoid_f(av[e]) * bv[e];
        if (whole) {
            st8(m, i0, mv);
        } else {
#pragma unroll
            for (int e = 0; e < kSwiPer; ++e)
                if (i0 + e < n) st(m, i0 + e, mv[e]);
        }
    }
}

template <class T>
__global__ void __launch_bounds__(kSwiThreads)
swiglu_bwd_kernel(const T* __restrict__ a, const T* __restrict__ b, const T* __restrict__ dm,
                  int64_t n, T* __restrict__ da, T* __restrict__ db) {
    const int64_t stride = (int64_t)gridDim.x * kSwiThreads * kSwiPer;
    for (int64_t i0 = ((int64_t)blockIdx.x * kSwiThreads + threadIdx.x) * kSwiPer; i0 < n; i0 += stride) {
        float av[kSwiPer], bv[kSwiPer], gv[kSwiPer], dav[kSwiPer], dbv[kSwiPer];
        const bool whole = i0 + kSwiPer <= n;
        if (whole) {
            ld8(a, i0, av);
            ld8(b, i0, bv);
            ld8(dm, i0, gv);
        } else {
#pragma unroll
            for (int e = 0; e < kSwiPer; ++e) {
                const bool ok = i0 + e < n;
                av[e] = ok ? ld(a, i0 + e) : 0.f;
                bv[e] = ok ? ld(b, i0 + e) : 0.f;
                gv[e] = ok ? ld(dm, i0 + e) : 0.f;
            }
        }
#pragma unroll
        for (int e = 0; e < kSwiPer; ++e) {
            const float s = sigmoid_f(av[e]);
            dbv[e] = gv[e] * (av[e] * s);
            dav[e] = gv[e] * bv[e] * (s * (1.0f + av[e] * (1.0f - s)));
        }
        if (whole) {
            st8(db, i0, dbv);
            st8(da, i0, dav);
        } else {
#pragma unroll
            for (int e = 0; e < kSwiPer; ++e) {
                if (i0 + e >= n) continue;
                st(db, i0 + e, dbv[e]);
                st(da, i0 + e, dav[e]);
            }
        }
    }
}

dim3 swiglu_grid(int64_t n) {
    const int64_t per_block = (int64_t)kSwiThreads * kSwiPer;
    return dim3((unsigned)std::max<int64_t>(1, std::min<int64_t>((n + per_block - 1) / per_block, 256 * 16)));
}

}  // namespace
}  // namespace mb

using namespace mb;

extern "C" int mb_swiglu_fwd(const void* a, const void* b, int64_t n, int dtype, void* m, void* stream) {
    MB_REQUIRE(n >= 0, "mb_swiglu_fwd: n=%lld < 0", (long long)n);
    if (dtype != MB_DTYPE_F32 && dtype != MB_DTYPE_BF16)
        return fail(MB_ERR_UNSUPPORTED, "mb_swiglu_fwd: dtype %d (supported: MB_DTYPE_F32, MB_DTYPE_BF16)", dtype);
    if (n == 0) return MB_OK;
    MB_REQUIRE(a && b && m, "mb_swiglu_fwd: null pointer argument");
    MB_REQUIRE((((uintptr_t)a | (uintptr_t)b | (uintptr_t)m) & 31) == 0,
               "mb_swiglu_fwd: pointers must be 32-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (dtype == MB_DTYPE_F32)
        hipLaunchKernelGGL(swiglu_fwd_kernel<float>, swiglu_grid(n), dim3(kSwiThreads), 0, st,
                           (const float*)a, (const float*)b, n, (float*)m);
    else
        hipLaunchKernelGGL(swiglu_fwd_kernel<__bf16>, swiglu_grid(n), dim3(kSwiThreads), 0, st,
                           (const __bf16*)a, (const __bf16*)b, n, (__bf16*)m);
    return check_launch("mb_swiglu_fwd");
}

extern "C" int mb_swiglu_bwd(const void* a, const void* b, const void* dm, int64_t n, int dtype,
                             void* da, void* db, void* stream) {
    MB_REQUIRE(n >= 0, "mb_swiglu_bwd: n=%lld < 0", (long long)n);
    if (dtype != MB_DTYPE_F32 && dtype != MB_DTYPE_BF16)
        return fail(MB_ERR_UNSUPPORTED, "mb_swiglu_bwd: dtype %d (supported: MB_DTYPE_F32, MB_DTYPE_BF16)", dtype);
    if (n == 0) return MB_OK;
    MB_REQUIRE(a && b && dm && da && db, "mb_swiglu_bwd: null pointer argument");
    MB_REQUIRE((((uintptr_t)a | (uintptr_t)b | (uintptr_t)dm | (uintptr_t)da | (uintptr_t)db) & 31) == 0,
               "mb_swiglu_bwd: pointers must be 32-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (dtype == MB_DTYPE_F32)
        hipLaunchKernelGGL(swiglu_bwd_kernel<float>, swiglu_grid(n), dim3(kSwiThreads), 0, st,
                           (const float*)a, (const float*)b, (const float*)dm, n, (float*)da, (float*)db);
    else
        hipLaunchKernelGGL(swiglu_bwd_kernel<__bf16>, swiglu_grid(n), dim3(kSwiThreads), 0, st,
                           (const __bf16*)a, (const __bf16*)b, (const __bf16*)dm, n, (__bf16*)da,
                           (__bf16*)db);
    return check_launch("mb_swiglu_bwd");
}
