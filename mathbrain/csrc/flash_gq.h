// Query prologue of the flash-EMA attention forward (its GQ variants): the workgroup computes
// its own queries, so Q never exists in HBM.
//
// Q = q_proj(LayerNorm(x_q * SiLU((C_seq + 1) W_pe)))  (the symmetric query gating of
// mathbrain/triton_fused_gating.py:179-197 followed by q_proj, model.py:75), for the
// workgroup's 32 steps.  The LayerNorm output x_ln is computed in LDS with the operations of
// gating_fwd_kernel in the same order, so it is the gating kernel's result bit for bit.
// q_proj runs on the matrix cores with both operands split into fp16 hi + lo pairs and
// three products accumulated in fp32 (lo terms first), ~2^-22 relative per product: the
// queries agree with an fp32 GEMM to fp32 rounding.
#pragma once
#include "flash_common.h"

namespace mb {

// Arguments of the GQ kernels.
struct FlashArgsG : FlashArgsV {
    const float* xq;  // x_q [B, L, D] rows, columns contiguous
    int64_t xq_sb, xq_sl;
    const float* Cq;  // C_seq [B, L, N], columns contiguous
    int64_t c_sb, c_sl;
    const float* lnw;  // ln_q.weight, ln_q.bias [D]
    const float* lnb;
    float eps;
    const float* Wq;  // q_proj.weight [D, D]: row o (output), column i (input), contiguous
};

// Argument type of a kernel variant: the GQ variants take FlashArgsG whatever VR is (it
// extends FlashArgsV); the others keep their own types and layouts.
template <bool VR, bool GQ> struct FlashArgsK { using type = typename FlashArgsOf<VR>::type; };
template <bool VR> struct FlashArgsK<VR, true> { using type = FlashArgsG; };

constexpr int kGQRows = kTB;  // steps per workgroup

// LDS of the forward prologue: x_emb / x_ln [32][D] fp32, (C_seq + 1)^T [N][32], row
// statistics [32][2].
__host__ __device__ inline size_t gq_fwd_lds_bytes(int D, int N) {
    return ((size_t)kGQRows * D + (size_t)N * kGQRows + 2 * kGQRows) * 4;
}

__device__ inline float gq_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ inline float gq_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// x_ln of steps t0 .. t0 + 31 over all D columns into xl[32][D] (LDS; steps past L give
// rows that nothing reads).  Every thread of the workgroup takes part; ends synchronised.
template <bool SILU>
__device__ void gq_layer_norm(const FlashArgsG& a, int b, int t0, int D, float* xl) {
    float* cst = xl + kGQRows * D;         // [N][32]: C_seq + 1, transposed
    float* stats = cst + a.N * kGQRows;    // [32][2]: mean, rstd
    const int nthr = blockDim.x;
    for (int i = threadIdx.x; i < kGQRows * a.N; i += nthr) {
        const int r = i / a.N;
        const int n = i % a.N;
        const int t = t0 + r;
        cst[n * kGQRows + r] = t < a.L ? a.Cq[(int64_t)b * a.c_sb + (int64_t)t * a.c_sl + n] + 1.0f : 0.f;
    }
    __syncthreads();
    for (int col = threadIdx.x; col < D; col += nthr) {
        float pre[kGQRows];
#pragma unroll
        for (int r = 0; r < kGQRows; ++r) pre[r] = 0.f;
        for (int n = 0; n < a.N; ++n) {
            const float w = a.W[(int64_t)n * D + col];
            const float4* c4 = reinterpret_cast<const float4*>(cst + n * kGQRows);
#pragma unroll
            for (int q = 0; q < kGQRows / 4; ++q) {
                const float4 c = c4[q];
                pre[4 * q + 0] = __builtin_fmaf(c.x, w, pre[4 * q + 0]);
                pre[4 * q + 1] = __builtin_fmaf(c.y, w, pre[4 * q + 1]);
                pre[4 * q + 2] = __builtin_fmaf(c.z, w, pre[4 * q + 2]);
                pre[4 * q + 3] = __builtin_fmaf(c.w, w, pre[4 * q + 3]);
            }
        }
#pragma unroll
        for (int r = 0; r < kGQRows; ++r) {
            const int t = t0 + r;
            const float xv = t < a.L ? a.xq[(int64_t)b * a.xq_sb + (int64_t)t * a.xq_sl + col] : 0.f;
            const float g = SILU ? pre[r] * gq_sigmoid(pre[r]) : pre[r];
            xl[r * D + col] = xv * g;
        }
    }
    __syncthreads();
    // row statistics, one wave per row, in gating_fwd_kernel's order
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    for (int r = wave; r < kGQRows; r += nthr / 64) {
        float s = 0.f;
        for (int c = lane; c < D; c += 64) s += xl[r * D + c];
        const float mean = gq_wave_sum(s) / (float)D;
        float v = 0.f;
        for (int c = lane; c < D; c += 64) {
            const float dd = xl[r * D + c] - mean;
            v = __builtin_fmaf(dd, dd, v);
        }
        const float var = gq_wave_sum(v) / (float)D;
        if (lane == 0) {
            stats[2 * r] = mean;
            stats[2 * r + 1] = 1.0f / sqrtf(var + a.eps);
        }
    }
    __syncthreads();
    for (int col = threadIdx.x; col < D; col += nthr) {
        const float w = a.lnw[col];
        const float bb = a.lnb[col];
#pragma unroll 8
        for (int r = 0; r < kGQRows; ++r)
            xl[r * D + col] = (xl[r * D + col] - stats[2 * r]) * stats[2 * r + 1] * w + bb;
    }
    __syncthreads();
}

// x ≈ hi + lo with both halves fp16.
__device__ inline void gq_split8(float4 x0, float4 x1, f16x8& hi, f16x8& lo) {
    const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        hi[e] = (_Float16)v[e];
        lo[e] = (_Float16)(v[e] - (float)hi[e]);
    }
}

__device__ inline f32x4 gq_mfma3(f16x8 ah, f16x8 al, f16x8 bh, f16x8 bl, f32x4 acc) {
    acc = mfma16x16x32(al, bh, acc);
    acc = mfma16x16x32(ah, bl, acc);
    return mfma16x16x32(ah, bh, acc);
}

// Forward queries of head h from x_ln in LDS: q[tt][dt][i] = Q[t0 + 16 tt + c16][h HD + 16 dt
// + 4 g + i], i.e. Q^T = W_q x_ln^T with W_q's rows as the A operand and x_ln's rows as B.
// W_q's columns stream from global memory one 32-column step ahead of the products.
template <int HD>
__device__ void gq_project_fwd(const FlashArgsG& a, int h, int D, const float* xl, int lane,
                               f32x4 (&q)[2][HD / 16]) {
    constexpr int DT = HD / 16;
    const int c16 = lane & 15;
    const int g = lane >> 4;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) q[tt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float* wrow = a.Wq + (int64_t)(h * HD + c16) * D + 8 * g;
    float4 wn[DT][2];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const float* w = wrow + (int64_t)16 * dt * D + k0;
            wn[dt][0] = *reinterpret_cast<const float4*>(w);
            wn[dt][1] = *reinterpret_cast<const float4*>(w + 4);
        }
    };
    fetch(0);
    for (int k0 = 0; k0 < D; k0 += 32) {
        f16x8 ah[DT], al[DT];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) gq_split8(wn[dt][0], wn[dt][1], ah[dt], al[dt]);
        if (k0 + 32 < D) fetch(k0 + 32);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const float* x = xl + (16 * tt + c16) * D + k0 + 8 * g;
            f16x8 bh, bl;
            gq_split8(*reinterpret_cast<const float4*>(x), *reinterpret_cast<const float4*>(x + 4), bh, bl);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) q[tt][dt] = gq_mfma3(ah[dt], al[dt], bh, bl, q[tt][dt]);
        }
    }
}


}  // namespace mb
