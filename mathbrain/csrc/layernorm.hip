// LayerNorm forward and backward on gfx950 (the model's ln_kv over the embedding rows).
//
// Replaces nn.LayerNorm's forward and backward where SlotAttentionLayer normalises the slot
// embeddings (mathbrain/model.py:63-64, ln_kv(E)): per row of D elements
//   forward   mu = mean(x),  rstd = rsqrt(mean((x - mu)^2) + eps),  y = (x - mu) rstd w + b
//   backward  xh = (x - mu) rstd,  g = dy w,  dx = rstd (g - mean(g) - xh mean(g xh)),
//             dw = sum_rows dy xh,  db = sum_rows dy
// One wave per row (lane l holds columns l, l + 64, ...; the two-pass statistics stay in
// registers); the backward walks rows with a grid stride on 512 workgroups, keeps its column
// sums in registers and adds them once per workgroup with atomics.
#include "common.h"

#include <algorithm>

namespace mb {
namespace {

constexpr int kLnThreads = 256;  // four rows (waves) per workgroup
constexpr int kLnMaxD = 1024;
constexpr int kLnBwdBlocks = 512;

__device__ inline float ln_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int PER>
__global__ void __launch_bounds__(kLnThreads)
ln_fwd_kernel(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
              int64_t rows, int D, float eps, float* __restrict__ y, float* __restrict__ mean,
              float* __restrict__ rstd) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kLnThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;  // the row is uniform across the wave
    const float* xr = x + row * D;
    float v[PER];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        v[i] = d < D ? xr[d] : 0.f;
        s += v[i];
    }
    const float mu = ln_wave_sum(s) / (float)D;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        const float c = d < D ? v[i] - mu : 0.f;
        ss = __builtin_fmaf(c, c, ss);
    }
    const float r = rsqrtf(ln_wave_sum(ss) / (float)D + eps);
    float* yr = y + row * D;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        if (d < D) yr[d] = __builtin_fmaf((v[i] - mu) * r, w[d], bias[d]);
    }
    if (lane == 0) {
        mean[row] = mu;
        rstd[row] = r;
    }
}

template <int PER>
__global__ void __launch_bounds__(kLnThreads)
ln_bwd_kernel(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ dy,
              const float* __restrict__ mean, const float* __restrict__ rstd, int64_t rows, int D,
              float* __restrict__ dx, float* __restrict__ dw, float* __restrict__ db) {
    __shared__ float part[2][kLnThreads / 64][kLnMaxD];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t nwaves = (int64_t)gridDim.x * (kLnThreads / 64);
    float wv[PER], accw[PER], accb[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        wv[i] = d < D ? w[d] : 0.f;
        accw[i] = 0.f;
        accb[i] = 0.f;
    }
    const float invD = 1.0f / (float)D;
    // rows are software-pipelined: the next row's loads are issued before this row's math
    int64_t row = (int64_t)blockIdx.x * (kLnThreads / 64) + wave;
    float xn[PER], gn[PER], mun = 0.f, rn = 0.f;
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
        mun = okr ? mean[rr] : 0.f;
        rn = okr ? rstd[rr] : 0.f;
    };
    fetch(row);
    for (; row < rows; row += nwaves) {
        float xh[PER], gv[PER];
        const float mu = mun, r = rn;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            xh[i] = (xn[i] - mu) * r;
            gv[i] = gn[i];
        }
        fetch(row + nwaves);
        float sg = 0.f, sgx = 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const float g = gv[i] * wv[i];
            sg += g;
            sgx = __builtin_fmaf(g, xh[i], sgx);
        }
        const float mg = ln_wave_sum(sg) * invD;
        const float mgx = ln_wave_sum(sgx) * invD;
        float* dxr = dx + row * D;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int d = lane + 64 * i;
            if (d < D) dxr[d] = r * (gv[i] * wv[i] - mg - xh[i] * mgx);
            accw[i] = __builtin_fmaf(gv[i], xh[i], accw[i]);
            accb[i] += gv[i];
        }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int d = lane + 64 * i;
        if (d < D) {
            part[0][wave][d] = accw[i];
            part[1][wave][d] = accb[i];
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += kLnThreads) {
        float sw = 0.f, sb = 0.f;
#pragma unroll
        for (int k = 0; k < kLnThreads / 64; ++k) {
            sw += part[0][k][d];
            sb += part[1][k][d];
        }
        atomicAdd(dw + d, sw);
        atomicAdd(db + d, sb);
    }
}

__global__ void ln_zero_kernel(float* p, float* q, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        p[i] = 0.f;
        q[i] = 0.f;
    }
}

int ln_per(int D) {
    const int need = (D + 63) / 64;
    return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : 16;
}

}  // namespace
}  // namespace mb

using namespace mb;

extern "C" int mb_layernorm_fwd(const float* x, const float* w, const float* b, int64_t rows, int D,
                                float eps, float* y, float* mean, float* rstd, void* stream) {
    MB_REQUIRE(rows >= 0, "mb_layernorm_fwd: rows=%lld < 0", (long long)rows);
    if (D < 1 || D > kLnMaxD)
        return fail(MB_ERR_UNSUPPORTED, "mb_layernorm_fwd: D=%d (supported: 1..%d)", D, kLnMaxD);
    if (rows == 0) return MB_OK;
    MB_REQUIRE(x && w && b && y && mean && rstd, "mb_layernorm_fwd: null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    const int64_t blocks = (rows + kLnThreads / 64 - 1) / (kLnThreads / 64);
    MB_REQUIRE(blocks <= 0x7fffffff, "mb_layernorm_fwd: rows=%lld too many", (long long)rows);
    const dim3 grid((unsigned)blocks), blk(kLnThreads);
#define MB_LN_FWD(P) hipLaunchKernelGGL(ln_fwd_kernel<P>, grid, blk, 0, st, x, w, b, rows, D, eps, y, mean, rstd)
    switch (ln_per(D)) {
        case 1: MB_LN_FWD(1); break;
        case 2: MB_LN_FWD(2); break;
        case 4: MB_LN_FWD(4); break;
        case 8: MB_LN_FWD(8); break;
        default: MB_LN_FWD(16); break;
    }
#undef MB_LN_FWD
    return check_launch("mb_layernorm_fwd");
}

extern "C" int mb_layernorm_bwd(const float* x, const float* w, const float* dy, const float* mean,
                                const float* rstd, int64_t rows, int D, float* dx, float* dw, float* db,
                                void* stream) {
    MB_REQUIRE(rows >= 0, "mb_layernorm_bwd: rows=%lld < 0", (long long)rows);
    if (D < 1 || D > kLnMaxD)
        return fail(MB_ERR_UNSUPPORTED, "mb_layernorm_bwd: D=%d (supported: 1..%d)", D, kLnMaxD);
    MB_REQUIRE(dw && db, "mb_layernorm_bwd: null dw / db");
    hipStream_t st = (hipStream_t)stream;
    // dw and db are accumulated with atomics: cleared here with a fill kernel (no memset)
    hipLaunchKernelGGL(ln_zero_kernel, dim3((D + 255) / 256), dim3(256), 0, st, dw, db, D);
    if (rows == 0) return check_launch("mb_layernorm_bwd");
    MB_REQUIRE(x && w && dy && mean && rstd && dx, "mb_layernorm_bwd: null pointer argument");
    // as many workgroups as keep the CUs busy; each adds its 2 x D column sums once
    const int64_t want = (rows + kLnThreads / 64 - 1) / (kLnThreads / 64);
    const dim3 grid((unsigned)std::min<int64_t>(want, kLnBwdBlocks)), blk(kLnThreads);
#define MB_LN_BWD(P) \
    hipLaunchKernelGGL(ln_bwd_kernel<P>, grid, blk, 0, st, x, w, dy, mean, rstd, rows, D, dx, dw, db)
    switch (ln_per(D)) {
        case 1: MB_LN_BWD(1); break;
        case 2: MB_LN_BWD(2); break;
        case 4: MB_LN_BWD(4); break;
        case 8: MB_LN_BWD(8); break;
        default: MB_LN_BWD(16); break;
    }
#undef MB_LN_BWD
    return check_launch("mb_layernorm_bwd");
}
