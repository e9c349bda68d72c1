// Factored linear EMA (mathbrain/factored_ema.py:22-146) on gfx950, fp32-accurate.
//
// Per sequence b and head h the reference runs a per-step state recurrence
// (S_n <- rho_n S_n; o_t = sum_n (q_t ⊙ W_n)^T S_n; S_n += e_k[x_t] ⊗ e_v[x_t]), which is
// O(L N hd^2) and keeps an [N, hd, hd] state per (b, h).  Here the same output is split
// into two exact parts:
//
//   token part   o_t += sum_{s<t} A[t,s] e_v[x_s],  A[t,s] = sum_i q_t[i] e_k[x_s][i] G[t-s][i],
//                G[d] = sum_n rho_n^d W_n  (a [L+1, D] table, one small GEMM on the host side)
//                -> O(L^2 hd) pair work with no state at all (L < N hd at the model's shapes);
//   c_base part  o_t += sum_n rho_n^(t+1) sum_i q_t[i] W_n[i] S_n[i,:],
//                S_n = sum_k c_base[k,n] e_k[u_k] ⊗ e_v[u_k]  (the reference's initial state).
//
// The kernels: fac_outer (scaled outer-product accumulation, builds S_n and the backward's
// M_n = sum_t rho_n^(t+1) q_t ⊗ dO_t), fac_apply (contracts such a state with rows: the
// c_base part of o, of dQ and of the slot gradients), and the three token-pair kernels
// (forward; backward by rows for dQ, by columns for the token embedding gradients, by
// diagonals for dG[d], from which dW_pe = P dG with P[n,d] = rho_n^d).
#include "flash_common.h"

namespace mb {
namespace {

__device__ inline int64_t clamp_row(const int64_t* idx, int64_t e, int64_t nrows) {
    int64_t r = idx ? idx[e] : e;
    r = r < 0 ? 0 : r;
    return r < nrows ? r : -1;
}

// out[b,h,n,i,j] = sum_r alpha[b,r,n] X[row_x(b,r), h*HD+i] Y[row_y(b,r), h*HD+j].
// Block (n block, h, b); thread (n, i) with 256/HD rates per block; the Y row of each r is
// the same for the whole block.
template <int HD>
__global__ void __launch_bounds__(256)
fac_outer_kernel(const float* __restrict__ X, const int64_t* __restrict__ xrow,
                 const float* __restrict__ Y, const int64_t* __restrict__ yrow, int64_t ld,
                 int64_t nrows, const float* __restrict__ alpha, int64_t as_b, int64_t as_r,
                 int64_t as_n, int R, int H, int N, float* __restrict__ out) {
    constexpr int NB = 256 / HD;
    const int b = blockIdx.z, h = blockIdx.y;
    const int n = blockIdx.x * NB + threadIdx.x / HD;
    const int i = threadIdx.x % HD;
    const bool nok = n < N;
    float acc[HD];
#pragma unroll
    for (int j = 0; j < HD; ++j) acc[j] = 0.0f;
    for (int r = 0; r < R; ++r) {
        const float a = nok ? alpha[b * as_b + r * as_r + n * as_n] : 0.0f;
        if (a == 0.0f) continue;
        const int64_t e = (int64_t)b * R + r;
        const int64_t rx = clamp_row(xrow, e, nrows), ry = clamp_row(yrow, e, nrows);
        if (rx < 0 || ry < 0) continue;
        const float av = a * X[rx * ld + h * HD + i];
        const float* yr = Y + ry * ld + h * HD;
#pragma unroll
        for (int j = 0; j < HD; ++j) acc[j] = __builtin_fmaf(av, yr[j], acc[j]);
    }
    if (nok) {
        float* o = out + ((((int64_t)b * H + h) * N + n) * HD + i) * HD;
#pragma unroll
        for (int j = 0; j < HD; ++j) o[j] = acc[j];
    }
}

// TRANS = false: out[b,r,h,i] (+)= sum_n alpha[b,r,n] sum_j w[n,i] M[b,h,n,i,j] Y[row(b,r),h,j]
// TRANS = true:  out[b,r,h,j] (+)= sum_n alpha[b,r,n] sum_i w[n,i] M[b,h,n,i,j] Y[row(b,r),h,i]
// (w NULL: 1).  A register-tiled GEMM per rate: block (kApplyRows rows, h, b), 16 x 16 threads
// each owning kApplyRows/16 rows x HD/16 outputs; the Y rows and the rows' alphas are staged
// once, the (scaled, oriented) M_n tile once per rate, with the next rate's tile loaded into
// registers while the current one is used.
constexpr int kApplyRows = 128;

template <int HD, bool TRANS>
__global__ void __launch_bounds__(256)
fac_apply_kernel(const float* __restrict__ M, const float* __restrict__ w, int64_t ldw,
                 const float* __restrict__ Y, const int64_t* __restrict__ yrow, int64_t ld,
                 int64_t nrows, const float* __restrict__ alpha, int64_t as_b, int64_t as_r,
                 int64_t as_n, int R, int H, int N, float* __restrict__ out, int64_t ldo,
                 int accumulate) {
    constexpr int RS = HD + 4;              // LDS row stride (floats)
    constexpr int CO = HD / 16;             // outputs per thread
    constexpr int RO = kApplyRows / 16;     // rows per thread
    constexpr int AN = 16;                  // rates whose alphas are staged at a time
    constexpr int ME = HD * HD / 256;       // M_n elements per thread
    __shared__ __align__(16) float Ys[kApplyRows * RS];
    __shared__ __align__(16) float Mt[HD * RS];
    __shared__ float As[kApplyRows * AN];
    const int b = blockIdx.z, h = blockIdx.y;
    const int r0 = blockIdx.x * kApplyRows;
    const int tid = threadIdx.x;
    const int tr = tid / 16, to = tid % 16;
    for (int e = tid; e < kApplyRows * (HD / 4); e += 256) {
        const int rr = e / (HD / 4), c = e % (HD / 4);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r0 + rr < R) {
            const int64_t ry = clamp_row(yrow, (int64_t)b * R + r0 + rr, nrows);
            if (ry >= 0) v = *reinterpret_cast<const float4*>(Y + ry * ld + h * HD + 4 * c);
        }
        *reinterpret_cast<float4*>(Ys + rr * RS + 4 * c) = v;
    }
    const float* Mb = M + ((int64_t)b * H + h) * N * HD * HD;
    float mreg[ME];
    auto load_m = [&](int n) {
#pragma unroll
        for (int q = 0; q < ME; ++q) {
            const int e = tid + 256 * q;
            float v = Mb[(int64_t)n * HD * HD + e];
            if (w) v *= w[n * ldw + h * HD + e / HD];
            mreg[q] = v;
        }
    };
    load_m(0);
    float acc[RO][CO];
#pragma unroll
    for (int a = 0; a < RO; ++a)
#pragma unroll
        for (int c = 0; c < CO; ++c) acc[a][c] = 0.0f;
    for (int n = 0; n < N; ++n) {
        __syncthreads();
        if (n % AN == 0) {
            for (int e = tid; e < kApplyRows * AN; e += 256) {
                const int rr = e / AN, nn = n + e % AN;
                As[e] = (r0 + rr < R && nn < N)
                            ? alpha[b * as_b + (int64_t)(r0 + rr) * as_r + nn * as_n] : 0.0f;
            }
        }
#pragma unroll
        for (int q = 0; q < ME; ++q) {
            const int e = tid + 256 * q;
            const int i = e / HD, j = e % HD;
            if (TRANS) Mt[j * RS + i] = mreg[q];
            else Mt[i * RS + j] = mreg[q];
        }
        __syncthreads();
        if (n + 1 < N) load_m(n + 1);
        float sacc[RO][CO];
#pragma unroll
        for (int a = 0; a < RO; ++a)
#pragma unroll
            for (int c = 0; c < CO; ++c) sacc[a][c] = 0.0f;
#pragma unroll 2
        for (int k0 = 0; k0 < HD; k0 += 4) {
            float4 mv[CO];
#pragma unroll
            for (int c = 0; c < CO; ++c) mv[c] = *reinterpret_cast<const float4*>(Mt + (to * CO + c) * RS + k0);
#pragma unroll
            for (int a = 0; a < RO; ++a) {
                const float4 yv = *reinterpret_cast<const float4*>(Ys + (tr * RO + a) * RS + k0);
#pragma unroll
                for (int c = 0; c < CO; ++c) {
                    float t = sacc[a][c];
                    t = __builtin_fmaf(yv.x, mv[c].x, t);
                    t = __builtin_fmaf(yv.y, mv[c].y, t);
                    t = __builtin_fmaf(yv.z, mv[c].z, t);
                    t = __builtin_fmaf(yv.w, mv[c].w, t);
                    sacc[a][c] = t;
                }
            }
        }
#pragma unroll
        for (int a = 0; a < RO; ++a) {
            const float al = As[(tr * RO + a) * AN + n % AN];
#pragma unroll
            for (int c = 0; c < CO; ++c) acc[a][c] = __builtin_fmaf(al, sacc[a][c], acc[a][c]);
        }
    }
#pragma unroll
    for (int a = 0; a < RO; ++a) {
        const int r = r0 + tr * RO + a;
        if (r >= R) continue;
        float* dst = out + ((int64_t)b * R + r) * ldo + h * HD + to * CO;
#pragma unroll
        for (int c = 0; c < CO; ++c) dst[c] = accumulate ? dst[c] + acc[a][c] : acc[a][c];
    }
}

// ---- MFMA forms of the state kernels (hd = 64) ------------------------------------------
//
// The state contractions are plain GEMMs per rate.  These forms run them on the bf16 matrix
// cores with every fp32 operand split into bf16 hi + lo parts and three products
// (hi*hi + hi*lo + lo*hi, fp32 accumulation), which keeps about 2^-16 relative error per
// product.  Operand layout of v_mfma_f32_16x16x16_bf16: A[row = lane%16][k = 4 (lane/16) + e],
// B[k = 4 (lane/16) + e][col = lane%16], D[row = 4 (lane/16) + i][col = lane%16].

__device__ inline void split_bf16x4(const float (&v)[4], bf16x4& hi, bf16x4& lo) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const __bf16 t = (__bf16)v[e];
        hi[e] = t;
        lo[e] = (__bf16)(v[e] - (float)t);
    }
}

__device__ inline f32x4 mfma3(bf16x4 ah, bf16x4 al, bf16x4 bh, bf16x4 bl, f32x4 c) {
    c = mfma16x16x16(ah, bh, c);
    c = mfma16x16x16(ah, bl, c);
    return mfma16x16x16(al, bh, c);
}

// fac_apply_kernel for hd = 64: block (64 rows, h, b); wave w owns outputs [16w, 16w + 16)
// of the 64 rows (4 row tiles); the Y rows are split once, each rate's M_n tile per rate.
template <bool TRANS>
__global__ void __launch_bounds__(256)
fac_apply_mfma_kernel(const float* __restrict__ M, const float* __restrict__ w, int64_t ldw,
                      const float* __restrict__ Y, const int64_t* __restrict__ yrow, int64_t ld,
                      int64_t nrows, const float* __restrict__ alpha, int64_t as_b, int64_t as_r,
                      int64_t as_n, int R, int H, int N, float* __restrict__ out, int64_t ldo,
                      int accumulate) {
    constexpr int HD = 64;
    constexpr int AN = 64;
    __shared__ float As[64 * AN];
    const int b = blockIdx.z, h = blockIdx.y;
    const int r0 = blockIdx.x * 64;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c16 = lane & 15, g = lane >> 4;
    bf16x4 ahi[4][4], alo[4][4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
        const int r = r0 + 16 * rt + c16;
        const int64_t ry = r < R ? clamp_row(yrow, (int64_t)b * R + r, nrows) : -1;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (ry >= 0) {
                const float4 q = *reinterpret_cast<const float4*>(Y + ry * ld + h * HD + 16 * kt + 4 * g);
                v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
            }
            split_bf16x4(v, ahi[rt][kt], alo[rt][kt]);
        }
    }
    f32x4 acc[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int o = 16 * wv + c16;
    const float* Mb = M + ((int64_t)b * H + h) * N * HD * HD;
    for (int n = 0; n < N; ++n) {
        if (n % AN == 0) {
            __syncthreads();
            for (int e = tid; e < 64 * AN; e += 256) {
                const int rr = e / AN, nn = n + e % AN;
                As[e] = (r0 + rr < R && nn < N)
                            ? alpha[b * as_b + (int64_t)(r0 + rr) * as_r + nn * as_n] : 0.0f;
            }
            __syncthreads();
        }
        const float* Mn = Mb + (int64_t)n * HD * HD;
        bf16x4 bhi[4], blo[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            float v[4];
            if (!TRANS) {  // B[k][o] = w[n, o] M_n[o][k]
                const float4 q = *reinterpret_cast<const float4*>(Mn + o * HD + 16 * kt + 4 * g);
                const float ws = w ? w[n * ldw + h * HD + o] : 1.0f;
                v[0] = q.x * ws; v[1] = q.y * ws; v[2] = q.z * ws; v[3] = q.w * ws;
            } else {       // B[k][o] = w[n, k] M_n[k][o]
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = 16 * kt + 4 * g + e;
                    v[e] = Mn[k * HD + o] * (w ? w[n * ldw + h * HD + k] : 1.0f);
                }
            }
            split_bf16x4(v, bhi[kt], blo[kt]);
        }
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) sacc = mfma3(ahi[rt][kt], alo[rt][kt], bhi[kt], blo[kt], sacc);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[rt][i] = __builtin_fmaf(As[(16 * rt + 4 * g + i) * AN + n % AN], sacc[i], acc[rt][i]);
        }
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + 16 * rt + 4 * g + i;
            if (r >= R) continue;
            float* dst = out + ((int64_t)b * R + r) * ldo + h * HD + o;
            *dst = accumulate ? *dst + acc[rt][i] : acc[rt][i];
        }
}

// fac_outer_kernel for hd = 64: block (4 rates, h, b), wave w = rate 4 blockIdx.x + w, the
// whole 64 x 64 output of its rate in 16 tiles.  The walked rows come in blocks of 32 (two
// MFMA k steps), staged in LDS once for the four rates: they share the X and Y rows and
// differ only in the weights alpha.
constexpr int kOuterRows = 32;

__global__ void __launch_bounds__(256)
fac_outer_mfma_kernel(const float* __restrict__ X, const int64_t* __restrict__ xrow,
                      const float* __restrict__ Y, const int64_t* __restrict__ yrow, int64_t ld,
                      int64_t nrows, const float* __restrict__ alpha, int64_t as_b, int64_t as_r,
                      int64_t as_n, int R, int H, int N, float* __restrict__ out) {
    constexpr int HD = 64;
    constexpr int RS = HD + 4;
    __shared__ __align__(16) float Xs[kOuterRows * RS];
    __shared__ __align__(16) float Ys[kOuterRows * RS];
    const int b = blockIdx.z, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int n = blockIdx.x * 4 + (tid >> 6);
    const int c16 = lane & 15, g = lane >> 4;
    const bool nv = n < N;
    f32x4 acc[4][4];
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) acc[it][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < R; k0 += kOuterRows) {
        __syncthreads();
        // stage the block's rows: thread tid copies float4 (tid % 16) of row tid / 16 of X
        // and of Y (rows of zero weight for every rate are staged as zeros)
        for (int e = tid; e < kOuterRows * (HD / 4); e += 256) {
            const int rr = e / (HD / 4), c = e % (HD / 4);
            const int r = k0 + rr;
            float4 vx = make_float4(0.f, 0.f, 0.f, 0.f), vy = vx;
            if (r < R) {
                const int64_t ex = (int64_t)b * R + r;
                const int64_t rx = clamp_row(xrow, ex, nrows), ry = clamp_row(yrow, ex, nrows);
                if (rx >= 0 && ry >= 0) {
                    vx = *reinterpret_cast<const float4*>(X + rx * ld + h * HD + 4 * c);
                    vy = *reinterpret_cast<const float4*>(Y + ry * ld + h * HD + 4 * c);
                }
            }
            *reinterpret_cast<float4*>(Xs + rr * RS + 4 * c) = vx;
            *reinterpret_cast<float4*>(Ys + rr * RS + 4 * c) = vy;
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < kOuterRows / 16; ++ks) {
            float al[4];
            bool any = false;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = k0 + 16 * ks + 4 * g + e;
                al[e] = (nv && r < R) ? alpha[b * as_b + (int64_t)r * as_r + n * as_n] : 0.0f;
                any = any || al[e] != 0.0f;
            }
            if (!__any(any)) continue;
            const float* xr = Xs + (16 * ks + 4 * g) * RS;
            const float* yr = Ys + (16 * ks + 4 * g) * RS;
            bf16x4 ahi[4], alo[4], bhi[4], blo[4];
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = al[e] * xr[e * RS + 16 * it + c16];
                split_bf16x4(v, ahi[it], alo[it]);
            }
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = yr[e * RS + 16 * jt + c16];
                split_bf16x4(v, bhi[jt], blo[jt]);
            }
#pragma unroll
            for (int it = 0; it < 4; ++it)
#pragma unroll
                for (int jt = 0; jt < 4; ++jt) acc[it][jt] = mfma3(ahi[it], alo[it], bhi[jt], blo[jt], acc[it][jt]);
        }
    }
    if (!nv) return;
    float* o = out + (((int64_t)b * H + h) * N + n) * HD * HD;
#pragma unroll
    for (int it = 0; it < 4; ++it)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[(16 * it + 4 * g + i) * HD + 16 * jt + c16] = acc[it][jt][i];
}

__device__ inline bool tok_ok(int64_t v, int64_t V) { return v >= 0 && v < V; }

// ---- token pairs ---------------------------------------------------------------------------
//
// The four kernels share one shape.  A block of 4 waves covers 64 steps of one (b, h) on its
// lanes (the "lane steps") and walks the 64-step blocks of the other index (the "walked
// steps"); the 4 waves take every fourth walked step and their partial sums are added in LDS
// at the end.  Each tile stages in LDS the rows of its walked block (q, dO, e_k or e_v: one
// row for the whole wave, read by every lane at the same address) and the 127
// distance-dependent G rows it needs (a different row per lane).  Each lane holds whole
// hd-rows in registers, so no cross-lane sums are needed per pair.

constexpr int kTW = 4;  // waves per block

template <int HD>
struct TokLds {
    static constexpr int RS = HD + 4;  // padded row stride (floats) of the staged rows
    static constexpr int GROWS = 127;
};

// Stages rows [lo, lo + n) of a [rows_total, D] table (head slice h) into dst with stride RS;
// rows outside [0, rows_total) are zero.
template <int HD>
__device__ inline void stage_rows(float* dst, const float* src, int64_t D, int h, int lo, int n,
                                  int rows_total) {
    constexpr int RS = TokLds<HD>::RS;
    constexpr int C4 = HD / 4;
    for (int e = threadIdx.x; e < n * C4; e += 64 * kTW) {
        const int r = e / C4, c = e % C4;
        const int row = lo + r;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (row >= 0 && row < rows_total)
            v = *reinterpret_cast<const float4*>(src + (int64_t)row * D + h * HD + 4 * c);
        *reinterpret_cast<float4*>(dst + r * RS + 4 * c) = v;
    }
}

// Same for token-indexed rows: row r is E[x[b, lo + r]] (zero outside [0, L) or for ids
// outside [0, V)).
template <int HD>
__device__ inline void stage_tok_rows(float* dst, const float* E, const int64_t* xb, int64_t V,
                                      int64_t D, int h, int lo, int n, int L) {
    constexpr int RS = TokLds<HD>::RS;
    constexpr int C4 = HD / 4;
    for (int e = threadIdx.x; e < n * C4; e += 64 * kTW) {
        const int r = e / C4, c = e % C4;
        const int s = lo + r;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (s >= 0 && s < L) {
            const int64_t xs = xb[s];
            if (tok_ok(xs, V)) v = *reinterpret_cast<const float4*>(E + xs * D + h * HD + 4 * c);
        }
        *reinterpret_cast<float4*>(dst + r * RS + 4 * c) = v;
    }
}

// Adds the kTW waves' per-lane rows acc[HD] in LDS (red holds (kTW-1)*64*HD floats) and
// leaves the sum in wave 0.
template <int HD>
__device__ inline void reduce_waves(float (&acc)[HD], float* red) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (w > 0) {
#pragma unroll
        for (int k = 0; k < HD; ++k) red[((w - 1) * HD + k) * 64 + lane] = acc[k];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
        for (int k = 0; k < HD; ++k) {
#pragma unroll
            for (int v = 0; v < kTW - 1; ++v) acc[k] += red[(v * HD + k) * 64 + lane];
        }
    }
}

// LDS of a token-pair block: the tile's 127 distance rows plus the walked block's two row
// sets (64 rows each), or the wave partials at the end.
template <int HD>
constexpr int tok_lds_floats() {
    constexpr int a = (TokLds<HD>::GROWS + 2 * 64) * TokLds<HD>::RS;
    constexpr int r = (kTW - 1) * 64 * HD;
    return a > r ? a : r;
}

// Forward token part (lanes = steps t, walked = steps s < t):
//   O[b,t,h,:] = sum_{s<t} (sum_i q_t[i] e_k[x_s][i] G[t-s][i]) e_v[x_s].
template <int HD>
__global__ void __launch_bounds__(64 * kTW)
fac_tok_fwd_kernel(const float* __restrict__ Q, const int64_t* __restrict__ x, int64_t V,
                   const float* __restrict__ Ek, const float* __restrict__ Ev,
                   const float* __restrict__ G, int L, int H, float* __restrict__ O) {
    constexpr int RS = TokLds<HD>::RS;
    __shared__ __align__(16) float lds[tok_lds_floats<HD>()];
    const int64_t D = (int64_t)H * HD;
    const int b = blockIdx.z, h = blockIdx.y, tb = blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = tb * 64 + lane;
    const bool tv = t < L;
    const int64_t* xb = x + (int64_t)b * L;
    float q[HD], o[HD];
#pragma unroll
    for (int k = 0; k < HD; ++k) {
        q[k] = tv ? Q[((int64_t)b * L + t) * D + h * HD + k] : 0.0f;
        o[k] = 0.0f;
    }
    float* sk = lds + TokLds<HD>::GROWS * RS;  // e_k rows of the walked block
    float* sv = sk + 64 * RS;                   // e_v rows
    for (int sb = 0; sb <= tb; ++sb) {
        const int dlo = (tb - sb) * 64 - 63;
        __syncthreads();
        stage_rows<HD>(lds, G, D, h, dlo, TokLds<HD>::GROWS, L + 1);
        stage_tok_rows<HD>(sk, Ek, xb, V, D, h, sb * 64, 64, L);
        stage_tok_rows<HD>(sv, Ev, xb, V, D, h, sb * 64, 64, L);
        __syncthreads();
        const int s_hi = min(sb * 64 + 64, L);
        for (int s = sb * 64 + w; s < s_hi; s += kTW) {
            const float* ek = sk + (s - sb * 64) * RS;
            const float* ev = sv + (s - sb * 64) * RS;
            const int di = t - s - dlo;
            const bool pair = tv && t > s;
            const float* g = lds + (pair ? di : 0) * RS;
            float a = 0.0f;
#pragma unroll
            for (int k = 0; k < HD; ++k) a = __builtin_fmaf(q[k] * ek[k], g[k], a);
            a = pair ? a : 0.0f;
#pragma unroll
            for (int k = 0; k < HD; ++k) o[k] = __builtin_fmaf(a, ev[k], o[k]);
        }
    }
    reduce_waves<HD>(o, lds);
    if (w == 0 && tv) {
#pragma unroll
        for (int k = 0; k < HD; ++k) O[((int64_t)b * L + t) * D + h * HD + k] = o[k];
    }
}

// Backward by rows (lanes = t, walked = s < t): dQ[b,t,h,:] = sum_{s<t} (dO_t . e_v[x_s])
// e_k[x_s] ⊙ G[t-s].
template <int HD>
__global__ void __launch_bounds__(64 * kTW)
fac_tok_bwd_row_kernel(const float* __restrict__ dO, const int64_t* __restrict__ x, int64_t V,
                       const float* __restrict__ Ek, const float* __restrict__ Ev,
                       const float* __restrict__ G, int L, int H, float* __restrict__ dQ) {
    constexpr int RS = TokLds<HD>::RS;
    __shared__ __align__(16) float lds[tok_lds_floats<HD>()];
    const int64_t D = (int64_t)H * HD;
    const int b = blockIdx.z, h = blockIdx.y, tb = blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = tb * 64 + lane;
    const bool tv = t < L;
    const int64_t* xb = x + (int64_t)b * L;
    float go[HD], dq[HD];
#pragma unroll
    for (int k = 0; k < HD; ++k) {
        go[k] = tv ? dO[((int64_t)b * L + t) * D + h * HD + k] : 0.0f;
        dq[k] = 0.0f;
    }
    float* sk = lds + TokLds<HD>::GROWS * RS;
    float* sv = sk + 64 * RS;
    for (int sb = 0; sb <= tb; ++sb) {
        const int dlo = (tb - sb) * 64 - 63;
        __syncthreads();
        stage_rows<HD>(lds, G, D, h, dlo, TokLds<HD>::GROWS, L + 1);
        stage_tok_rows<HD>(sk, Ek, xb, V, D, h, sb * 64, 64, L);
        stage_tok_rows<HD>(sv, Ev, xb, V, D, h, sb * 64, 64, L);
        __syncthreads();
        const int s_hi = min(sb * 64 + 64, L);
        for (int s = sb * 64 + w; s < s_hi; s += kTW) {
            const float* ek = sk + (s - sb * 64) * RS;
            const float* ev = sv + (s - sb * 64) * RS;
            const int di = t - s - dlo;
            const bool pair = tv && t > s;
            const float* g = lds + (pair ? di : 0) * RS;
            float da = 0.0f;
#pragma unroll
            for (int k = 0; k < HD; ++k) da = __builtin_fmaf(go[k], ev[k], da);
            da = pair ? da : 0.0f;
#pragma unroll
            for (int k = 0; k < HD; ++k) dq[k] = __builtin_fmaf(da * ek[k], g[k], dq[k]);
        }
    }
    reduce_waves<HD>(dq, lds);
    if (w == 0 && tv) {
#pragma unroll
        for (int k = 0; k < HD; ++k) dQ[((int64_t)b * L + t) * D + h * HD + k] = dq[k];
    }
}

// Backward by columns (lanes = s, walked = t > s).  KEY = true: dEk_tok[b,s,h,:] =
// sum_{t>s} (dO_t . e_v[x_s]) q_t ⊙ G[t-s]; KEY = false: dEv_tok[b,s,h,:] =
// sum_{t>s} (sum_i q_t[i] e_k[x_s][i] G[t-s][i]) dO_t.
template <int HD, bool KEY>
__global__ void __launch_bounds__(64 * kTW)
fac_tok_bwd_col_kernel(const float* __restrict__ Q, const float* __restrict__ dO,
                       const int64_t* __restrict__ x, int64_t V, const float* __restrict__ Ek,
                       const float* __restrict__ Ev, const float* __restrict__ G, int L, int H,
                       float* __restrict__ out) {
    constexpr int RS = TokLds<HD>::RS;
    __shared__ __align__(16) float lds[tok_lds_floats<HD>()];
    const int64_t D = (int64_t)H * HD;
    const int b = blockIdx.z, h = blockIdx.y, sb = blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int s = sb * 64 + lane;
    bool sv = s < L;
    const int64_t xs = sv ? x[(int64_t)b * L + s] : 0;
    sv = sv && tok_ok(xs, V);
    const float* E = KEY ? Ev : Ek;  // the row this lane keeps: e_v for dA, e_k for A
    float e[HD], acc[HD];
#pragma unroll
    for (int k = 0; k < HD; ++k) {
        e[k] = sv ? E[xs * D + h * HD + k] : 0.0f;
        acc[k] = 0.0f;
    }
    const int nb = (L + 63) / 64;
    float* sq = lds + TokLds<HD>::GROWS * RS;  // q rows of the walked block
    float* so = sq + 64 * RS;                   // dO rows
    for (int tb = sb; tb < nb; ++tb) {
        const int dlo = (tb - sb) * 64 - 63;
        __syncthreads();
        stage_rows<HD>(lds, G, D, h, dlo, TokLds<HD>::GROWS, L + 1);
        stage_rows<HD>(sq, Q + (int64_t)b * L * D, D, h, tb * 64, 64, L);
        stage_rows<HD>(so, dO + (int64_t)b * L * D, D, h, tb * 64, 64, L);
        __syncthreads();
        const int t_hi = min(tb * 64 + 64, L);
        for (int t = tb * 64 + w; t < t_hi; t += kTW) {
            const float* q = sq + (t - tb * 64) * RS;
            const float* go = so + (t - tb * 64) * RS;
            const int di = t - s - dlo;
            const bool pair = sv && t > s;
            const float* g = lds + (pair ? di : 0) * RS;
            if (KEY) {
                float da = 0.0f;
#pragma unroll
                for (int k = 0; k < HD; ++k) da = __builtin_fmaf(go[k], e[k], da);
                da = pair ? da : 0.0f;
#pragma unroll
                for (int k = 0; k < HD; ++k) acc[k] = __builtin_fmaf(da * q[k], g[k], acc[k]);
            } else {
                float a = 0.0f;
#pragma unroll
                for (int k = 0; k < HD; ++k) a = __builtin_fmaf(q[k] * e[k], g[k], a);
                a = pair ? a : 0.0f;
#pragma unroll
                for (int k = 0; k < HD; ++k) acc[k] = __builtin_fmaf(a, go[k], acc[k]);
            }
        }
    }
    reduce_waves<HD>(acc, lds);
    if (w == 0 && s < L) {
#pragma unroll
        for (int k = 0; k < HD; ++k) out[((int64_t)b * L + s) * D + h * HD + k] = acc[k];
    }
}

// Backward by diagonals (lanes = distances d, walked = t): dGb[b,d,h,:] =
// sum_t (dO_t . e_v[x_{t-d}]) q_t ⊙ e_k[x_{t-d}] for d in [1, L); row 0 is zero.  The e_k /
// e_v rows of the 127 steps t - d a tile needs are staged in LDS.
template <int HD>
__global__ void __launch_bounds__(64 * kTW)
fac_tok_bwd_diag_kernel(const float* __restrict__ Q, const float* __restrict__ dO,
                        const int64_t* __restrict__ x, int64_t V, const float* __restrict__ Ek,
                        const float* __restrict__ Ev, int L, int H, float* __restrict__ dGb) {
    constexpr int RS = TokLds<HD>::RS;
    constexpr int GR = TokLds<HD>::GROWS;
    constexpr int NF = 2 * GR * RS > (kTW - 1) * 64 * HD ? 2 * GR * RS : (kTW - 1) * 64 * HD;
    __shared__ __align__(16) float lds[NF];
    float* sk = lds;
    float* sv = lds + GR * RS;
    const int64_t D = (int64_t)H * HD;
    const int b = blockIdx.z, h = blockIdx.y, db = blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int d = db * 64 + lane;
    const bool dv = d >= 1 && d < L;
    const int64_t* xb = x + (int64_t)b * L;
    float dg[HD];
#pragma unroll
    for (int k = 0; k < HD; ++k) dg[k] = 0.0f;
    const int nb = (L + 63) / 64;
    for (int tb = db; tb < nb; ++tb) {
        const int slo = tb * 64 - db * 64 - 63;  // s = t - d spans [slo, slo + 126]
        __syncthreads();
        stage_tok_rows<HD>(sk, Ek, xb, V, D, h, slo, GR, L);
        stage_tok_rows<HD>(sv, Ev, xb, V, D, h, slo, GR, L);
        __syncthreads();
        const int t_hi = min(tb * 64 + 64, L);
        for (int t = tb * 64 + w; t < t_hi; t += kTW) {
            // the walked rows come from global memory here: staging them too (104 KB of LDS)
            // leaves one block per CU and measured slower
            const float* q = Q + ((int64_t)b * L + t) * D + h * HD;
            const float* go = dO + ((int64_t)b * L + t) * D + h * HD;
            const int si = t - d - slo;
            const bool pair = dv && t - d >= 0;
            const float* ekr = sk + (pair ? si : 0) * RS;
            const float* evr = sv + (pair ? si : 0) * RS;
            float da = 0.0f;
#pragma unroll
            for (int k = 0; k < HD; ++k) da = __builtin_fmaf(go[k], evr[k], da);
            da = pair ? da : 0.0f;
#pragma unroll
            for (int k = 0; k < HD; ++k) dg[k] = __builtin_fmaf(da * q[k], ekr[k], dg[k]);
        }
    }
    reduce_waves<HD>(dg, lds);
    if (w == 0 && d < L) {
#pragma unroll
        for (int k = 0; k < HD; ++k) dGb[((int64_t)b * L + d) * D + h * HD + k] = dv ? dg[k] : 0.0f;
    }
}

int check_hd(int hd, const char* what) {
    if (hd != 32 && hd != 64)
        return fail(MB_ERR_UNSUPPORTED, "%s: head_dim=%d (supported: 32, 64)", what, hd);
    return MB_OK;
}

}  // namespace
}  // namespace mb

using namespace mb;

extern "C" int mb_factored_outer(const float* X, const int64_t* xrow, const float* Y,
                                 const int64_t* yrow, int64_t ld, int64_t nrows, const float* alpha,
                                 int64_t as_b, int64_t as_r, int64_t as_n, int B, int R, int H,
                                 int N, int hd, float* out, void* stream) {
    MB_REQUIRE(B >= 0 && R >= 0 && H >= 1 && N >= 1 && nrows >= 0,
               "mb_factored_outer: bad sizes B=%d R=%d H=%d N=%d", B, R, H, N);
    if (int rc = check_hd(hd, "mb_factored_outer")) return rc;
    MB_REQUIRE(ld >= (int64_t)H * hd, "mb_factored_outer: row stride %lld < H*hd", (long long)ld);
    if (B == 0) return MB_OK;
    MB_REQUIRE(X && Y && alpha && out, "mb_factored_outer: null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    const dim3 blk(256);
    if (hd == 64) {
        hipLaunchKernelGGL(fac_outer_mfma_kernel, dim3((N + 3) / 4, H, B), blk, 0, st, X, xrow, Y,
                           yrow, ld, nrows, alpha, as_b, as_r, as_n, R, H, N, out);
    } else {
        hipLaunchKernelGGL(fac_outer_kernel<32>, dim3((N + 7) / 8, H, B), blk, 0, st, X, xrow, Y,
                           yrow, ld, nrows, alpha, as_b, as_r, as_n, R, H, N, out);
    }
    return check_launch("mb_factored_outer");
}

extern "C" int mb_factored_apply(const float* M, const float* w, int64_t ldw, const float* Y,
                                 const int64_t* yrow, int64_t ld, int64_t nrows, const float* alpha,
                                 int64_t as_b, int64_t as_r, int64_t as_n, int B, int R, int H,
                                 int N, int hd, int transpose, float* out, int64_t ldo,
                                 int accumulate, void* stream) {
    MB_REQUIRE(B >= 0 && R >= 0 && H >= 1 && N >= 1 && nrows >= 0,
               "mb_factored_apply: bad sizes B=%d R=%d H=%d N=%d", B, R, H, N);
    if (int rc = check_hd(hd, "mb_factored_apply")) return rc;
    MB_REQUIRE(ld >= (int64_t)H * hd && ldo >= (int64_t)H * hd,
               "mb_factored_apply: row strides must be >= H*hd");
    if (B == 0 || R == 0) return MB_OK;
    MB_REQUIRE(M && Y && alpha && out, "mb_factored_apply: null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((R + kApplyRows - 1) / kApplyRows, H, B), blk(256);
#define MB_FAC_APPLY(HDV, TR)                                                                     \
    hipLaunchKernelGGL((fac_apply_kernel<HDV, TR>), grid, blk, 0, st, M, w, ldw, Y, yrow, ld, nrows, \
                       alpha, as_b, as_r, as_n, R, H, N, out, ldo, accumulate)
    if (hd == 64) {
        const dim3 g64((R + 63) / 64, H, B);
        if (transpose)
            hipLaunchKernelGGL(fac_apply_mfma_kernel<true>, g64, blk, 0, st, M, w, ldw, Y, yrow, ld,
                               nrows, alpha, as_b, as_r, as_n, R, H, N, out, ldo, accumulate);
        else
            hipLaunchKernelGGL(fac_apply_mfma_kernel<false>, g64, blk, 0, st, M, w, ldw, Y, yrow, ld,
                               nrows, alpha, as_b, as_r, as_n, R, H, N, out, ldo, accumulate);
    } else {
        if (transpose) MB_FAC_APPLY(32, true); else MB_FAC_APPLY(32, false);
    }
#undef MB_FAC_APPLY
    return check_launch("mb_factored_apply");
}

extern "C" int mb_factored_tok_fwd(const float* Q, const int64_t* x, int64_t V, const float* E_k,
                                   const float* E_v, const float* G, int B, int L, int H, int hd,
                                   float* O, void* stream) {
    MB_REQUIRE(B >= 0 && L >= 0 && H >= 1 && V >= 1, "mb_factored_tok_fwd: bad sizes");
    if (int rc = check_hd(hd, "mb_factored_tok_fwd")) return rc;
    if (B == 0 || L == 0) return MB_OK;
    MB_REQUIRE(Q && x && E_k && E_v && G && O, "mb_factored_tok_fwd: null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((L + 63) / 64, H, B), blk(64 * kTW);
    if (hd == 64)
        hipLaunchKernelGGL(fac_tok_fwd_kernel<64>, grid, blk, 0, st, Q, x, V, E_k, E_v, G, L, H, O);
    else
        hipLaunchKernelGGL(fac_tok_fwd_kernel<32>, grid, blk, 0, st, Q, x, V, E_k, E_v, G, L, H, O);
    return check_launch("mb_factored_tok_fwd");
}

extern "C" int mb_factored_tok_bwd(const float* Q, const float* dO, const int64_t* x, int64_t V,
                                   const float* E_k, const float* E_v, const float* G, int B, int L,
                                   int H, int hd, float* dQ, float* dEk_tok, float* dEv_tok,
                                   float* dG_b, void* stream) {
    MB_REQUIRE(B >= 0 && L >= 0 && H >= 1 && V >= 1, "mb_factored_tok_bwd: bad sizes");
    if (int rc = check_hd(hd, "mb_factored_tok_bwd")) return rc;
    if (B == 0 || L == 0) return MB_OK;
    MB_REQUIRE(Q && dO && x && E_k && E_v && G && dQ && dEk_tok && dEv_tok && dG_b,
               "mb_factored_tok_bwd: null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((L + 63) / 64, H, B), blk(64 * kTW);
#define MB_FAC_BWD(HDV)                                                                           \
    do {                                                                                          \
        hipLaunchKernelGGL(fac_tok_bwd_row_kernel<HDV>, grid, blk, 0, st, dO, x, V, E_k, E_v, G, L, \
                           H, dQ);                                                                \
        hipLaunchKernelGGL((fac_tok_bwd_col_kernel<HDV, true>), grid, blk, 0, st, Q, dO, x, V, E_k, \
                           E_v, G, L, H, dEk_tok);                                                \
        hipLaunchKernelGGL((fac_tok_bwd_col_kernel<HDV, false>), grid, blk, 0, st, Q, dO, x, V,     \
                           E_k, E_v, G, L, H, dEv_tok);                                           \
        hipLaunchKernelGGL(fac_tok_bwd_diag_kernel<HDV>, grid, blk, 0, st, Q, dO, x, V, E_k, E_v, L, \
                           H, dG_b);                                                              \
    } while (0)
    if (hd == 64) MB_FAC_BWD(64);
    else MB_FAC_BWD(32);
#undef MB_FAC_BWD
    return check_launch("mb_factored_tok_bwd");
}
