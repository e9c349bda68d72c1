// Factored linear EMA (mathbrain/factored_ema.py:22-146) on gfx950, fp32.
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
#include "common.h"

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
// (w NULL: 1).  Block (64 rows, h, b); thread (row, quarter of the outputs); M_n is staged
// in LDS once per rate for the 64 rows.
template <int HD, bool TRANS>
__global__ void __launch_bounds__(256)
fac_apply_kernel(const float* __restrict__ M, const float* __restrict__ w, int64_t ldw,
                 const float* __restrict__ Y, const int64_t* __restrict__ yrow, int64_t ld,
                 int64_t nrows, const float* __restrict__ alpha, int64_t as_b, int64_t as_r,
                 int64_t as_n, int R, int H, int N, float* __restrict__ out, int64_t ldo,
                 int accumulate) {
    constexpr int QP = HD / 4;
    __shared__ float Ms[HD][HD + 1];
    const int b = blockIdx.z, h = blockIdx.y;
    const int r = blockIdx.x * 64 + threadIdx.x / 4;
    const int part = threadIdx.x % 4;
    const bool rok = r < R;
    int64_t ry = -1;
    if (rok) ry = clamp_row(yrow, (int64_t)b * R + r, nrows);
    float y[HD];
#pragma unroll
    for (int k = 0; k < HD; ++k) y[k] = ry >= 0 ? Y[ry * ld + h * HD + k] : 0.0f;
    float acc[QP];
#pragma unroll
    for (int o = 0; o < QP; ++o) acc[o] = 0.0f;
    for (int n = 0; n < N; ++n) {
        __syncthreads();
        const float* Mn = M + (((int64_t)b * H + h) * N + n) * HD * HD;
        for (int e = threadIdx.x; e < HD * HD; e += 256) {
            const int i = e / HD, j = e % HD;
            float v = Mn[e];
            if (w) v *= w[n * ldw + h * HD + i];
            if (TRANS) Ms[j][i] = v;
            else Ms[i][j] = v;
        }
        __syncthreads();
        const float a = rok ? alpha[b * as_b + r * as_r + n * as_n] : 0.0f;
#pragma unroll
        for (int o = 0; o < QP; ++o) {
            const float* row = Ms[part * QP + o];
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < HD; ++k) s = __builtin_fmaf(row[k], y[k], s);
            acc[o] = __builtin_fmaf(a, s, acc[o]);
        }
    }
    if (rok) {
        float* dst = out + ((int64_t)b * R + r) * ldo + h * HD + part * QP;
#pragma unroll
        for (int o = 0; o < QP; ++o) dst[o] = accumulate ? dst[o] + acc[o] : acc[o];
    }
}

// Reduction over the four lanes that hold the quarters of one row.
__device__ inline float quad_sum(float a) {
    a += __shfl_xor(a, 1, 64);
    a += __shfl_xor(a, 2, 64);
    return a;
}

__device__ inline bool tok_ok(int64_t v, int64_t V) { return v >= 0 && v < V; }

// Token part of the forward: O[b,t,h,:] = sum_{s<t} A[t,s] ev_s.  Block (64 steps, h, b);
// thread (t, quarter): q_t and o_t quarters in registers, e_k / e_v rows of step s shared
// by the block, G[t-s] per thread.
template <int HD>
__global__ void __launch_bounds__(256)
fac_tok_fwd_kernel(const float* __restrict__ Q, const int64_t* __restrict__ x, int64_t V,
                   const float* __restrict__ Ek, const float* __restrict__ Ev,
                   const float* __restrict__ G, int L, int H, float* __restrict__ O) {
    constexpr int QP = HD / 4;
    const int64_t D = (int64_t)H * HD;
    const int b = blockIdx.z, h = blockIdx.y;
    const int t = blockIdx.x * 64 + threadIdx.x / 4;
    const int part = threadIdx.x % 4;
    const int off = h * HD + part * QP;
    const bool tv = t < L;
    float q[QP], o[QP];
#pragma unroll
    for (int k = 0; k < QP; ++k) {
        q[k] = tv ? Q[((int64_t)b * L + t) * D + off + k] : 0.0f;
        o[k] = 0.0f;
    }
    const int t_hi = min(L, blockIdx.x * 64 + 64);  // s < t < t_hi
    for (int s = 0; s < t_hi - 1; ++s) {
        const int64_t xs = x[(int64_t)b * L + s];
        if (!tok_ok(xs, V)) continue;
        const float* ek = Ek + xs * D + off;
        const float* ev = Ev + xs * D + off;
        float a = 0.0f;
        if (tv && t > s) {
            const float* g = G + (int64_t)(t - s) * D + off;
#pragma unroll
            for (int k = 0; k < QP; ++k) a = __builtin_fmaf(q[k] * ek[k], g[k], a);
        }
        a = quad_sum(a);
#pragma unroll
        for (int k = 0; k < QP; ++k) o[k] = __builtin_fmaf(a, ev[k], o[k]);
    }
    if (tv) {
#pragma unroll
        for (int k = 0; k < QP; ++k) O[((int64_t)b * L + t) * D + off + k] = o[k];
    }
}

// Backward by rows: dQ[b,t,h,i] = sum_{s<t} dA[t,s] ek_s[i] G[t-s][i], dA = dO_t . ev_s.
template <int HD>
__global__ void __launch_bounds__(256)
fac_tok_bwd_row_kernel(const float* __restrict__ dO, const int64_t* __restrict__ x, int64_t V,
                       const float* __restrict__ Ek, const float* __restrict__ Ev,
                       const float* __restrict__ G, int L, int H, float* __restrict__ dQ) {
    constexpr int QP = HD / 4;
    const int64_t D = (int64_t)H * HD;
    const int b = blockIdx.z, h = blockIdx.y;
    const int t = blockIdx.x * 64 + threadIdx.x / 4;
    const int part = threadIdx.x % 4;
    const int off = h * HD + part * QP;
    const bool tv = t < L;
    float g_o[QP], dq[QP];
#pragma unroll
    for (int k = 0; k < QP; ++k) {
        g_o[k] = tv ? dO[((int64_t)b * L + t) * D + off + k] : 0.0f;
        dq[k] = 0.0f;
    }
    const int t_hi = min(L, blockIdx.x * 64 + 64);
    for (int s = 0; s < t_hi - 1; ++s) {
        const int64_t xs = x[(int64_t)b * L + s];
        if (!tok_ok(xs, V)) continue;
        const float* ek = Ek + xs * D + off;
        const float* ev = Ev + xs * D + off;
        float da = 0.0f;
#pragma unroll
        for (int k = 0; k < QP; ++k) da = __builtin_fmaf(g_o[k], ev[k], da);
        da = quad_sum(da);
        if (tv && t > s) {
            const float* g = G + (int64_t)(t - s) * D + off;
#pragma unroll
            for (int k = 0; k < QP; ++k) dq[k] = __builtin_fmaf(da * ek[k], g[k], dq[k]);
        }
    }
    if (tv) {
#pragma unroll
        for (int k = 0; k < QP; ++k) dQ[((int64_t)b * L + t) * D + off + k] = dq[k];
    }
}

// Backward by columns: for step s, dEk_tok[b,s,h,i] = sum_{t>s} dA[t,s] q_t[i] G[t-s][i] and
// dEv_tok[b,s,h,j] = sum_{t>s} A[t,s] dO_t[j].
template <int HD>
__global__ void __launch_bounds__(256)
fac_tok_bwd_col_kernel(const float* __restrict__ Q, const float* __restrict__ dO,
                       const int64_t* __restrict__ x, int64_t V, const float* __restrict__ Ek,
                       const float* __restrict__ Ev, const float* __restrict__ G, int L, int H,
                       float* __restrict__ dEk, float* __restrict__ dEv) {
    constexpr int QP = HD / 4;
    const int64_t D = (int64_t)H * HD;
    const int b = blockIdx.z, h = blockIdx.y;
    const int s = blockIdx.x * 64 + threadIdx.x / 4;
    const int part = threadIdx.x % 4;
    const int off = h * HD + part * QP;
    bool sv = s < L;
    int64_t xs = sv ? x[(int64_t)b * L + s] : 0;
    sv = sv && tok_ok(xs, V);
    float ek[QP], ev[QP], dek[QP], dev[QP];
#pragma unroll
    for (int k = 0; k < QP; ++k) {
        ek[k] = sv ? Ek[xs * D + off + k] : 0.0f;
        ev[k] = sv ? Ev[xs * D + off + k] : 0.0f;
        dek[k] = dev[k] = 0.0f;
    }
    for (int t = blockIdx.x * 64 + 1; t < L; ++t) {
        const float* q = Q + ((int64_t)b * L + t) * D + off;
        const float* go = dO + ((int64_t)b * L + t) * D + off;
        const bool pair = sv && t > s;
        float gv[QP];
        const float* g = G + (int64_t)(pair ? t - s : 0) * D + off;
#pragma unroll
        for (int k = 0; k < QP; ++k) gv[k] = pair ? g[k] : 0.0f;
        float a = 0.0f, da = 0.0f;
#pragma unroll
        for (int k = 0; k < QP; ++k) {
            a = __builtin_fmaf(q[k] * ek[k], gv[k], a);
            da = __builtin_fmaf(go[k], ev[k], da);
        }
        a = quad_sum(a);
        da = quad_sum(da);
        if (pair) {
#pragma unroll
            for (int k = 0; k < QP; ++k) {
                dev[k] = __builtin_fmaf(a, go[k], dev[k]);
                dek[k] = __builtin_fmaf(da * q[k], gv[k], dek[k]);
            }
        }
    }
    if (s < L) {
#pragma unroll
        for (int k = 0; k < QP; ++k) {
            dEk[((int64_t)b * L + s) * D + off + k] = dek[k];
            dEv[((int64_t)b * L + s) * D + off + k] = dev[k];
        }
    }
}

// Backward by diagonals: dGb[b,d,h,i] = sum_t dA[t,t-d] q_t[i] ek_{t-d}[i] for d in [1, L);
// row 0 is zero.  Thread (d, quarter); each thread gathers its own e_k / e_v rows.
template <int HD>
__global__ void __launch_bounds__(256)
fac_tok_bwd_diag_kernel(const float* __restrict__ Q, const float* __restrict__ dO,
                        const int64_t* __restrict__ x, int64_t V, const float* __restrict__ Ek,
                        const float* __restrict__ Ev, int L, int H, float* __restrict__ dGb) {
    constexpr int QP = HD / 4;
    const int64_t D = (int64_t)H * HD;
    const int b = blockIdx.z, h = blockIdx.y;
    const int d = blockIdx.x * 64 + threadIdx.x / 4;
    const int part = threadIdx.x % 4;
    const int off = h * HD + part * QP;
    float dg[QP];
#pragma unroll
    for (int k = 0; k < QP; ++k) dg[k] = 0.0f;
    for (int t = blockIdx.x * 64; t < L; ++t) {
        const int s = t - d;
        const bool pair = d >= 1 && d < L && s >= 0;
        int64_t xs = pair ? x[(int64_t)b * L + s] : 0;
        const bool ok = pair && tok_ok(xs, V);
        const float* q = Q + ((int64_t)b * L + t) * D + off;
        const float* go = dO + ((int64_t)b * L + t) * D + off;
        float ek[QP], ev[QP];
#pragma unroll
        for (int k = 0; k < QP; ++k) {
            ek[k] = ok ? Ek[xs * D + off + k] : 0.0f;
            ev[k] = ok ? Ev[xs * D + off + k] : 0.0f;
        }
        float da = 0.0f;
#pragma unroll
        for (int k = 0; k < QP; ++k) da = __builtin_fmaf(go[k], ev[k], da);
        da = quad_sum(da);
#pragma unroll
        for (int k = 0; k < QP; ++k) dg[k] = __builtin_fmaf(da * q[k], ek[k], dg[k]);
    }
    if (d < L) {
#pragma unroll
        for (int k = 0; k < QP; ++k) dGb[((int64_t)b * L + d) * D + off + k] = d >= 1 ? dg[k] : 0.0f;
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
        hipLaunchKernelGGL(fac_outer_kernel<64>, dim3((N + 3) / 4, H, B), blk, 0, st, X, xrow, Y,
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
    const dim3 grid((R + 63) / 64, H, B), blk(256);
#define MB_FAC_APPLY(HDV, TR)                                                                     \
    hipLaunchKernelGGL((fac_apply_kernel<HDV, TR>), grid, blk, 0, st, M, w, ldw, Y, yrow, ld, nrows, \
                       alpha, as_b, as_r, as_n, R, H, N, out, ldo, accumulate)
    if (hd == 64) {
        if (transpose) MB_FAC_APPLY(64, true); else MB_FAC_APPLY(64, false);
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
    const dim3 grid((L + 63) / 64, H, B), blk(256);
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
    const dim3 grid((L + 63) / 64, H, B), blk(256);
    if (hd == 64) {
        hipLaunchKernelGGL(fac_tok_bwd_row_kernel<64>, grid, blk, 0, st, dO, x, V, E_k, E_v, G, L, H, dQ);
        hipLaunchKernelGGL(fac_tok_bwd_col_kernel<64>, grid, blk, 0, st, Q, dO, x, V, E_k, E_v, G, L,
                           H, dEk_tok, dEv_tok);
        hipLaunchKernelGGL(fac_tok_bwd_diag_kernel<64>, grid, blk, 0, st, Q, dO, x, V, E_k, E_v, L, H,
                           dG_b);
    } else {
        hipLaunchKernelGGL(fac_tok_bwd_row_kernel<32>, grid, blk, 0, st, dO, x, V, E_k, E_v, G, L, H, dQ);
        hipLaunchKernelGGL(fac_tok_bwd_col_kernel<32>, grid, blk, 0, st, Q, dO, x, V, E_k, E_v, G, L,
                           H, dEk_tok, dEv_tok);
        hipLaunchKernelGGL(fac_tok_bwd_diag_kernel<32>, grid, blk, 0, st, Q, dO, x, V, E_k, E_v, L, H,
                           dG_b);
    }
    return check_launch("mb_factored_tok_bwd");
}
