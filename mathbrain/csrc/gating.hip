// Fused symmetric query gating on gfx950: forward and backward row kernels.
//
// Replaces _fused_gating_fwd / _fused_gating_bwd and FusedGatingFunction
// (mathbrain/triton_fused_gating.py:12-57, :61-119, :122-177).  Per row r (one (b, t)
// position) and column d:
//   pre[r,d]  = p_pre[r,d] + bias[d]                         (FusedGatingFunction form)
//             = sum_n (C_seq[r,n] + 1) W_pe[n,d]             (projection folded in; this is
//               pe_proj(C_seq) + pe_proj.weight.sum(1), triton_fused_gating.py:180-183)
//   g         = SiLU(pre)  (or pre for the linear gate)
//   x_emb     = x_q * g
//   y         = LayerNorm_eps(x_emb) * ln_w + ln_b
// The backward is the reference's closed form (:95-118): with x_hat = (x_emb - mu) rstd,
//   dx_hat = dy ln_w,  dx_emb = (dx_hat - mean(dx_hat) - x_hat mean(dx_hat x_hat)) rstd
//   dx_q = dx_emb g,   dp_pre = dx_emb x_q SiLU'(pre)
// and the column sums dln_w = sum_r dy x_hat, dln_b = sum_r dy, dbias = sum_r dp_pre
// (the reference writes [rows, D] partials and reduces them with torch, :159-160,
// :173-175; here each workgroup reduces its rows in registers and adds once).
//
// Layout: a workgroup of 256 threads owns a tile of kRows rows; thread i owns columns
// i, i + 256, ... (coalesced row reads and writes).  The per-element work runs
// column-parallel, the LayerNorm row statistics one wave per row over a copy of the
// tile in LDS.  x_emb and the gate are recomputed in the backward instead of being
// stored (the reference saves x_emb and p_gate, two more [rows, D] tensors).
#include "common.h"

#include <algorithm>

namespace mb {

constexpr int kGateThreads = 256;
constexpr int kGateRows = 8;

struct GateArgs {
    const float* xq;
    int64_t xq_sr;  // row stride of x_q (elements); columns contiguous
    const float* pp;
    int64_t pp_sr;
    const float* bias;
    const float* C;
    int64_t c_sr;
    const float* W;  // [N, D]
    int N;
    const float* lnw;
    const float* lnb;
    int64_t rows;
    int D;
    float eps;
    float* y;
    float* mu;
    float* rstd;
    float* pre_out;  // optional [rows, D]: the forward's pre-activation, kept for the backward
    // backward
    const float* dy;
    float* dxq;
    float* dpp;
    float* dbias;
    float* dlnw;
    float* dlnb;
};

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Gate pre-activation of rows r0 .. r0 + kGateRows - 1 at column col.  `cst` holds
// (C_seq + 1) transposed, [N][kGateRows], for the folded projection.
// Pre-activations of all CPT columns of this thread for the tile's rows, one pass over the
// rates: each rate's eight staged counts are read once for all columns.
template <bool FUSED, int CPT>
__device__ inline void gate_pre_all(const GateArgs& a, int64_t r0, int nr, int tid, const float* cst,
                                    float (&pre)[CPT][kGateRows]) {
    if (FUSED) {
#pragma unroll
        for (int j = 0; j < CPT; ++j)
#pragma unroll
            for (int r = 0; r < kGateRows; ++r) pre[j][r] = 0.f;
#pragma unroll 8
        for (int n = 0; n < a.N; ++n) {
            const float4 c0 = *reinterpret_cast<const float4*>(cst + n * kGateRows);
            const float4 c1 = *reinterpret_cast<const float4*>(cst + n * kGateRows + 4);
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                const int col = tid + j * kGateThreads;
                const float w = col < a.D ? a.W[(int64_t)n * a.D + col] : 0.f;
                pre[j][0] = __builtin_fmaf(c0.x, w, pre[j][0]);
                pre[j][1] = __builtin_fmaf(c0.y, w, pre[j][1]);
                pre[j][2] = __builtin_fmaf(c0.z, w, pre[j][2]);
                pre[j][3] = __builtin_fmaf(c0.w, w, pre[j][3]);
                pre[j][4] = __builtin_fmaf(c1.x, w, pre[j][4]);
                pre[j][5] = __builtin_fmaf(c1.y, w, pre[j][5]);
                pre[j][6] = __builtin_fmaf(c1.z, w, pre[j][6]);
                pre[j][7] = __builtin_fmaf(c1.w, w, pre[j][7]);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int col = tid + j * kGateThreads;
            const float bv = col < a.D && a.bias ? a.bias[col] : 0.f;
#pragma unroll
            for (int r = 0; r < kGateRows; ++r)
                pre[j][r] = (r < nr && col < a.D) ? a.pp[(r0 + r) * a.pp_sr + col] + bv : 0.f;
        }
    }
}

__device__ inline float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Stages (C_seq + 1)^T of the tile: cst[n][r].
__device__ inline void stage_counts(const GateArgs& a, int64_t r0, int nr, float* cst) {
    for (int i = threadIdx.x; i < kGateRows * a.N; i += blockDim.x) {
        const int r = i / a.N;
        const int n = i % a.N;
        cst[n * kGateRows + r] = r < nr ? a.C[(r0 + r) * a.c_sr + n] + 1.0f : 0.f;
    }
}

template <int CPT, bool FUSED, bool SILU>
__global__ void __launch_bounds__(kGateThreads)
gating_fwd_kernel(GateArgs a) {
    extern __shared__ __align__(16) float gsm[];
    float* xe = gsm;                          // [kGateRows][D]
    float* stats = xe + kGateRows * a.D;      // [kGateRows][2]
    float* cst = stats + 2 * kGateRows;       // [N][kGateRows]
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int64_t ntiles = (a.rows + kGateRows - 1) / kGateRows;
    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t r0 = tile * kGateRows;
        const int nr = (int)std::min<int64_t>(kGateRows, a.rows - r0);
        // the tile's x_q values are requested first, so that their latency overlaps the
        // staging and the gate sums
        float xv[CPT][kGateRows];
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int col = tid + j * kGateThreads;
#pragma unroll
            for (int r = 0; r < kGateRows; ++r)
                xv[j][r] = (col < a.D && r < nr) ? a.xq[(r0 + r) * a.xq_sr + col] : 0.f;
        }
        if (FUSED) {
            stage_counts(a, r0, nr, cst);
            __syncthreads();
        }
        float pre[CPT][kGateRows];
        gate_pre_all<FUSED, CPT>(a, r0, nr, tid, cst, pre);
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int col = tid + j * kGateThreads;
            if (col >= a.D) break;
#pragma unroll
            for (int r = 0; r < kGateRows; ++r) {
                if (r >= nr) break;
                if (a.pre_out) a.pre_out[(r0 + r) * a.D + col] = pre[j][r];
                const float g = SILU ? pre[j][r] * sigmoidf_(pre[j][r]) : pre[j][r];
                xe[r * a.D + col] = xv[j][r] * g;
            }
        }
        __syncthreads();
        for (int r = wave; r < nr; r += kGateThreads / 64) {
            float s = 0.f;
            for (int c = lane; c < a.D; c += 64) s += xe[r * a.D + c];
            const float mean = wave_sum(s) / (float)a.D;
            float v = 0.f;
            for (int c = lane; c < a.D; c += 64) {
                const float dd = xe[r * a.D + c] - mean;
                v = __builtin_fmaf(dd, dd, v);
            }
            const float var = wave_sum(v) / (float)a.D;
            const float rs = 1.0f / sqrtf(var + a.eps);
            if (lane == 0) {
                stats[2 * r] = mean;
                stats[2 * r + 1] = rs;
                a.mu[r0 + r] = mean;
                a.rstd[r0 + r] = rs;
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int col = tid + j * kGateThreads;
            if (col >= a.D) break;
            const float w = a.lnw[col];
            const float bb = a.lnb[col];
            for (int r = 0; r < nr; ++r)
                a.y[(r0 + r) * a.D + col] = (xe[r * a.D + col] - stats[2 * r]) * stats[2 * r + 1] * w + bb;
        }
        __syncthreads();
    }
}

template <int CPT, bool FUSED, bool SILU>
__global__ void __launch_bounds__(kGateThreads)
gating_bwd_kernel(GateArgs a) {
    extern __shared__ __align__(16) float gsm[];
    float* xh = gsm;                           // [kGateRows][D]  x_hat
    float* dxh = xh + kGateRows * a.D;         // [kGateRows][D]  dy * ln_w
    float* stats = dxh + kGateRows * a.D;      // [kGateRows][2]  c1, c2
    float* cst = stats + 2 * kGateRows;        // [N][kGateRows]
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    float acc_w[CPT], acc_b[CPT], acc_p[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) acc_w[j] = acc_b[j] = acc_p[j] = 0.f;
    const int64_t ntiles = (a.rows + kGateRows - 1) / kGateRows;
    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t r0 = tile * kGateRows;
        const int nr = (int)std::min<int64_t>(kGateRows, a.rows - r0);
        // this tile's inputs are requested first (their latency overlaps the gate sums)
        float xv[CPT][kGateRows], dyv_[CPT][kGateRows], muv[kGateRows], rsv[kGateRows];
#pragma unroll
        for (int r = 0; r < kGateRows; ++r) {
            muv[r] = r < nr ? a.mu[r0 + r] : 0.f;
            rsv[r] = r < nr ? a.rstd[r0 + r] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int col = tid + j * kGateThreads;
#pragma unroll
            for (int r = 0; r < kGateRows; ++r) {
                const bool ok = col < a.D && r < nr;
                xv[j][r] = ok ? a.xq[(r0 + r) * a.xq_sr + col] : 0.f;
                dyv_[j][r] = ok ? a.dy[(r0 + r) * a.D + col] : 0.f;
            }
        }
        if (FUSED) {
            stage_counts(a, r0, nr, cst);
            __syncthreads();
        }
        float gv[CPT][kGateRows], ds[CPT][kGateRows];
        float pre_all[CPT][kGateRows];
        gate_pre_all<FUSED, CPT>(a, r0, nr, tid, cst, pre_all);
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int col = tid + j * kGateThreads;
            if (col >= a.D) break;
            const float* pre = pre_all[j];
            const float w = a.lnw[col];
#pragma unroll
            for (int r = 0; r < kGateRows; ++r) {
                if (r >= nr) break;
                float g = pre[r], dsil = 1.f;
                if (SILU) {
                    const float sg = sigmoidf_(pre[r]);
                    g = pre[r] * sg;
                    dsil = g + sg * (1.0f - g);  // SiLU' (triton_fused_gating.py:113-114)
                }
                gv[j][r] = g;
                ds[j][r] = dsil;
                const float x = xv[j][r];
                const float dyv = dyv_[j][r];
                const float xhat = (x * g - muv[r]) * rsv[r];
                xh[r * a.D + col] = xhat;
                dxh[r * a.D + col] = dyv * w;
                acc_w[j] = __builtin_fmaf(dyv, xhat, acc_w[j]);
                acc_b[j] += dyv;
            }
        }
        __syncthreads();
        for (int r = wave; r < nr; r += kGateThreads / 64) {
            float s1 = 0.f, s2 = 0.f;
            for (int c = lane; c < a.D; c += 64) {
                const float v = dxh[r * a.D + c];
                s1 += v;
                s2 = __builtin_fmaf(v, xh[r * a.D + c], s2);
            }
            s1 = wave_sum(s1);
            s2 = wave_sum(s2);
            if (lane == 0) {
                stats[2 * r] = s1 / (float)a.D;
                stats[2 * r + 1] = s2 / (float)a.D;
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int col = tid + j * kGateThreads;
            if (col >= a.D) break;
#pragma unroll
            for (int r = 0; r < kGateRows; ++r) {
                if (r >= nr) break;
                const float dxe = (dxh[r * a.D + col] - stats[2 * r] - xh[r * a.D + col] * stats[2 * r + 1]) *
                                  rsv[r];
                const float x = xv[j][r];
                a.dxq[(r0 + r) * a.D + col] = dxe * gv[j][r];
                const float dp = dxe * x * ds[j][r];
                a.dpp[(r0 + r) * a.D + col] = dp;
                acc_p[j] += dp;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int col = tid + j * kGateThreads;
        if (col >= a.D) break;
        atomicAdd(&a.dlnw[col], acc_w[j]);
        atomicAdd(&a.dlnb[col], acc_b[j]);
        atomicAdd(&a.dbias[col], acc_p[j]);
    }
}

// Forward with the projection folded in, R rows per wave: lane l owns columns 4 l + 256 q + e
// of every row of the wave's tile, so the LayerNorm row sums are wave reductions (no LDS
// pass, no barrier) and every load and store is a coalesced float4.  The tile's (C_seq + 1)
// rows sit in the wave's own LDS area, read back as broadcasts; each W_pe row a lane needs
// is loaded once per tile (from L2) and applied to all R rows, R times fewer W reads per row
// than one row at a time.
template <int Q4, bool SILU, int R>
__global__ void __launch_bounds__(kGateThreads)
gating_fwd_rows_kernel(GateArgs a) {
    extern __shared__ __align__(16) float rsm[];  // [wave][R][NP]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    constexpr int NW = kGateThreads / 64;
    const int D = a.D;
    const int N = a.N;
    const int NP = (N + 3) & ~3;
    float* mc = rsm + wave * R * NP;
    float4 lnw4[Q4], lnb4[Q4];
#pragma unroll
    for (int q = 0; q < Q4; ++q) {
        lnw4[q] = *reinterpret_cast<const float4*>(a.lnw + 4 * lane + 256 * q);
        lnb4[q] = *reinterpret_cast<const float4*>(a.lnb + 4 * lane + 256 * q);
    }
    const int64_t ntiles = (a.rows + R - 1) / R;
    for (int64_t tile = (int64_t)blockIdx.x * NW + wave; tile < ntiles; tile += (int64_t)gridDim.x * NW) {
        const int64_t r0 = tile * R;
        const int nr = (int)std::min<int64_t>(R, a.rows - r0);
        // every lane is done reading the previous tile's counts
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        for (int i = lane; i < R * NP; i += 64) {
            const int r = i / NP, n = i % NP;
            mc[i] = (r < nr && n < N) ? a.C[(r0 + r) * a.c_sr + n] + 1.0f : 0.f;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float4 pre[R][Q4];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int q = 0; q < Q4; ++q) pre[r][q] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 2
        for (int n = 0; n < NP; n += 4) {
            float4 w[4][Q4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int q = 0; q < Q4; ++q)
                    w[k][q] = n + k < N ? *reinterpret_cast<const float4*>(a.W + (int64_t)(n + k) * D + 4 * lane + 256 * q)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float4 cv = *reinterpret_cast<const float4*>(mc + r * NP + n);
                const float cc[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
                for (int k = 0; k < 4; ++k)
#pragma unroll
                    for (int q = 0; q < Q4; ++q) {
                        pre[r][q].x = __builtin_fmaf(cc[k], w[k][q].x, pre[r][q].x);
                        pre[r][q].y = __builtin_fmaf(cc[k], w[k][q].y, pre[r][q].y);
                        pre[r][q].z = __builtin_fmaf(cc[k], w[k][q].z, pre[r][q].z);
                        pre[r][q].w = __builtin_fmaf(cc[k], w[k][q].w, pre[r][q].w);
                    }
            }
        }
        float4 xv[Q4];
        auto load_x = [&](int r) {
#pragma unroll
            for (int q = 0; q < Q4; ++q)
                xv[q] = *reinterpret_cast<const float4*>(a.xq + (r0 + r) * a.xq_sr + 4 * lane + 256 * q);
        };
        load_x(0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r >= nr) continue;  // (uniform; keeps the loop unrolled, pre[] in registers)
            const int64_t row = r0 + r;
            float xe[Q4][4];
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < Q4; ++q) {
                const float pe[4] = {pre[r][q].x, pre[r][q].y, pre[r][q].z, pre[r][q].w};
                const float xx[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
                if (a.pre_out) st_stream4(a.pre_out + row * D + 4 * lane + 256 * q, pre[r][q]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float g = SILU ? pe[e] * sigmoidf_(pe[e]) : pe[e];
                    xe[q][e] = xx[e] * g;
                    s += xe[q][e];
                }
            }
            if (r + 1 < nr) load_x(r + 1);  // the next row's x_q while this row's sums reduce
            const float mean = wave_sum(s) / (float)D;
            float v = 0.f;
#pragma unroll
            for (int q = 0; q < Q4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float dd = xe[q][e] - mean;
                    v = __builtin_fmaf(dd, dd, v);
                }
            const float rs = 1.0f / sqrtf(wave_sum(v) / (float)D + a.eps);
#pragma unroll
            for (int q = 0; q < Q4; ++q) {
                const float wv[4] = {lnw4[q].x, lnw4[q].y, lnw4[q].z, lnw4[q].w};
                const float bv[4] = {lnb4[q].x, lnb4[q].y, lnb4[q].z, lnb4[q].w};
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = (xe[q][e] - mean) * rs * wv[e] + bv[e];
                st_stream4(a.y + row * D + 4 * lane + 256 * q, make_float4(o[0], o[1], o[2], o[3]));
            }
            if (lane == 0) {
                a.mu[row] = mean;
                a.rstd[row] = rs;
            }
        }
    }
}

// Backward with the pre-activation given (p_pre + bias; bias may be NULL, as for the
// forward's kept pre-activation): one wave per row, lane l owning columns 4 l + 256 q + e,
// so every load and store is a coalesced float4 and the LayerNorm row sums are wave
// reductions (no LDS, no barrier per row).  A wave walks rows r, r + stride, ...; the next
// row's inputs are requested before the current row is computed.  The column sums (dln_w,
// dln_b, dbias) accumulate in registers over the wave's rows, go through LDS once per
// workgroup and are added with one atomic per column and workgroup.
template <int Q4, bool SILU>
__global__ void __launch_bounds__(kGateThreads)
gating_bwd_rows_kernel(GateArgs a) {
    extern __shared__ __align__(16) float csm[];  // [3][kGateThreads / 64][D]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    constexpr int NW = kGateThreads / 64;
    const int D = a.D;
    float4 bias4[Q4], lnw4[Q4], accw[Q4], accb[Q4], accp[Q4];
#pragma unroll
    for (int q = 0; q < Q4; ++q) {
        const int c = 4 * lane + 256 * q;
        bias4[q] = a.bias ? *reinterpret_cast<const float4*>(a.bias + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        lnw4[q] = *reinterpret_cast<const float4*>(a.lnw + c);
        accw[q] = accb[q] = accp[q] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int64_t stride = (int64_t)gridDim.x * NW;
    int64_t r = (int64_t)blockIdx.x * NW + wave;
    float4 xv[Q4], dyv[Q4], ppv[Q4];
    auto load_row = [&](int64_t rr) {
#pragma unroll
        for (int q = 0; q < Q4; ++q) {
            const int c = 4 * lane + 256 * q;
            xv[q] = *reinterpret_cast<const float4*>(a.xq + rr * a.xq_sr + c);
            dyv[q] = *reinterpret_cast<const float4*>(a.dy + rr * D + c);
            ppv[q] = *reinterpret_cast<const float4*>(a.pp + rr * a.pp_sr + c);
        }
    };
    if (r < a.rows) load_row(r);
    for (; r < a.rows; r += stride) {
        const float mu = a.mu[r], rs = a.rstd[r];
        float xh[Q4][4], dxh[Q4][4], gg[Q4][4], xds[Q4][4];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int q = 0; q < Q4; ++q) {
            const float xe[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
            const float de[4] = {dyv[q].x, dyv[q].y, dyv[q].z, dyv[q].w};
            const float pe[4] = {ppv[q].x + bias4[q].x, ppv[q].y + bias4[q].y, ppv[q].z + bias4[q].z,
                                 ppv[q].w + bias4[q].w};
            const float we[4] = {lnw4[q].x, lnw4[q].y, lnw4[q].z, lnw4[q].w};
            float aw[4], ab[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float g = pe[e], dsil = 1.f;
                if (SILU) {
                    const float sg = sigmoidf_(pe[e]);
                    g = pe[e] * sg;
                    dsil = g + sg * (1.0f - g);  // SiLU' (triton_fused_gating.py:113-114)
                }
                gg[q][e] = g;
                xds[q][e] = xe[e] * dsil;
                xh[q][e] = (xe[e] * g - mu) * rs;
                dxh[q][e] = de[e] * we[e];
                s1 += dxh[q][e];
                s2 = __builtin_fmaf(dxh[q][e], xh[q][e], s2);
                aw[e] = de[e] * xh[q][e];
                ab[e] = de[e];
            }
            accw[q].x += aw[0]; accw[q].y += aw[1]; accw[q].z += aw[2]; accw[q].w += aw[3];
            accb[q].x += ab[0]; accb[q].y += ab[1]; accb[q].z += ab[2]; accb[q].w += ab[3];
        }
        // the next row's inputs while this one's sums reduce
        if (r + stride < a.rows) load_row(r + stride);
        const float c1 = wave_sum(s1) / (float)D;
        const float c2 = wave_sum(s2) / (float)D;
#pragma unroll
        for (int q = 0; q < Q4; ++q) {
            const int c = 4 * lane + 256 * q;
            float dq[4], dp[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float dxe = (dxh[q][e] - c1 - xh[q][e] * c2) * rs;
                dq[e] = dxe * gg[q][e];
                dp[e] = dxe * xds[q][e];
            }
            st_stream4(a.dxq + r * D + c, make_float4(dq[0], dq[1], dq[2], dq[3]));
            st_stream4(a.dpp + r * D + c, make_float4(dp[0], dp[1], dp[2], dp[3]));
            accp[q].x += dp[0]; accp[q].y += dp[1]; accp[q].z += dp[2]; accp[q].w += dp[3];
        }
    }
    // column sums: the workgroup's waves through LDS, then one atomic per column
#pragma unroll
    for (int q = 0; q < Q4; ++q) {
        const int c = 4 * lane + 256 * q;
        *reinterpret_cast<float4*>(csm + (0 * NW + wave) * D + c) = accw[q];
        *reinterpret_cast<float4*>(csm + (1 * NW + wave) * D + c) = accb[q];
        *reinterpret_cast<float4*>(csm + (2 * NW + wave) * D + c) = accp[q];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 3 * D; i += blockDim.x) {
        const int k = i / D, c = i % D;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += csm[(k * NW + w) * D + c];
        atomicAdd((k == 0 ? a.dlnw : k == 1 ? a.dlnb : a.dbias) + c, v);
    }
}

__global__ void gate_zero_kernel(float* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0.f;
}

// Workgroups walk row tiles with a grid stride.  The backward's workgroups each add their
// 3 x D column sums with atomics at the end, on the same 3 x D addresses, and only two of
// them fit on a CU at once (VGPRs): it runs on as many as are resident.
static int gate_grid(int64_t rows, bool bwd) {
    const int64_t ntiles = (rows + kGateRows - 1) / kGateRows;
    return (int)std::max<int64_t>(1, std::min<int64_t>(ntiles, bwd ? 256 * 2 : 256 * 8));
}

template <bool BWD>
static int gate_launch(const GateArgs& a, bool fused, bool silu, hipStream_t st) {
    const int cpt = (a.D + kGateThreads - 1) / kGateThreads;
    const size_t lds = ((BWD ? 2 : 1) * (size_t)kGateRows * a.D + 2 * kGateRows +
                        (fused ? (size_t)kGateRows * a.N : 0)) * sizeof(float);
    const dim3 grid(gate_grid(a.rows, BWD));
#define MB_GATE_K(C, F, S) (BWD ? gating_bwd_kernel<C, F, S> : gating_fwd_kernel<C, F, S>)
#define MB_GATE_CPT(C)                                                                          \
    do {                                                                                        \
        auto k = fused ? (silu ? MB_GATE_K(C, true, true) : MB_GATE_K(C, true, false))          \
                       : (silu ? MB_GATE_K(C, false, true) : MB_GATE_K(C, false, false));       \
        if (lds > 64 * 1024) {                                                                  \
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),                 \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); \
            if (e != hipSuccess) {                                                              \
                (void)hipGetLastError();                                                        \
                return fail((int)e, "gating: LDS attribute: %s", hipGetErrorString(e));         \
            }                                                                                   \
        }                                                                                       \
        hipLaunchKernelGGL(k, grid, dim3(kGateThreads), lds, st, a);                            \
    } while (0)
    switch (cpt) {
        case 1: MB_GATE_CPT(1); break;
        case 2: MB_GATE_CPT(2); break;
        case 3: MB_GATE_CPT(3); break;
        case 4: MB_GATE_CPT(4); break;
        default: return fail(MB_ERR_UNSUPPORTED, "gating: D=%d > %d", a.D, 4 * kGateThreads);
    }
#undef MB_GATE_CPT
#undef MB_GATE_K
    return check_launch(BWD ? "mb_gating_bwd" : "mb_gating_fwd");
}

constexpr int kGateRowsPerWave = 4;

static int gate_rows_fwd_launch(const GateArgs& a, bool silu, hipStream_t st) {
    constexpr int NW = kGateThreads / 64;
    constexpr int R = kGateRowsPerWave;
    const int64_t tiles = (a.rows + R - 1) / R;
    const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>((tiles + NW - 1) / NW, 1024)));
    const size_t lds = (size_t)NW * R * ((a.N + 3) & ~3) * sizeof(float);
#define MB_GATE_FROWS(Q)                                                                           \
    do {                                                                                           \
        auto k = silu ? gating_fwd_rows_kernel<Q, true, R> : gating_fwd_rows_kernel<Q, false, R>;  \
        hipLaunchKernelGGL(k, grid, dim3(kGateThreads), lds, st, a);                               \
    } while (0)
    switch (a.D / 256) {
        case 1: MB_GATE_FROWS(1); break;
        case 2: MB_GATE_FROWS(2); break;
        case 3: MB_GATE_FROWS(3); break;
        default: return fail(MB_ERR_UNSUPPORTED, "mb_gating_fwd: D=%d", a.D);
    }
#undef MB_GATE_FROWS
    return check_launch("mb_gating_fwd");
}

static int gate_rows_bwd_launch(const GateArgs& a, bool silu, hipStream_t st) {
    constexpr int NW = kGateThreads / 64;
    const int64_t waves = (a.rows + NW - 1) / NW;
    const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>(waves, 512)));
    const size_t lds = (size_t)3 * NW * a.D * sizeof(float);
#define MB_GATE_ROWS(Q)                                                                            \
    do {                                                                                           \
        auto k = silu ? gating_bwd_rows_kernel<Q, true> : gating_bwd_rows_kernel<Q, false>;        \
        hipLaunchKernelGGL(k, grid, dim3(kGateThreads), lds, st, a);                               \
    } while (0)
    switch (a.D / 256) {
        case 1: MB_GATE_ROWS(1); break;
        case 2: MB_GATE_ROWS(2); break;
        case 3: MB_GATE_ROWS(3); break;
        case 4: MB_GATE_ROWS(4); break;
        default: return fail(MB_ERR_UNSUPPORTED, "mb_gating_bwd: D=%d", a.D);
    }
#undef MB_GATE_ROWS
    return check_launch("mb_gating_bwd");
}

static int gate_validate(const char* who, const GateArgs& a, bool fused) {
    MB_REQUIRE(a.rows >= 0, "%s: negative rows %lld", who, (long long)a.rows);
    MB_REQUIRE(a.D >= 1, "%s: D=%d must be >= 1", who, a.D);
    if (a.D > 4 * kGateThreads) return fail(MB_ERR_UNSUPPORTED, "%s: D=%d > %d", who, a.D, 4 * kGateThreads);
    MB_REQUIRE(a.xq_sr >= a.D, "%s: x_q row stride %lld < D=%d", who, (long long)a.xq_sr, a.D);
    if (fused) {
        MB_REQUIRE(a.N >= 1 && a.N <= 1024, "%s: N=%d out of range 1..1024", who, a.N);
        MB_REQUIRE(a.c_sr >= a.N, "%s: C_seq row stride %lld < N=%d", who, (long long)a.c_sr, a.N);
    } else {
        MB_REQUIRE(a.pp_sr >= a.D, "%s: p_pre row stride %lld < D=%d", who, (long long)a.pp_sr, a.D);
    }
    return MB_OK;
}

}  // namespace mb

using namespace mb;

extern "C" int mb_gating_fwd(const float* x_q, int64_t xq_row_stride, const float* p_pre,
                             int64_t pp_row_stride, const float* bias, const float* C_seq,
                             int64_t c_row_stride, const float* W_pe, int N, const float* ln_w,
                             const float* ln_b, int64_t rows, int D, int use_silu, float eps,
                             float* y, float* mu, float* rstd, float* pre_out, void* stream) {
    GateArgs a{};
    a.xq = x_q; a.xq_sr = xq_row_stride; a.pp = p_pre; a.pp_sr = pp_row_stride; a.bias = bias;
    a.C = C_seq; a.c_sr = c_row_stride; a.W = W_pe; a.N = N; a.lnw = ln_w; a.lnb = ln_b;
    a.rows = rows; a.D = D; a.eps = eps; a.y = y; a.mu = mu; a.rstd = rstd; a.pre_out = pre_out;
    const bool fused = p_pre == nullptr;
    int rc = gate_validate("mb_gating_fwd", a, fused);
    if (rc) return rc;
    if (rows == 0) return MB_OK;
    MB_REQUIRE(x_q && ln_w && ln_b && y && mu && rstd, "mb_gating_fwd: null pointer");
    MB_REQUIRE(fused ? (C_seq && W_pe) : true, "mb_gating_fwd: need p_pre, or C_seq and W_pe");
    // with the projection folded in: the rows kernel, when its float4 lanes fit the layout
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (fused && D % 256 == 0 && D <= 768 && N <= 128 && xq_row_stride % 4 == 0 && al16(x_q) &&
        al16(W_pe) && al16(ln_w) && al16(ln_b) && al16(y) && (!pre_out || al16(pre_out)))
        return gate_rows_fwd_launch(a, use_silu != 0, (hipStream_t)stream);
    return gate_launch<false>(a, fused, use_silu != 0, (hipStream_t)stream);
}

extern "C" int mb_gating_bwd(const float* dy, const float* x_q, int64_t xq_row_stride,
                             const float* p_pre, int64_t pp_row_stride, const float* bias,
                             const float* C_seq, int64_t c_row_stride, const float* W_pe, int N,
                             const float* ln_w, const float* mu, const float* rstd, int64_t rows,
                             int D, int use_silu, float* dx_q, float* dp_pre, float* dbias,
                             float* dln_w, float* dln_b, void* stream) {
    GateArgs a{};
    a.dy = dy; a.xq = x_q; a.xq_sr = xq_row_stride; a.pp = p_pre; a.pp_sr = pp_row_stride;
    a.bias = bias; a.C = C_seq; a.c_sr = c_row_stride; a.W = W_pe; a.N = N; a.lnw = ln_w;
    a.mu = const_cast<float*>(mu); a.rstd = const_cast<float*>(rstd);
    a.rows = rows; a.D = D;
    a.dxq = dx_q; a.dpp = dp_pre; a.dbias = dbias; a.dlnw = dln_w; a.dlnb = dln_b;
    const bool fused = p_pre == nullptr;
    int rc = gate_validate("mb_gating_bwd", a, fused);
    if (rc) return rc;
    MB_REQUIRE(dbias && dln_w && dln_b, "mb_gating_bwd: null column-sum output");
    hipStream_t st = (hipStream_t)stream;
    // The column sums are accumulated with atomics: clear them first (fill kernel).
    hipLaunchKernelGGL(gate_zero_kernel, dim3(1), dim3(256), 0, st, dbias, D);
    hipLaunchKernelGGL(gate_zero_kernel, dim3(1), dim3(256), 0, st, dln_w, D);
    hipLaunchKernelGGL(gate_zero_kernel, dim3(1), dim3(256), 0, st, dln_b, D);
    if ((rc = check_launch("mb_gating_bwd: clear"))) return rc;
    if (rows == 0) return MB_OK;
    MB_REQUIRE(dy && x_q && ln_w && mu && rstd && dx_q && dp_pre, "mb_gating_bwd: null pointer");
    MB_REQUIRE(fused ? (C_seq && W_pe) : true, "mb_gating_bwd: need p_pre, or C_seq and W_pe");
    // with the pre-activation given: the row kernel, when its float4 lanes fit the layout
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (!fused && D % 256 == 0 && D <= 1024 && xq_row_stride % 4 == 0 && pp_row_stride % 4 == 0 &&
        al16(x_q) && al16(p_pre) && al16(dy) && al16(dx_q) && al16(dp_pre) && al16(ln_w) &&
        (!bias || al16(bias)))
        return gate_rows_bwd_launch(a, use_silu != 0, st);
    return gate_launch<true>(a, fused, use_silu != 0, st);
}
