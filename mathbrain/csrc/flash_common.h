// Pieces shared by the flash-EMA forward and backward kernels (gfx950).
//
// Both kernels work on one (sequence b, 32-step block) per workgroup and walk the valid
// slots of b in batches of SB.  For every batch the whole workgroup first builds, in LDS,
//   cdec[j][t][n]  (fp16)  the decayed key-side counter c_dec[t, u_j, n] that gates step t,
//   cdecT[j][n][t] (bf16)  the same counter, transposed, for the backward's dW_pe product,
//   E[j][0|1][D]   (fp32)  the slot's key and value embeddings,
// and every wave then consumes the batch for its head(s).  The counter comes from the
// chunk-start state S = C_bounds[b, t0 / Br, k] and the slot's occurrences inside the
// window [cb, t0 + 32) (cb = chunk start):
//   c_dec[t] = S rho^(t-cb+1) + sum_{cb <= s < t, x_s = u} rho^(t-s)
// which is the reference's per-step  c_dec = C * rho ; C = c_dec + match
// (mathbrain/triton_flash_ema.py:150-153, 175, 185, 241) unrolled from the chunk start.
//
// Gate operands are fp16 (c_dec and W_pe * log2 e, round to nearest even), not bf16: the
// gate pre-activation sum_n c_n W_n cancels, and the dW_pe sums over thousands of steps
// cancel further, so bf16's 8-bit significand moved dW_pe by ~2.5e-2 (norm-wise, against
// float64) at T = 4096 with long half-lives.  Where the lo tiles fit (N <= 64, head_dim <=
// 64) each operand is split into an fp16 hi part and an fp16 lo part (three products,
// ~2^-22 relative): with scores near 100 the softmax multiplies a relative gate error by
// ~100, and one fp16 product per operand (11 bits) then moves the output by ~2e-2.  The
// counter stays in fp16 range: the host refuses rates whose EMA of one occurrence per step
// could pass kCMax; a caller-supplied initial state above kCMax (which no such EMA reaches)
// saturates at kCMax when loaded; the window adds at most kMaxWin; rho <= 1.  dpre, whose
// scale is unbounded, keeps bf16 for the dW_pe product, so that product takes the bf16 copy
// of the tile.
#pragma once

#include <hip/hip_bf16.h>

#include "common.h"

namespace mb {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;
constexpr int kTB = 32;      // time steps per workgroup
constexpr int kMaxWin = 64;  // positions [cb, t0 + 32) of the match window
constexpr float kCMax = 65504.0f - kMaxWin;  // chunk-start counters saturate here (fp16)

struct FlashArgs {
    const float* Q;
    int64_t q_sb, q_sh, q_sl, q_sd;
    const int64_t* x;
    int64_t x_sb, x_sl;
    const float* Ek;  // [B, K, D], or [e_rows, D] indexed by token id (FlashArgsV)
    const float* Ev;  // the same
    const float* W;   // [N, D]  (pe_proj.weight transposed)
    const float* rhos;
    const int64_t* unique;  // [B, K], -1 = padding
    const float* Cb;        // [B, nc, K, Np]
    int B, H, L, hd, K, N, Np, Br, nc;
    float v_total;  // vocabulary size; < 0 drops the absent-slot softmax mass
    int silu;
    float* O;    // [B, H, L, hd]
    float* LSE;  // [B, H, L]
    float* S2out;        // optional [B, H, K, L]: scores * log2 e (forward output)
    const float* S2in;   // optional, the same, read by the backward
    // backward only
    const float* dO;   // [B, H, L, hd], same strides as Q
    const float* Oin;  // forward output, [B, H, L, hd] contiguous
    const float* LSEin;
    float* dQ;   // [B, H, L, hd] contiguous
    float* dEk;  // like Ek, accumulated with atomics (zeroed by the host)
    float* dEv;
    float* dW;   // [N, D], accumulated with atomics (zeroed by the host)
    int head_groups;  // backward: workgroups per (b, block) along heads
};

// Arguments of the kernels whose E_k / E_v (and dE_k / dE_v) rows are token ids into
// [e_rows, D] vocabulary tables (their VR template parameter).  A separate type, so that
// the other kernels keep their argument layout (and with it their code schedule).
struct FlashArgsV : FlashArgs {
    int64_t e_rows;
};
template <bool VR> struct FlashArgsOf { using type = FlashArgs; };
template <> struct FlashArgsOf<true> { using type = FlashArgsV; };

__device__ inline int64_t e_rows_of(const FlashArgs& a) { return (int64_t)a.B * a.K; }
__device__ inline int64_t e_rows_of(const FlashArgsV& a) { return a.e_rows; }

// Sets a kernel's dynamic LDS limit and launches it with its arguments.
template <class Kern, class... Args>
static int launch_with_lds(Kern k, dim3 grid, int nthr, size_t lds, hipStream_t st, const char* who,
                           const Args&... args) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail((int)e, "%s: LDS attribute: %s", who, hipGetErrorString(e));
    }
    hipLaunchKernelGGL(k, grid, dim3(nthr), lds, st, args...);
    return MB_OK;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ inline f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 16x16x16 bf16 MFMA: A[row = lane%16][k = 4*(lane/16) + e], B[k][col = lane%16].
__device__ inline f32x4 mfma16x16x16(bf16x4 a, bf16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

// Exchange helpers on the four 16-lane rows of a wave (gfx950 v_permlane{16,32}_swap).
// Inline asm: __builtin_amdgcn_permlane{16,32}_swap give the same lanes (checked on the
// GPU) but measured 0.5 % slower in the backward.  The s_nop pads cover the VALU-write ->
// permlane-read hazard.
__device__ inline float2 swap_halves(float a, float b) {
    // a' = {a.lo, b.lo}, b' = {a.hi, b.hi}
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return make_float2(a, b);
}
__device__ inline float2 swap_odd_rows(float a, float b) {
    // a' = {a.r0, b.r0, a.r2, b.r2}, b' = {a.r1, b.r1, a.r3, b.r3}
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return make_float2(a, b);
}

// Reduce-scatter over the four rows: v[k] holds per-lane partials of 4 quantities;
// returns, in row g, the sum over all rows of v[g] (lane l gets sum_r v[g][16 r + l%16]).
__device__ inline float rows4_reduce_scatter(float v0, float v1, float v2, float v3) {
    const float2 a = swap_halves(v0, v2);  // lo: v0 halves, hi: v2 halves
    const float2 b = swap_halves(v1, v3);
    const float x02 = a.x + a.y;           // rows 0,1: v0 over halves; rows 2,3: v2
    const float x13 = b.x + b.y;
    const float2 c = swap_odd_rows(x02, x13);
    return c.x + c.y;                      // row 0: v0, row 1: v1, row 2: v2, row 3: v3
}

// Same for two quantities: row 0 gets the sum of v0, row 2 the sum of v1 (rows 1, 3: 0).
__device__ inline float rows4_reduce_scatter2(float v0, float v1) {
    const float2 a = swap_halves(v0, v1);
    const float x = a.x + a.y;             // rows 0,1: v0 over halves; rows 2,3: v1
    const float2 c = swap_odd_rows(x, 0.0f);
    return c.x + c.y;
}

// Sums over the 16 lanes of a DPP row of n values, stage by stage: the n independent
// chains interleave, so no DPP read waits on the VALU write just before it.
template <int n>
__device__ inline void row_sum16_n(float (&v)[n]) {
#pragma unroll
    for (int i = 0; i < n; ++i) v[i] += __builtin_amdgcn_update_dpp(0.0f, v[i], 0xB1, 0xF, 0xF, false);
#pragma unroll
    for (int i = 0; i < n; ++i) v[i] += __builtin_amdgcn_update_dpp(0.0f, v[i], 0x4E, 0xF, 0xF, false);
#pragma unroll
    for (int i = 0; i < n; ++i) v[i] += __builtin_amdgcn_update_dpp(0.0f, v[i], 0x141, 0xF, 0xF, false);
#pragma unroll
    for (int i = 0; i < n; ++i) v[i] += __builtin_amdgcn_update_dpp(0.0f, v[i], 0x140, 0xF, 0xF, false);
}

// Two floats to a packed bf16 pair (round to nearest even) in one v_cvt_pk_bf16_f32; a
// vector cast compiles to one conversion per value plus a v_perm here.
__device__ inline bf16x2 cvt_pk_bf16(float lo, float hi) {
    uint32_t r;
    asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
    return __builtin_bit_cast(bf16x2, r);
}

// Sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15); every lane gets the sum.
__device__ inline float row_sum16(float v) {
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, false);  // row_mirror
    return v;
}

// Workgroup id -> logical id so that consecutive logical ids (the blocks of one
// sequence, which share its slot embeddings) land on the same XCD and its L2:
// the dispatcher hands workgroups to the 8 XCDs round-robin.
__device__ inline int xcd_major(int bid, int G) {
    if (G % 8) return bid;
    return (bid % 8) * (G / 8) + bid / 8;
}

// LDS carve-up of the per-batch staging buffers: cdec (fp16), with BF the transposed bf16
// copy cdecT ([SB][NPAD][TROW], steps contiguous, for the backward's dW_pe product), then E.
// With PG (the split gate) the cdec tile has a second, "lo" tile right after it,
// cdec_lo = fp16(c - cdec), so that hi + lo carries the counter to ~2^-22 relative; with PW
// (the split dW_pe product) the cdecT tile has one too, cdecT_lo = bf16(c - cdecT) (~2^-16).
template <int NPAD, int SB, bool BF = false, bool PG = false, bool PW = false>
struct Stage {
    static_assert(!PW || (BF && PG), "the split dW_pe product comes with the split gate's tiles");
    static constexpr int CROW = NPAD + 8;  // 16-bit entries per cdec row (16 B pad against conflicts)
    static constexpr int CDEC = SB * kTB * CROW;  // entries per tile
    static constexpr int NTC = PG ? 2 : 1;        // cdec tiles (hi, lo)
    static constexpr int NTT = PW ? 2 : 1;        // cdecT tiles (hi, lo)
    // cdecT row: kTB steps + 4 entries of padding, so that 16 rates x 4 step groups read by
    // one wave start on 64 distinct LDS banks
    static constexpr int TROW = kTB + 4;
    static constexpr int CT = BF ? SB * NPAD * TROW : 0;
    static constexpr int CTOFF = NTC * CDEC * 2;             // byte offset of cdecT
    static constexpr int EOFF = (NTC * CDEC + NTT * CT) * 2;  // byte offset of E
    // width: embedding columns staged per slot
    __host__ __device__ static size_t bytes(int width) {
        return (size_t)EOFF + (size_t)SB * 2 * width * 4;
    }
};

// Gate arithmetic of a flash-EMA call, the same in the forward and the backward:
// 2 = MB_FLASH_FP32 (split gate and split dW_pe product), 1 = the default's split gate with
// bf16 dW_pe operands, 0 = single fp16 gate products (MB_FLASH_FAST_GATE, and the default
// where the lo tiles do not fit in LDS: N > 64 or head_dim 128).  Negative: MB_FLASH_FP32
// with a shape it does not take (the error is set).
static inline int flash_gate_mode(const char* who, int flags, int N, int hd) {
    if (flags & MB_FLASH_FP32) {
        if (N > 64) return fail(MB_ERR_UNSUPPORTED, "%s: MB_FLASH_FP32 needs N <= 64 (N=%d)", who, N);
        if (hd > 64) return fail(MB_ERR_UNSUPPORTED, "%s: MB_FLASH_FP32 needs head_dim <= 64 (hd=%d)", who, hd);
        return 2;
    }
    if (flags & MB_FLASH_FAST_GATE) return 0;
    return N <= 64 && hd <= 64 ? 1 : 0;
}

// Row of slot (b, k), token id u, in E_k / E_v / dE_k / dE_v: b*K + k, or with VR
// the token id (padding slots, -1, read row 0; ids are clamped to the table).  u comes from
// the batch's slot info in LDS: a global read here would make the producer's other loads
// wait with it (memory reads complete in order).
template <bool VR, class A>
__device__ inline int64_t e_row(const A& a, int b, int k, int64_t u) {
    if (!VR) return (int64_t)b * a.K + k;
    return min(max(u, (int64_t)0), e_rows_of(a) - 1);
}

struct BatchMeta {
    int64_t u;
    uint64_t mask;
};

// Per-workgroup setup shared by both kernels: the match window tokens, the rho^j table
// (j = 0..64) and the valid-slot range of sequence b.
template <int NPAD>
__device__ void flash_setup(const FlashArgs& a, int b, int t0, int cb, int64_t* win,
                            float* powt, int* kinfo) {
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    for (int p = tid; p < kMaxWin; p += nthr) {
        const int pos = cb + p;
        win[p] = (pos < a.L && pos < t0 + kTB) ? a.x[(int64_t)b * a.x_sb + (int64_t)pos * a.x_sl]
                                              : (int64_t)-1;
    }
    for (int i = tid; i < 65 * NPAD; i += nthr) {
        const int j = i / NPAD;
        const int n = i % NPAD;
        float v = 0.0f;
        if (n < a.N) {
            float hi, lo;
            log2_split(a.rhos[n], hi, lo);
            v = pow_steps(hi, lo, j);
        }
        powt[i] = v;
    }
    if (tid == 0) {
        kinfo[0] = 0;   // valid slots K_b
        kinfo[1] = 0;   // one past the last valid slot
    }
    __syncthreads();
    int cnt = 0, last = 0;
    for (int k = tid; k < a.K; k += nthr) {
        if (a.unique[(int64_t)b * a.K + k] >= 0) {
            ++cnt;
            last = k + 1;
        }
    }
    if (cnt) atomicAdd(&kinfo[0], cnt);
    if (last) atomicMax(&kinfo[1], last);
    __syncthreads();
}

// Rate tiles of the default mode's split gate that take the lo products (bit ns: tile ns),
// for two 32-rate tiles: a counter is an EMA of at most one occurrence per step, so it stays
// near or below B = 1 / (1 - rho), and a single fp16 product's rounding on a rate's term
// scales with its counter; the first tile is left to the single product (2) when its largest
// B is below 1/32 of the second's, else both are corrected (3).  Lane n reads rate n; every
// wave computes the same value, so it is uniform over the workgroup.
__device__ inline int split_tiles(const FlashArgs& a, int lane) {
    float bh = lane < a.N ? 1.0f / fmaxf(1.0f - a.rhos[lane], 1e-30f) : 0.f;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) bh = fmaxf(bh, __shfl_xor(bh, off));
    const float bo = __shfl_xor(bh, 32);
    const float b0 = lane < 32 ? bh : bo;
    const float b1 = lane < 32 ? bo : bh;
    return 32.0f * b0 < fmaxf(b0, b1) ? 2 : 3;
}

// Slot ids and 64-bit occurrence masks of batch `bi`: wave j < SB handles slot j.
template <int SB>
__device__ void flash_batch_meta(const FlashArgs& a, int b, int bi, int kend, const int64_t* win,
                                 BatchMeta* meta) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int nwaves = blockDim.x >> 6;
    for (int j = wave; j < SB; j += nwaves) {
        const int k = bi * SB + j;
        const int64_t u = (k < kend) ? a.unique[(int64_t)b * a.K + k] : (int64_t)-1;
        const bool hit = u >= 0 && win[lane] == u;
        const uint64_t m = __ballot(hit);
        if (lane == 0) {
            meta[j].u = u;
            meta[j].mask = m;
        }
    }
}

typedef __attribute__((address_space(3))) void lds_void;

// Producer: each thread owns up to MAXI blocks (slot j, 4 steps, 4 rates) of the batch's
// cdec tiles and up to MAXE float4 of the embedding copy.  MAXE = 0: the embedding rows go
// from global memory straight into the staging buffer (load_e_lds), without registers.
template <int NPAD, int SB, int MAXI, int MAXE>
struct Producer {
    static constexpr int BPS = (kTB / 4) * (NPAD / 4);  // blocks per slot
    float4 s[MAXI];
    float4 e[MAXE > 0 ? MAXE : 1];

    // The batch's E_k / E_v rows ([SB][2][width] floats) into E with global_load_lds_dwordx4:
    // wave w issues the 1 KB pieces w, w + waves, ...; lane l of a piece moves float4 64 c + l,
    // which lands at E + 4 (64 c + l) (the instruction writes lane l's 16 bytes at the LDS
    // address in M0 plus 16 l).  Rows of slots past kend are not loaded (no slot reads them).
    // The caller waits for the loads (vmcnt) before the barrier that publishes E.
    template <bool VR, class A>
    __device__ void load_e_lds(const A& a, int b, int bi, int kend, int D, int col0, int width,
                               const BatchMeta* meta, float* E) const {
        const int w4 = width / 4;
        const int nvec = SB * 2 * w4;
        const int lane = threadIdx.x & 63;
        const int nw = blockDim.x >> 6;
        for (int c = threadIdx.x >> 6; c * 64 < nvec; c += nw) {
            const int i = c * 64 + lane;
            const int j = i / (2 * w4);
            const int r = i % (2 * w4);
            const int which = r / w4;
            const int c4 = r % w4;
            const int k = bi * SB + j;
            if (i < nvec && k < kend && col0 + c4 * 4 < D) {
                const float* src =
                    (which ? a.Ev : a.Ek) + e_row<VR>(a, b, k, VR ? meta[j].u : 0) * D + col0 + c4 * 4;
                __builtin_amdgcn_global_load_lds(src, (lds_void*)(E + 256 * c), 16, 0, 0);
            }
        }
    }

    template <bool VR, class A>
    __device__ void load(const A& a, int b, int cbi, int bi, int kend, int D, int col0,
                         int width, const BatchMeta* meta) {
        const int tid = threadIdx.x;
        const int nthr = blockDim.x;
#pragma unroll
        for (int ii = 0; ii < MAXI; ++ii) {
            const int item = tid + ii * nthr;
            const int j = item / BPS;
            const int n0 = (item % (NPAD / 4)) * 4;
            const int k = bi * SB + j;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (j < SB && k < kend) {
                const float* src = a.Cb + (((int64_t)b * a.nc + cbi) * a.K + k) * a.Np + n0;
                if (n0 + 3 < a.N && (a.Np & 3) == 0) {
                    v = *reinterpret_cast<const float4*>(src);
                } else {
                    if (n0 + 0 < a.N) v.x = src[0];
                    if (n0 + 1 < a.N) v.y = src[1];
                    if (n0 + 2 < a.N) v.z = src[2];
                    if (n0 + 3 < a.N) v.w = src[3];
                }
            }
            s[ii] = v;
        }
        const int w4 = width / 4;
        const int nvec = SB * 2 * w4;
#pragma unroll
        for (int ie = 0; ie < MAXE; ++ie) {
            const int i = tid + ie * nthr;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < nvec) {
                const int j = i / (2 * w4);
                const int r = i % (2 * w4);
                const int which = r / w4;
                const int c4 = r % w4;
                const int k = bi * SB + j;
                // columns past D (heads a partial head group does not have) stay zero
                if (k < kend && col0 + c4 * 4 < D) {
                    const float* src =
                        (which ? a.Ev : a.Ek) + e_row<VR>(a, b, k, VR ? meta[j].u : 0) * D + col0 + c4 * 4;
                    v = *reinterpret_cast<const float4*>(src);
                }
            }
            e[ie] = v;
        }
    }

    // Builds cdec ([SB][kTB][CROW], fp16), with BF also cdecT ([SB][NPAD][TROW], bf16), and E
    // ([SB][2][width]) of the batch into the staging buffer.  With PG also cdec's lo tile, CLO
    // entries after cdec, and with PW cdecT's, CTLO entries after cdecT (see Stage).  With PG
    // the bf16 copy rounds the float32 counter; without, the gate's fp16 counter (the gate and
    // the dW_pe product then see one c_dec).  lo_tiles (PG): the 32-rate tiles whose lo entries
    // are the rounding remainders (bit ns); the others' are written as zeros (split_tiles).
    template <bool BF, int CROW, int TROW, bool PG = false, bool PW = false, int CLO = 0, int CTLO = 0>
    __device__ void store(int t0, int cb, const float* powt, const BatchMeta* meta,
                          _Float16* cdec, __bf16* cdecT, float* E, int width, int lo_tiles = 3) {
        const int tid = threadIdx.x;
        const int nthr = blockDim.x;
#pragma unroll
        for (int ii = 0; ii < MAXI; ++ii) {
            const int item = tid + ii * nthr;
            const int j = item / BPS;
            if (j >= SB) continue;
            const int tq = (item % BPS) / (NPAD / 4);
            const int n0 = (item % (NPAD / 4)) * 4;
            // Clamped here, not at the load, so that the load's wait stays at this use.
            const float4 sv = make_float4(fminf(s[ii].x, kCMax), fminf(s[ii].y, kCMax),
                                          fminf(s[ii].z, kCMax), fminf(s[ii].w, kCMax));
            const uint64_t mask = meta[j].mask;
            bf16x4 tb[4], tl4[4];
            // The quad's first step sums its window directly; the next three follow by
            // c_dec[t + 1] = rho (c_dec[t] + [x_t == u]).
            const float4 rho = *reinterpret_cast<const float4*>(powt + NPAD + n0);
            float c0, c1, c2, c3;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tl = 4 * tq + r;
                const int tr = t0 - cb + tl;  // 0 .. 63
                if (r == 0) {
                    const float4 pw = *reinterpret_cast<const float4*>(powt + (tr + 1) * NPAD + n0);
                    c0 = sv.x * pw.x;
                    c1 = sv.y * pw.y;
                    c2 = sv.z * pw.z;
                    c3 = sv.w * pw.w;
                    uint64_t m = mask & ((1ull << tr) - 1ull);
                    while (m) {
                        const int p = __builtin_ctzll(m);
                        m &= m - 1;
                        const float4 q = *reinterpret_cast<const float4*>(powt + (tr - p) * NPAD + n0);
                        c0 += q.x;
                        c1 += q.y;
                        c2 += q.z;
                        c3 += q.w;
                    }
                } else {
                    const float hit = (mask >> (tr - 1)) & 1ull ? 1.f : 0.f;
                    c0 = (c0 + hit) * rho.x;
                    c1 = (c1 + hit) * rho.y;
                    c2 = (c2 + hit) * rho.z;
                    c3 = (c3 + hit) * rho.w;
                }
                if (PG) {
                    // hi and lo come from one materialised float32 counter: a conversion the
                    // compiler fused with the last add would round hi from a different value
                    asm volatile("" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3));
                }
                // two values per conversion (round to nearest even, as one at a time)
                const f16x2 w01 = __builtin_convertvector(f32x2{c0, c1}, f16x2);
                const f16x2 w23 = __builtin_convertvector(f32x2{c2, c3}, f16x2);
                const f16x4 w = {w01[0], w01[1], w23[0], w23[1]};
                *reinterpret_cast<f16x4*>(cdec + (j * kTB + tl) * CROW + n0) = w;
                if (PG) {  // the fp16 rounding remainder
                    f16x4 wl = {0, 0, 0, 0};
                    if ((lo_tiles >> (n0 >> 5)) & 1) {
                        wl[0] = (_Float16)(c0 - (float)w[0]);
                        wl[1] = (_Float16)(c1 - (float)w[1]);
                        wl[2] = (_Float16)(c2 - (float)w[2]);
                        wl[3] = (_Float16)(c3 - (float)w[3]);
                    }
                    *reinterpret_cast<f16x4*>(cdec + CLO + (j * kTB + tl) * CROW + n0) = wl;
                }
                if (BF && PG) {  // bf16 (with PW hi + lo) of the float32 counter
                    const float cv[4] = {c0, c1, c2, c3};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const __bf16 h = (__bf16)cv[q];
                        tb[q][r] = h;
                        if (PW) tl4[q][r] = (__bf16)(cv[q] - (float)h);
                    }
                } else if (BF) {  // bf16 of the gate's fp16 counter (the gate and dW_pe see one c_dec)
                    tb[0][r] = (__bf16)(float)w[0];
                    tb[1][r] = (__bf16)(float)w[1];
                    tb[2][r] = (__bf16)(float)w[2];
                    tb[3][r] = (__bf16)(float)w[3];
                }
            }
            if (BF) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    *reinterpret_cast<bf16x4*>(cdecT + (j * NPAD + n0 + q) * TROW + 4 * tq) = tb[q];
                    if (PW)
                        *reinterpret_cast<bf16x4*>(cdecT + CTLO + (j * NPAD + n0 + q) * TROW + 4 * tq) = tl4[q];
                }
            }
        }
        const int nvec = SB * 2 * (width / 4);
#pragma unroll
        for (int ie = 0; ie < MAXE; ++ie) {
            const int i = tid + ie * nthr;
            if (i < nvec) reinterpret_cast<float4*>(E)[i] = e[ie];
        }
    }
};

}  // namespace mb
