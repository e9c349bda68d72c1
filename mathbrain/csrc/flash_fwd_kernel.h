// Flash-EMA gated cross-attention forward kernel on gfx950 (template, its LDS size and its
// launcher), shared by the entry points of flash_fwd.hip and flash_gq_fwd.hip.
//
// Replaces _flash_ema_fwd and flash_ema_forward (mathbrain/triton_flash_ema.py:121-241,
// :529-568).  Semantics, per sequence b, head h, step t and valid slot k:
//   g[t,k,:] = SiLU(c_dec[t,k,:] . W_pe[:, h])         (fp16 operands, fp32 accumulate)
//   s[t,k]   = q_t . (e_k[k] * g[t,k]) / sqrt(hd)
//   O_t      = sum_k softmax_k(s) e_v[k] * g[t,k],   LSE_t = log sum_k exp(s)
// where, when v_total >= 0, the softmax also holds the V - K_b absent slots of the
// dense reference (mathbrain/flash_ema_attention.py:76-77): their counters are zero,
// so their gate SiLU(0) = 0 gives score 0 and value 0, i.e. they add (V - K_b) e^0 to
// the denominator and nothing to the numerator.
//
// Layout: one workgroup per (b, 32-step block) with one wave per head.  The gate GEMM
// is computed transposed, pre^T[d, t] = W^T[d, :] c_dec^T[:, t], with
// v_mfma_f32_16x16x32_f16, so each lane owns one step t (lane % 16 of a 16-step tile)
// and 16 of the head's 64 dims (rows 16*dt + 4*(lane/16) + i): the score's sum over d
// stays in registers (plus two cross-lane adds), and O_t's sum over slots accumulates
// in registers across the slot loop.  The online softmax runs in the log2 domain
// (W is pre-scaled by log2 e) and rescales only when a score beats the running max by
// more than 2^8, which keeps every exponential <= 256.
#pragma once
#include "flash_gq.h"

#include <algorithm>

namespace mb {

constexpr float kTau = 8.0f;

// VR: E_k / E_v are vocabulary tables indexed by the slot's token id (MB_FLASH_VOCAB_ROWS).
// PREC (MB_FLASH_FP32): the gate GEMM carries both operands as fp16 hi + lo pairs,
//   pre = W_lo c_hi + W_hi c_lo + W_hi c_hi  (three MFMAs, fp32 accumulation),
// which leaves ~2^-22 relative error per product instead of fp16's 2^-11; W_lo waits in
// LDS (W_hi stays in registers) and the producer writes a c_lo tile beside c_hi.  The default
// mode (PREC without FwdSplit::full) takes the two lo products only for the 32-rate tiles
// whose counters can be large (split_tiles: with rates spread from half-life 1 to 4096, the
// first tile's counters stay below ~87 against the second's ~5900, and the first takes the
// single product).  MB_FLASH_FP32 corrects every tile.
// GQ: the workgroup computes its queries from the gating inputs (flash_gq.h) instead of
// reading Q.
// Slot parts of the forward: each (b, block, head group) runs as ksplit workgroups over
// consecutive ranges of its slot batches.  With ksplit > 1 each part writes its unnormalised
// softmax state to `part` (ksplit x [B*H*L][hd] sums o, then ksplit x [B*H*L] (m, l) pairs)
// and flash_fwd_merge_kernel forms O and LSE.  A second kernel argument, so that the
// argument block the backward shares keeps its layout.
struct FwdSplit {
    float* part;
    int ksplit;
    int full;  // PREC: every rate tile takes the lo products (MB_FLASH_FP32)
};

// TW: 16-step tiles per wave.  2 (head_dim <= 64): wave w < hpg takes head w and both tiles
// of the block; 1 (head_dim 128): wave w < 2 hpg takes head w % hpg and tile w / hpg, so that
// a lane's queries, outputs and gate tiles stay within the register budget.
// CM (PREC): the rate tiles whose gate takes the lo products (bit ns: tile ns).  With two
// tiles a default-mode launch runs the CM = 3 and the CM = 2 instantiation over the same grid,
// and each workgroup returns at entry unless split_tiles picks its CM (one global read and a
// few shuffles); a mask fixed at compile time keeps each slot loop's MFMA chain unbroken.
template <int HD, int NS, int SB, int MAXI, int MAXE, bool SILU, bool VR, bool PREC = false, bool GQ = false,
          int CM = (1 << NS) - 1>
__global__ void __launch_bounds__(512, 1)
flash_ema_fwd_kernel(typename FlashArgsK<VR, GQ>::type a, FwdSplit sp) {
    constexpr int NPAD = 32 * NS;
    constexpr int DT = HD / 16;
    constexpr int TW = HD > 64 ? 1 : 2;
    static_assert(TW == 2 || (!GQ && !PREC), "head_dim 128: default mode only");
    using S = Stage<NPAD, SB, false, PREC, false>;
    extern __shared__ __align__(16) unsigned char smem[];

    const int D = a.H * HD;
    const int ntb = (a.L + kTB - 1) / kTB;
    const int logical = xcd_major(blockIdx.x, gridDim.x);
    // one workgroup per (b, slot part, 32-step block, head group); a group holds hpg heads
    // (hpg divides H), one wave each, and waves past hpg only help stage and synchronise.
    // The blocks of one (b, part) are neighbours, so they share an XCD's L2 for their rows.
    const int hg = logical % a.head_groups;
    const int t0 = ((logical / a.head_groups) % ntb) * kTB;
    const int part = (logical / (a.head_groups * ntb)) % sp.ksplit;
    const int b = logical / (a.head_groups * ntb * sp.ksplit);
    const int cbi = t0 / a.Br;
    const int cb = cbi * a.Br;
    const int hpg = a.H / a.head_groups;
    const int WIDF = hpg * HD;     // embedding columns staged: this group's heads
    const int col0 = hg * WIDF;

    // LDS: two staging buffers, a 3-deep ring of batch slot info (batch i+2's info is
    // written while batch i is still being read), the window, the power table.
    const int stage_bytes = (int)S::bytes(WIDF);
    BatchMeta* metas = reinterpret_cast<BatchMeta*>(smem + 2 * stage_bytes);
    int64_t* win = reinterpret_cast<int64_t*>(metas + 3 * SB);
    float* powt = reinterpret_cast<float*>(win + kMaxWin);
    int* kinfo = reinterpret_cast<int*>(powt + 65 * NPAD);
    // PREC: each wave's W_lo fragments [wave][dt][ns][lane]; TW = 1: the group's W fragments
    // [head][dt][ns][lane], one copy that the two waves of a head read
    f16x8* wlo = reinterpret_cast<f16x8*>(kinfo + 4);
#define cdec_of(i) reinterpret_cast<_Float16*>(smem + (i) * stage_bytes)
#define E_of(i) reinterpret_cast<float*>(smem + (i) * stage_bytes + S::EOFF)
#define meta_of(batch) (metas + ((batch) % 3) * SB)

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int c16 = lane & 15;
    const int g = lane >> 4;
    const bool active = wave < (TW == 2 ? hpg : 2 * hpg);
    const int tile0 = TW == 2 ? 0 : wave / hpg;  // the wave's first 16-step tile
    const int hw = TW == 2 ? wave : wave % hpg;  // the wave's head within the group
    const int h = active ? hg * hpg + hw : 0;    // idle waves read head 0 and write nothing
    if constexpr (PREC && NS == 2 && TW == 2) {
        if (!sp.full && split_tiles(a, lane) != CM) return;  // the other instantiation's (uniform)
    }

    // Queries of this lane's steps (lane c16 of step tile tile0 + tt, dims 16 dt + 4 g + i).
    f32x4 qs[TW][DT];
    if constexpr (GQ) {
        // the prologue uses the start of LDS before anything else is staged there
        float* xl = reinterpret_cast<float*>(smem);
        gq_layer_norm<SILU>(a, b, t0, D, xl);
        if (active) gq_project_fwd<HD>(a, h, D, xl, lane, qs);
        __syncthreads();
    }

    flash_setup<NPAD>(a, b, t0, cb, win, powt, kinfo);
    const int kvalid = kinfo[0];
    const int kend = kinfo[1];
    // this part's batches [bi0, bi1)
    const int nball = (kend + SB - 1) / SB;
    const int bi0 = part * nball / sp.ksplit;
    const int bi1 = (part + 1) * nball / sp.ksplit;
    const int x32 = (lane ^ 32) << 2;  // ds_bpermute byte address of lane l ^ 32

    // Gate weights as the A operand: W^T[d = 16 dt + c16][n = 32 ns + 8 g + e] * log2 e.
    // Rows n >= N are zero; their loads read row N - 1 so that all loads issue at once.
    f16x8 wf[TW == 2 ? DT : 1][TW == 2 ? NS : 1];
    if constexpr (TW == 1) {
        if (active && tile0 == 0) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int ns = 0; ns < NS; ++ns) {
                    f16x8 v;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int n = 32 * ns + 8 * g + e;
                        v[e] = (_Float16)(n < a.N ? a.W[(int64_t)n * D + h * HD + 16 * dt + c16] * kLog2e : 0.f);
                    }
                    wlo[((hw * DT + dt) * NS + ns) * 64 + lane] = v;
                }
        }
    } else {
        float wraw[DT][NS][8];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int ns = 0; ns < NS; ++ns)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int n = min(32 * ns + 8 * g + e, a.N - 1);
                    wraw[dt][ns][e] = a.W[(int64_t)n * D + h * HD + 16 * dt + c16];
                }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int ns = 0; ns < NS; ++ns) {
                f16x8 lo;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int n = 32 * ns + 8 * g + e;
                    float ws = n < a.N ? wraw[dt][ns][e] * kLog2e : 0.f;
                    if (PREC) asm volatile("" : "+v"(ws));  // hi and lo of one float32 product
                    wf[dt][ns][e] = (_Float16)ws;
                    lo[e] = (_Float16)(ws - (float)wf[dt][ns][e]);
                }
                // this wave's head's W_lo fragments, read back in the slot loop
                if (PREC) wlo[((wave * DT + dt) * NS + ns) * 64 + lane] = lo;
            }
    }

    // Queries pre-scaled by 1/sqrt(hd).
    const float qscale = 1.0f / sqrtf((float)HD);
    f32x4 o[TW][DT];
    float m[TW], l[TW];
    // the absent slots' mass (score 0, no value) joins part 0's softmax sum
    const float absent = a.v_total >= 0.f && part == 0 ? fmaxf(a.v_total - (float)kvalid, 0.f) : 0.f;
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
        const int t = t0 + 16 * (tile0 + tt) + c16;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 16 * dt + 4 * g + i;
                if constexpr (GQ) {
                    qs[tt][dt][i] = t < a.L ? qs[tt][dt][i] * qscale : 0.f;
                } else {
                    const float* qrow = a.Q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)t * a.q_sl;
                    qs[tt][dt][i] = t < a.L ? qrow[(int64_t)d * a.q_sd] * qscale : 0.f;
                }
                o[tt][dt][i] = 0.f;
            }
        }
        m[tt] = a.v_total >= 0.f ? 0.f : -INFINITY;
        l[tt] = absent;
    }

    Producer<NPAD, SB, MAXI, MAXE> prod;
    // MAXE = 0: the rows go to LDS directly; wait for them before the barrier that publishes them
    auto wait_e_lds = [&]() {
        if constexpr (MAXE == 0) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    };
    if (bi1 > bi0) {
        flash_batch_meta<SB>(a, b, bi0, kend, win, meta_of(bi0));
        if (VR) __syncthreads();  // the load reads the batch's token ids
        prod.template load<VR>(a, b, cbi, bi0, kend, D, col0, WIDF, meta_of(bi0));
        if constexpr (MAXE == 0) prod.template load_e_lds<VR>(a, b, bi0, kend, D, col0, WIDF, meta_of(bi0), E_of(0));
        __syncthreads();
        prod.template store<false, S::CROW, S::TROW, PREC, false, S::CDEC>(t0, cb, powt, meta_of(bi0), cdec_of(0), nullptr, E_of(0), WIDF, CM);
        if (bi0 + 1 < bi1) flash_batch_meta<SB>(a, b, bi0 + 1, kend, win, meta_of(bi0 + 1));
        wait_e_lds();
        __syncthreads();
    }

    for (int bi = bi0; bi < bi1; ++bi) {
        const int cur = (bi - bi0) & 1;
        if (bi + 1 < bi1) {
            prod.template load<VR>(a, b, cbi, bi + 1, kend, D, col0, WIDF, meta_of(bi + 1));
            if constexpr (MAXE == 0)
                prod.template load_e_lds<VR>(a, b, bi + 1, kend, D, col0, WIDF, meta_of(bi + 1), E_of(cur ^ 1));
        }
        const _Float16* cdec = cdec_of(cur);
        const float* E = E_of(cur);
        const BatchMeta* meta = meta_of(bi);
        for (int j = 0; j < SB; ++j) {
            // padding slot (uniform across the workgroup), or a wave without a head
            if (meta[j].u < 0 || !active) continue;
            f16x8 cf[TW][NS];
#pragma unroll
            for (int tt = 0; tt < TW; ++tt)
#pragma unroll
                for (int ns = 0; ns < NS; ++ns)
                    cf[tt][ns] = *reinterpret_cast<const f16x8*>(
                        cdec + (j * kTB + 16 * (tile0 + tt) + c16) * S::CROW + 32 * ns + 8 * g);
            // the slot's e_k / e_v rows, this lane's dims; with one tile per wave read where used
            auto e_row4 = [&](int which, int dt) {
                return *reinterpret_cast<const f32x4*>(E + (j * 2 + which) * WIDF + hw * HD + 16 * dt + 4 * g);
            };
            f32x4 ek[DT], ev[DT];
            if constexpr (TW == 2) {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    ek[dt] = e_row4(0, dt);
                    ev[dt] = e_row4(1, dt);
                }
            }
            f32x4 gt[TW][DT];
#pragma unroll
            for (int tt = 0; tt < TW; ++tt) {
                f16x8 cl[NS];
                if (PREC) {
#pragma unroll
                    for (int ns = 0; ns < NS; ++ns)
                        if ((CM >> ns) & 1)
                            cl[ns] = *reinterpret_cast<const f16x8*>(
                                cdec + S::CDEC + (j * kTB + 16 * (tile0 + tt) + c16) * S::CROW + 32 * ns + 8 * g);
                }
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    if (PREC) {  // small terms first
#pragma unroll
                        for (int ns = 0; ns < NS; ++ns)
                            if ((CM >> ns) & 1)
                                acc = mfma16x16x32(wlo[((wave * DT + dt) * NS + ns) * 64 + lane], cf[tt][ns], acc);
#pragma unroll
                        for (int ns = 0; ns < NS; ++ns)
                            if ((CM >> ns) & 1) acc = mfma16x16x32(wf[dt][ns], cl[ns], acc);
                    }
#pragma unroll
                    for (int ns = 0; ns < NS; ++ns) {
                        if constexpr (TW == 2) acc = mfma16x16x32(wf[dt][ns], cf[tt][ns], acc);
                        else acc = mfma16x16x32(wlo[((hw * DT + dt) * NS + ns) * 64 + lane], cf[tt][ns], acc);
                    }
                    gt[tt][dt] = acc;
                }
            }
            float s[TW];
#pragma unroll
            for (int tt = 0; tt < TW; ++tt) {
                float sacc = 0.f;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const f32x4 ekd = TW == 2 ? ek[dt] : e_row4(0, dt);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float x = gt[tt][dt][i];
                        float gv = x;
                        if (SILU) {
                            const float ex = __builtin_amdgcn_exp2f(-x);
                            gv = x * __builtin_amdgcn_rcpf(1.0f + ex);
                        }
                        gt[tt][dt][i] = gv;
                        sacc = __builtin_fmaf(qs[tt][dt][i], ekd[i] * gv, sacc);
                    }
                }
                // lanes l ^ 16 (ds_swizzle, bitmask mode: and 0x1f, xor 0x10) and l ^ 32
                // (ds_bpermute with a byte address computed once)
                sacc += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(sacc), 0x401F));
                sacc += __int_as_float(__builtin_amdgcn_ds_bpermute(x32, __float_as_int(sacc)));
                s[tt] = sacc;
            }
            // One (rare) rescale branch for both step tiles, so that the softmax and P.V of
            // the two tiles form one block the scheduler can interleave.
            const bool need0 = s[0] > m[0] + kTau;
            const bool need1 = TW == 2 && s[TW - 1] > m[TW - 1] + kTau;
            if (__any(need0 || need1)) {
#pragma unroll
                for (int tt = 0; tt < TW; ++tt) {
                    const float mn = (tt ? need1 : need0) ? s[tt] : m[tt];
                    const float alpha = __builtin_amdgcn_exp2f(m[tt] - mn);
                    l[tt] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) o[tt][dt] *= alpha;
                    m[tt] = mn;
                }
            }
#pragma unroll
            for (int tt = 0; tt < TW; ++tt) {
                const float p = __builtin_amdgcn_exp2f(s[tt] - m[tt]);
                l[tt] += p;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const f32x4 evd = TW == 2 ? ev[dt] : e_row4(1, dt);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[tt][dt][i] = __builtin_fmaf(p, evd[i] * gt[tt][dt][i], o[tt][dt][i]);
                }
            }
            if (a.S2out && g == 0) {
                float* srow = a.S2out + (((int64_t)b * a.H + h) * a.K + bi * SB + j) * a.L;
#pragma unroll
                for (int tt = 0; tt < TW; ++tt) {
                    const int t = t0 + 16 * (tile0 + tt) + c16;
                    if (t < a.L) st_stream(srow + t, s[tt]);
                }
            }
        }
        if (bi + 1 < bi1) {
            prod.template store<false, S::CROW, S::TROW, PREC, false, S::CDEC>(t0, cb, powt, meta_of(bi + 1), cdec_of(cur ^ 1), nullptr,
                                              E_of(cur ^ 1), WIDF, CM);
            if (bi + 2 < bi1) flash_batch_meta<SB>(a, b, bi + 2, kend, win, meta_of(bi + 2));
        }
        wait_e_lds();
        __syncthreads();
    }

    if (sp.ksplit > 1) {  // this part's (o, m, l); flash_fwd_merge_kernel combines the parts
        const int64_t rows = (int64_t)a.B * a.H * a.L;
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) {
            const int t = t0 + 16 * (tile0 + tt) + c16;
            if (t >= a.L || !active) continue;
            const int64_t r = ((int64_t)b * a.H + h) * a.L + t;
            float* prow = sp.part + ((int64_t)part * rows + r) * HD;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(prow + 16 * dt + 4 * g) = o[tt][dt];
            if (g == 0)
                reinterpret_cast<float2*>(sp.part + (int64_t)sp.ksplit * rows * HD)[(int64_t)part * rows + r] =
                    make_float2(m[tt], l[tt]);
        }
        return;
    }
    // O = ln2 * o / l  (the gate carried a factor log2 e), LSE = ln2 * (m + log2 l).
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
        const int t = t0 + 16 * (tile0 + tt) + c16;
        if (t >= a.L || !active) continue;
        const bool any = l[tt] > 0.f;
        const float inv = any ? kLn2 / l[tt] : 0.f;
        float* orow = a.O + (((int64_t)b * a.H + h) * a.L + t) * HD;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const f32x4 v = o[tt][dt] * inv;
            *reinterpret_cast<f32x4*>(orow + 16 * dt + 4 * g) = v;
        }
        if (g == 0)
            a.LSE[((int64_t)b * a.H + h) * a.L + t] = any ? (m[tt] + __log2f(l[tt])) * kLn2 : -INFINITY;
    }
#undef cdec_of
#undef E_of
#undef meta_of
}

// Combines the ksplit partial softmax states of each row (b, h, t): with M = max_p m_p and
// w_p = 2^(m_p - M), l = sum_p w_p l_p, O = ln2 sum_p w_p o_p / l and LSE = ln2 (M + log2 l),
// what one pass over all the slots gives up to the order of the sums.  HD / 4 lanes per
// row, one f32x4 of O each.
template <int HD>
__global__ void __launch_bounds__(256)
flash_fwd_merge_kernel(const float* __restrict__ part, int ks, int64_t rows, float* __restrict__ O,
                       float* __restrict__ LSE) {
    constexpr int LPR = HD / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t r = i / LPR;
    const int c = (int)(i % LPR) * 4;
    if (r >= rows) return;
    const float2* ml = reinterpret_cast<const float2*>(part + (int64_t)ks * rows * HD);
    float M = -INFINITY;
    for (int p = 0; p < ks; ++p) M = fmaxf(M, ml[p * rows + r].x);
    float l = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {  // else no part saw a slot or an absent mass: l stays 0
        for (int p = 0; p < ks; ++p) {
            const float2 v = ml[p * rows + r];
            const float w = __builtin_amdgcn_exp2f(v.x - M);  // 0 for an empty part (m = -inf)
            l += w * v.y;
            o += w * *reinterpret_cast<const f32x4*>(part + (p * rows + r) * HD + c);
        }
    }
    const bool any = l > 0.f;
    const float inv = any ? kLn2 / l : 0.f;
    *reinterpret_cast<f32x4*>(O + r * HD + c) = o * inv;
    if (c == 0) LSE[r] = any ? (M + __log2f(l)) * kLn2 : -INFINITY;
}

// Compute units of the current device (cached per device).
static int device_cus() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256;
    }
    if (cus[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cus[dev] = n;
    }
    return cus[dev];
}

// Slot parts per workgroup of the forward.  The workgroups of one launch run in rounds of
// `conc` (all that the device holds at once) and take about equally long, so G of them
// take ceil(G / conc) rounds: 896 at configuration 2 take 4 rounds of 256 where 3.5 would
// do.  Splitting each workgroup's slot batches into ks parts gives G ks workgroups of
// 1 / ks the length; a split must save at least 3 % (each part repeats the prologue and
// its state goes through the merge) and keep at least four batches per part.
static int fwd_parts(int64_t G, int64_t conc, int nbatch) {
    if (G <= 0 || conc <= 0) return 1;
    int best = 1;
    double best_cost = (double)((G + conc - 1) / conc);
    for (int ks = 2; ks <= 4; ++ks) {
        if (nbatch < 4 * ks) break;
        const double cost = (double)((G * ks + conc - 1) / conc) / ks * (1.0 + 0.02 * (ks - 1));
        if (cost < 0.97 * best_cost) {
            best = ks;
            best_cost = cost;
        }
    }
    return best;
}

// Bytes of the forward's split workspace for ks parts.
static int64_t fwd_part_bytes(int ks, int B, int H, int L, int hd) {
    return ks > 1 ? (int64_t)ks * B * H * L * (hd + 2) * 4 : 0;
}

// The CM = 2 instantiation a default-mode launch adds (two rate tiles), or nullptr.  Without
// the first tile's lo products it has the registers to stage the slot rows itself (ME = 2,
// which every split-gate shape fits: at most 512 columns of three slots over 512 threads)
// instead of by LDS DMA, whose wait at the end of a batch also waits for the batch's score
// stores (forward 11.58 -> 10.85 ms at configuration 2).
template <int HD, int NS, int SB, int MI, int ME, bool SILU, bool VR, bool PREC, bool GQ>
constexpr auto fwd_kernel_cm2() {
    using K = decltype(&flash_ema_fwd_kernel<HD, NS, SB, MI, ME, SILU, VR, PREC, GQ>);
    if constexpr (PREC && NS == 2 && HD <= 64) return (K)&flash_ema_fwd_kernel<HD, NS, SB, MI, 2, SILU, VR, PREC, GQ, 2>;
    else return (K) nullptr;
}

// nfrag: W fragment sets in LDS (PREC: one W_lo set per wave; head_dim 128: one W set per head)
template <int HD, int NS, int SB, bool PREC>
static size_t fwd_lds_bytes(int width, int nfrag) {
    return 2 * Stage<32 * NS, SB, false, PREC, false>::bytes(width) + 3 * SB * sizeof(BatchMeta) + kMaxWin * 8 +
           65 * 32 * NS * 4 + 16 + (size_t)nfrag * (HD / 16) * NS * 64 * 16;
}

// Heads per workgroup: all of them up to hmax (8 with one wave per head, 4 with two), else
// the largest divisor of H that is at most hmax, so that every group is whole.
static int fwd_heads_per_group(int H, int hmax) {
    if (H <= hmax) return H;
    for (int d = hmax; d > 1; --d)
        if (H % d == 0) return d;
    return 1;
}

// Launches the forward (and, when the slot batches are split, the merge).  With ws_need set
// it only plans: *ws_need = the workspace bytes the split wants (0: no split).  A launch
// splits only when `part` holds that many bytes (ws_bytes); otherwise it runs unsplit.
template <int HD, int NS, int SB, bool PREC = false, bool GQ = false, class A = FlashArgsV>
static int launch_fwd(const A& a0, bool vr, hipStream_t st, float* part = nullptr, int64_t ws_bytes = 0,
                      int64_t* ws_need = nullptr, bool full = false) {
    A a = a0;
    constexpr int TW = HD > 64 ? 1 : 2;  // 16-step tiles per wave, as the kernel takes them
    // head_dim 128: up to four heads (eight waves), fewer where their W fragments and
    // staging would not fit in LDS
    int hpg = fwd_heads_per_group(a.H, TW == 2 ? 8 : 4);
    while (TW == 1 && hpg > 1 && fwd_lds_bytes<HD, NS, SB, PREC>(hpg * HD, hpg) > 160 * 1024)
        hpg = fwd_heads_per_group(a.H, hpg - 1);
    a.head_groups = a.H / hpg;
    const int width = hpg * HD;
    // at least four waves, so that the producer's share per thread stays bounded
    const int nwv = TW == 2 ? hpg : 2 * hpg;
    const int nthr = 64 * (nwv < 4 ? 4 : nwv);
    constexpr int NPAD = 32 * NS;
    const int mi = (SB * (kTB / 4) * (NPAD / 4) + nthr - 1) / nthr;
    const int nvec = SB * 2 * (width / 4);
    const int me = (nvec + nthr - 1) / nthr;  // float4 row copies per thread
    size_t lds = fwd_lds_bytes<HD, NS, SB, PREC>(width, PREC ? nthr / 64 : (TW == 1 ? hpg : 0));
    if (GQ) lds = std::max(lds, gq_fwd_lds_bytes(a.H * HD, a.N));
    if (lds > 160 * 1024)
        return fail(MB_ERR_UNSUPPORTED, "mb_flash_ema_fwd: %d heads of %d, N=%d need %zu B of LDS", hpg, HD, a.N, lds);
    const int ntb = (a.L + kTB - 1) / kTB;
    const int64_t G = (int64_t)a.B * ntb * a.head_groups;
    const int64_t rows = (int64_t)a.B * a.H * a.L;
    // the kernels without VR take the base argument block, the GQ ones always FlashArgsG
    // kern2 (or nullptr): the CM = 2 instantiation, launched over the same grid before kern
    auto run = [&](auto kern, const auto& args, decltype(kern) kern2 = nullptr) -> int {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nthr, lds) != hipSuccess || per_cu < 1) {
            (void)hipGetLastError();
            per_cu = 1;
        }
        const int ks = GQ ? 1 : fwd_parts(G, (int64_t)device_cus() * per_cu, (a.K + SB - 1) / SB);
        const int64_t need = fwd_part_bytes(ks, a.B, a.H, a.L, HD);
        if (ws_need) {
            *ws_need = need;
            return MB_OK;
        }
        // two instantiations only when the CM = 2 one exists and its row copy fits (me <= 2);
        // otherwise the one launch corrects every rate tile (sp.full: no workgroup returns)
        const bool two = kern2 && !full && me <= 2;
        const FwdSplit sp{part, (ks > 1 && part && ws_bytes >= need) ? ks : 1, two ? 0 : 1};
        if (two) {
            const int rc2 = launch_with_lds(kern2, dim3(G * sp.ksplit), nthr, lds, st, "mb_flash_ema_fwd", args, sp);
            if (rc2) return rc2;
        }
        const int rc = launch_with_lds(kern, dim3(G * sp.ksplit), nthr, lds, st, "mb_flash_ema_fwd", args, sp);
        if (rc || sp.ksplit == 1) return rc;
        const int64_t threads = rows * (HD / 4);
        hipLaunchKernelGGL(flash_fwd_merge_kernel<HD>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                           (const float*)part, sp.ksplit, rows, a.O, a.LSE);
        return MB_OK;
    };
    const typename FlashArgsK<false, GQ>::type& base = a;
#define MB_FWD(MI, ME)                                                                                       \
    do {                                                                                                     \
        const int rc_ = vr ? (a.silu ? run(flash_ema_fwd_kernel<HD, NS, SB, MI, ME, true, true, PREC, GQ>, a,                 \
                                           fwd_kernel_cm2<HD, NS, SB, MI, ME, true, true, PREC, GQ>())                      \
                                     : run(flash_ema_fwd_kernel<HD, NS, SB, MI, ME, false, true, PREC, GQ>, a,                \
                                           fwd_kernel_cm2<HD, NS, SB, MI, ME, false, true, PREC, GQ>()))                    \
                           : (a.silu ? run(flash_ema_fwd_kernel<HD, NS, SB, MI, ME, true, false, PREC, GQ>, base,             \
                                           fwd_kernel_cm2<HD, NS, SB, MI, ME, true, false, PREC, GQ>())                     \
                                     : run(flash_ema_fwd_kernel<HD, NS, SB, MI, ME, false, false, PREC, GQ>, base,            \
                                           fwd_kernel_cm2<HD, NS, SB, MI, ME, false, false, PREC, GQ>()));                  \
        if (rc_ || ws_need) return rc_;                                                                      \
    } while (0)
    // With the split gate the embedding rows are staged by LDS DMA (ME = 0), which keeps the
    // slot loop out of scratch (the forward at configuration 2: 14 spilled registers with the
    // rows staged through registers, 2 with the DMA; 13.10 -> 12.40 ms).  The single-product
    // gate keeps the register copy: the DMA's wait at the end of a batch (vmcnt(0)) also waits
    // for the batch's score stores, and that forward measured 9.47 -> 9.97 ms with it.
    if (mi > 4 || me > 4)
        return fail(MB_ERR_UNSUPPORTED, "mb_flash_ema_fwd: width %d, N=%d too wide for %d threads", width, a.N, nthr);
    if (PREC) {
        if (mi <= 1) MB_FWD(1, 0);
        else if (mi <= 2) MB_FWD(2, 0);
        else MB_FWD(4, 0);
    } else {
        if (mi <= 1 && me <= 1) MB_FWD(1, 1);
        else if (mi <= 1 && me <= 2) MB_FWD(1, 2);
        else if (mi <= 2 && me <= 2) MB_FWD(2, 2);
        else MB_FWD(4, 4);
    }
#undef MB_FWD
    return check_launch("mb_flash_ema_fwd");
}

}  // namespace mb
