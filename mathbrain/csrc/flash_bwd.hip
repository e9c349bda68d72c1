// Flash-EMA gated cross-attention backward on gfx950.
//
// Replaces FlashEMAFunction.backward and its kernels _flash_ema_bwd_dq_de and
// _flash_ema_bwd_dw (mathbrain/triton_flash_ema.py:586-650, :250-355, :359-469) with one
// fused pass that recomputes the gate once.  With D_t = dO_t . O_t and, per step t and
// valid slot k,
//   p = exp(s - LSE_t),  dp = dO_t . (e_v * g),  ds = p (dp - D_t)
//   dQ_t  += ds e_k * g / sqrt(hd)          dE_k[k] += ds q_t * g / sqrt(hd)
//   dE_v[k] += p dO_t * g
//   dpre  = (ds q_t * e_k / sqrt(hd) + p dO_t * e_v) * SiLU'(pre)
//   dW_pe[:, h] += c_dec^T dpre             (bf16 operands, fp32 accumulate)
// (the reference's formulas, triton_flash_ema.py:336-350 and :446-465).
//
// Layout: one workgroup per (b, 32-step block, group of 4 heads); wave w takes head
// w % 4 of the group and 16-step half w / 4.  The gate is computed as
// pre[t, d] = c_dec[t, :] W[:, d], so each lane owns one dim d (lane % 16 of a 16-dim
// tile, 4 tiles) and steps 4*(lane/16) + i: the sums over t (dE_k, dE_v, and dW through
// a second MFMA fed from the c_dec tile) stay in registers, dQ accumulates in registers
// across the slot loop, and only the scores s and dp need a sum over the 16 lanes of a
// DPP row.  Each wave adds its 16 steps' dE_k/dE_v of a slot to global memory with one
// coalesced atomic per lane (cheaper, measured, than summing the two half-waves in LDS
// first and flushing once).  dW is added once per wave at the end.
#include "flash_common.h"

#include <algorithm>

namespace mb {

constexpr int kBwdHeads = 4;  // heads per workgroup
// Batch slot info ring: a fast wave writes batch i+2's info while slow waves still read
// batch i's, so at least three entries; four makes the ring index a mask.
constexpr int kMetaRing = 4;
// Default mode: a slot takes the backward's split gate in a wave where the forward's
// probability reaches this at one of the wave's steps (2^-7).
constexpr float kSplitP = 0.0078125f;

__global__ void zero_fill_kernel(float* p, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.f;
}

static int zero_fill(float* p, int64_t n, hipStream_t st) {
    if (n <= 0) return MB_OK;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, st, p, n);
    return check_launch("zero fill");
}

// NTW: the 16-rate tiles of dW_pe a wave accumulates (a 64 x 64 fp32 accumulator is 64
// registers).  XH (N > 64 at head_dim 64, one slot per batch): the rate tiles outnumber what
// a wave holds, so the two half-waves of a head swap their dpre tiles through LDS and each
// multiplies all 32 steps into its own half of the tiles [NTW th, NTW th + NTW).
// VR: E_k / E_v and dE_k / dE_v are vocabulary tables indexed by the slot's token id.
// PG (the default mode's split gate, and the fp32 mode's): the gate GEMM takes fp16 hi + lo
// operand pairs (W_lo c_hi + W_hi c_lo + W_hi c_hi, fp32 accumulation); the producer writes
// the lo tile beside the hi one and W_lo's fragments sit beside W_hi's in LDS.
// PW (MB_FLASH_FP32, with PG): the dW_pe product takes bf16 hi + lo pairs too (dpre_lo c_hi +
// dpre_hi c_lo + dpre_hi c_hi); without PW it takes bf16 c_dec and bf16 dpre.
// SUB (head_dim 128 = 2 HD): a wave takes one 64-dim half ("sub-head") of a head, waves hl
// and hl ^ 1 the two halves of one; everything is per dim except the score and dO . v sums
// (and D = dO . O), which the pair adds through LDS: one barrier per slot.
template <int HD, int NS, int SB, int MAXI, int MAXE, bool SILU, bool HAS_S, int NTW, bool XH, bool VR,
          bool PG = false, bool PW = false, bool SUB = false>
__global__ void __launch_bounds__(512, 1)
flash_ema_bwd_kernel(typename FlashArgsOf<VR>::type a) {
    constexpr int NPAD = 32 * NS;
    constexpr int DT = HD / 16;
    constexpr int WID = kBwdHeads * HD;  // embedding columns of this head group
    // The producer writes a transposed bf16 copy of the counter tile for the dW_pe product
    // (TT) when more than one slot shares a batch or when every wave reads both halves' steps
    // (XH); otherwise the copy costs more on the producer's critical path than the per-wave
    // fp16 -> bf16 conversion it saves (measured), and the waves convert instead.
    constexpr bool TT = SB > 1 || XH || PG;
    static_assert(!XH || SB == 1, "the dpre exchange buffer is reused slot after slot");
    static_assert(!(XH && PG), "the split gate takes N <= 64");
    static_assert(!(SUB && PG), "the split gate takes head_dim <= 64");
    static_assert(!PW || PG, "the split dW_pe product comes with the split gate");
    constexpr int HDR = SUB ? 2 * HD : HD;  // the head's dims
    using S = Stage<NPAD, SB, TT, PG, PW>;
    extern __shared__ __align__(16) unsigned char smem[];

    const int D = a.H * HDR;
    const int ntb = (a.L + kTB - 1) / kTB;
    const int logical = xcd_major(blockIdx.x, gridDim.x);
    const int hg = logical % a.head_groups;
    const int b = logical / (a.head_groups * ntb);
    const int t0 = ((logical / a.head_groups) % ntb) * kTB;
    const int cbi = t0 / a.Br;
    const int cb = cbi * a.Br;

    // LDS: 2 staging buffers (cdec | E | probabilities [SB][heads][kTB]) | W fragments |
    // meta ring | window | power table | slot info
    constexpr int SCN = HAS_S ? SB * kBwdHeads * kTB : 0;  // staged probabilities per buffer
    static_assert(SCN <= 2 * kBwdHeads * 64, "one staged score per thread");
    const int stage_bytes = (int)S::bytes(WID) + SCN * 4;
    f16x8* wfr = reinterpret_cast<f16x8*>(smem + 2 * stage_bytes);
    f16x8* wfl = wfr + kBwdHeads * DT * NS * 64;  // PG: the W_lo fragments
    BatchMeta* metas = reinterpret_cast<BatchMeta*>(wfr + (PG ? 2 : 1) * kBwdHeads * DT * NS * 64);
    int64_t* win = reinterpret_cast<int64_t*>(metas + kMetaRing * SB);
    float* powt = reinterpret_cast<float*>(win + kMaxWin);
    int* kinfo = reinterpret_cast<int*>(powt + 65 * NPAD);
    bf16x4* xbuf = reinterpret_cast<bf16x4*>(kinfo + 4);  // XH: [head][half][DT][64 lanes]
    // SUB: the sub-heads' partial sums, [exchange parity][sub-head][half][2 sums][16 steps]
    float* pbuf = reinterpret_cast<float*>(xbuf + (XH ? kBwdHeads * 2 * DT * 64 : 0));
#define cdec_of(i) reinterpret_cast<_Float16*>(smem + (i) * stage_bytes)
#define cdecT_of(i) reinterpret_cast<__bf16*>(smem + (i) * stage_bytes + S::CTOFF)
#define E_of(i) reinterpret_cast<float*>(smem + (i) * stage_bytes + S::EOFF)
#define S2_of(i) (E_of(i) + SB * 2 * WID)
#define meta_of(batch) (metas + ((batch) % kMetaRing) * SB)

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int c16 = lane & 15;
    const int g = lane >> 4;
    const int hl = wave & 3;
    const int th = wave >> 2;
    // a group holds hpg <= 4 heads (hpg divides H; with SUB, hpg sub-heads of hpg / 2 heads);
    // waves of the missing heads only help stage and synchronise, and read head 0 for their
    // (unused) setup
    const int hpg = (SUB ? 2 : 1) * (a.H / a.head_groups);
    const bool active = hl < hpg;
    const int h = active ? (SUB ? hg * (hpg >> 1) + (hl >> 1) : hg * hpg + hl) : 0;
    const int sub0 = SUB ? (hl & 1) * HD : 0;  // the wave's first dim within head h
    // SUB: adds the partner sub-head's values of this wave's 16 steps (v[i], w[i]: step
    // 4 g + i, equal over the lanes of a row) through pbuf.  Every wave of the group makes
    // the same exchanges, so the areas alternate with them: an area is written again only
    // after the next exchange's barrier, when both waves have read it.
    int xpar = 0;
    auto pair_sum = [&](float (&v)[4], float (&w)[4]) {
        float* mine = pbuf + ((xpar * kBwdHeads + hl) * 2 + th) * 32;
        const float* other = pbuf + ((xpar * kBwdHeads + (hl ^ 1)) * 2 + th) * 32;
        xpar ^= 1;
        if (active && c16 == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                mine[4 * g + i] = v[i];
                mine[16 + 4 * g + i] = w[i];
            }
        }
        __syncthreads();
        if (active) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] += other[4 * g + i];
                w[i] += other[16 + 4 * g + i];
            }
        }
    };

    // The default mode's split gate is the forward's, whose lo products cover only the rate
    // tiles split_tiles picks: the other tiles' W_lo fragments and c_lo entries are zeros here,
    // so that a split slot's gate (and with recomputed scores, its scores) are the forward's.
    // The fp32 mode splits every tile.
    int ctile = 3;
    if constexpr (PG && !PW && NS == 2) ctile = split_tiles(a, lane);

    // Gate weights as the B operand: W[n = 32 ns + 8 g + e][d = 16 dt + c16] * log2 e,
    // one fragment per (head, dt, ns, lane) in LDS.
    // Rows n >= N are zero; their loads read row N - 1 so that all loads issue at once.
    for (int f = threadIdx.x; f < kBwdHeads * DT * NS * 64; f += blockDim.x) {
        const int ln = f & 63;
        const int ns = (f >> 6) % NS;
        const int dt = ((f >> 6) / NS) % DT;
        const int hh = (f >> 6) / (NS * DT);
        float w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int n = min(32 * ns + 8 * (ln >> 4) + e, a.N - 1);
            w[e] = a.W[(int64_t)n * D + (hh < hpg ? hg * hpg + hh : 0) * HD + 16 * dt + (ln & 15)];
        }
        f16x8 v, vl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int n = 32 * ns + 8 * (ln >> 4) + e;
            float ws = n < a.N ? w[e] * kLog2e : 0.f;
            if (PG) asm volatile("" : "+v"(ws));  // hi and lo of one float32 product
            v[e] = (_Float16)ws;
            vl[e] = (_Float16)(ws - (float)v[e]);
        }
        wfr[f] = v;
        if (PG) wfl[f] = (ctile >> ns) & 1 ? vl : f16x8{};
    }
    flash_setup<NPAD>(a, b, t0, cb, win, powt, kinfo);
    const int kend = kinfo[1];
    const int nb = (kend + SB - 1) / SB;

    // Per-lane rows: steps t = t0 + 16 th + 4 g + i, dims d = 16 dt + c16 of head h.
    const float qscale = 1.0f / sqrtf((float)HDR);
    float qs[DT][4], dov[DT][4], dq[DT][4];
    float lse2[4], Dv[4];
    {
        float dsum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = t0 + 16 * th + 4 * g + i;
            const bool ok = t < a.L;
            const int64_t qoff = (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)t * a.q_sl;
            const int64_t ooff = (((int64_t)b * a.H + h) * a.L + t) * HDR;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int d = sub0 + 16 * dt + c16;
                qs[dt][i] = ok ? a.Q[qoff + (int64_t)d * a.q_sd] * qscale : 0.f;
                dov[dt][i] = ok ? a.dO[qoff + (int64_t)d * a.q_sd] : 0.f;
                dq[dt][i] = 0.f;
                if (ok) dsum[i] = __builtin_fmaf(dov[dt][i], a.Oin[ooff + d], dsum[i]);
            }
            lse2[i] = ok ? a.LSEin[((int64_t)b * a.H + h) * a.L + t] * kLog2e : INFINITY;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) Dv[i] = row_sum16(dsum[i]);
        if (SUB) pair_sum(Dv, dsum);  // (dsum's partner values are not used)
    }
    f32x4 dWacc[DT][NTW];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) dWacc[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    Producer<NPAD, SB, MAXI, MAXE> prod;
    const int col0 = hg * hpg * HD;  // WID columns from here are staged (zeros past D)
    // Forward scores of a batch, one float per thread (SCN <= blockDim.x): one register held
    // across the slot loop, not four.  The thread's (head, step) is the same in every batch,
    // so its LSE is read once, and the staged value is the probability p = 2^(s2 - lse2):
    // one exp per (step, slot, head) here instead of one in each of the 16 lanes (dims) of
    // a row that needs it; the same operation on the same operands as in the lanes.
    float s2pre = 0.f;
    float lse2s = INFINITY;
    if (HAS_S && (int)threadIdx.x < SCN) {
        const int hh = (threadIdx.x / kTB) % kBwdHeads;
        const int t = t0 + threadIdx.x % kTB;
        const int hs = SUB ? hg * (hpg >> 1) + (hh >> 1) : hg * hpg + hh;
        if (t < a.L && hh < hpg) lse2s = a.LSEin[((int64_t)b * a.H + hs) * a.L + t] * kLog2e;
    }
    auto load_scores = [&](int batch) {
        if (!HAS_S || (int)threadIdx.x >= SCN) return;
        const int j = threadIdx.x / (kBwdHeads * kTB);
        const int hh = (threadIdx.x / kTB) % kBwdHeads;
        const int t = t0 + threadIdx.x % kTB;
        const int k = batch * SB + j;
        const int hs = SUB ? hg * (hpg >> 1) + (hh >> 1) : hg * hpg + hh;  // the scores' head
        s2pre = (k < kend && t < a.L && hh < hpg)
                    ? a.S2in[(((int64_t)b * a.H + hs) * a.K + k) * a.L + t]
                    : 0.f;
    };
    auto store_scores = [&](float* dst) {
        if (HAS_S && (int)threadIdx.x < SCN) dst[threadIdx.x] = __builtin_amdgcn_exp2f(s2pre - lse2s);
    };
    // MAXE = 0: the rows go to LDS directly; wait for them before the barrier that publishes them
    auto wait_e_lds = [&]() {
        if constexpr (MAXE == 0) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    };
    if (nb > 0) {
        flash_batch_meta<SB>(a, b, 0, kend, win, meta_of(0));
        if (VR) __syncthreads();  // the load reads the batch's token ids
        prod.template load<VR>(a, b, cbi, 0, kend, D, col0, WID, meta_of(0));
        if constexpr (MAXE == 0) prod.template load_e_lds<VR>(a, b, 0, kend, D, col0, WID, meta_of(0), E_of(0));
        load_scores(0);
        __syncthreads();
        store_scores(S2_of(0));
        prod.template store<TT, S::CROW, S::TROW, PG, PW, S::CDEC, S::CT>(t0, cb, powt, meta_of(0), cdec_of(0), cdecT_of(0), E_of(0), WID,
                                                                     ctile);
        if (nb > 1) flash_batch_meta<SB>(a, b, 1, kend, win, meta_of(1));
        wait_e_lds();
        __syncthreads();
    }

    for (int bi = 0; bi < nb; ++bi) {
        const int cur = bi & 1;
        if (bi + 1 < nb) {
            prod.template load<VR>(a, b, cbi, bi + 1, kend, D, col0, WID, meta_of(bi + 1));
            if constexpr (MAXE == 0)
                prod.template load_e_lds<VR>(a, b, bi + 1, kend, D, col0, WID, meta_of(bi + 1), E_of(cur ^ 1));
            load_scores(bi + 1);
        }
        const _Float16* cdec = cdec_of(cur);
        const float* E = E_of(cur);
        const BatchMeta* meta = meta_of(bi);
        for (int j = 0; j < SB; ++j) {
            if (meta[j].u < 0) continue;  // padding slot (uniform across the workgroup)
            if (!active) {                // a wave without a head: only the exchange barriers
                if (SUB) {
                    float unused[4] = {0.f, 0.f, 0.f, 0.f};
                    pair_sum(unused, unused);
                }
                if (XH) __syncthreads();
                continue;
            }
            // Probabilities of this lane's 4 steps, staged in LDS with the batch.
            f32x4 s2v = {0.f, 0.f, 0.f, 0.f};
            if (HAS_S)
                s2v = *reinterpret_cast<const f32x4*>(S2_of(cur) + (j * kBwdHeads + hl) * kTB + 16 * th + 4 * g);
            const _Float16* crow = cdec + (j * kTB + 16 * th) * S::CROW;
            f16x8 cf[NS];
#pragma unroll
            for (int ns = 0; ns < NS; ++ns)
                cf[ns] = *reinterpret_cast<const f16x8*>(crow + c16 * S::CROW + 32 * ns + 8 * g);
            float ek[DT], ev[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                ek[dt] = E[(j * 2 + 0) * WID + hl * HD + 16 * dt + c16];
                ev[dt] = E[(j * 2 + 1) * WID + hl * HD + 16 * dt + c16];
            }
            // The split gate where this slot carries weight: every gradient term of the slot
            // has a factor p (dE_v, and ds = p (dp - D) in dQ, dE_k and dpre), so where the
            // forward's probability stays below kSplitP at all of the wave's 16 steps the
            // single fp16 product's rounding is scaled down by it (the fp32 mode, and the
            // recomputed scores, whose p comes after the gate, always split).  The split is
            // the forward's (ctile).
            bool split = PG;
            if constexpr (PG && !PW && HAS_S)
                split = __any(fmaxf(fmaxf(s2v[0], s2v[1]), fmaxf(s2v[2], s2v[3])) >= kSplitP);
            f32x4 g2[DT], sg[DT];
            if (split) {
                f16x8 cfl[NS];
#pragma unroll
                for (int ns = 0; ns < NS; ++ns)
                    cfl[ns] = *reinterpret_cast<const f16x8*>(crow + S::CDEC + c16 * S::CROW + 32 * ns + 8 * g);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    f32x4 accg = {0.f, 0.f, 0.f, 0.f};  // small terms first
#pragma unroll
                    for (int ns = 0; ns < NS; ++ns)
                        accg = mfma16x16x32(cf[ns], wfl[((hl * DT + dt) * NS + ns) * 64 + lane], accg);
#pragma unroll
                    for (int ns = 0; ns < NS; ++ns)
                        accg = mfma16x16x32(cfl[ns], wfr[((hl * DT + dt) * NS + ns) * 64 + lane], accg);
#pragma unroll
                    for (int ns = 0; ns < NS; ++ns)
                        accg = mfma16x16x32(cf[ns], wfr[((hl * DT + dt) * NS + ns) * 64 + lane], accg);
                    g2[dt] = accg;
                }
            } else {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    f32x4 accg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ns = 0; ns < NS; ++ns)
                        accg = mfma16x16x32(cf[ns], wfr[((hl * DT + dt) * NS + ns) * 64 + lane], accg);
                    g2[dt] = accg;
                }
            }
            // Phase 1: gate, score and dO . v partial sums over this lane's dims.
            float s[4] = {0.f, 0.f, 0.f, 0.f}, dp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float x = g2[dt][i];  // pre * log2 e
                    float sig = 1.f, gv = x;
                    if (SILU) {
                        sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x));
                        gv = x * sig;
                    }
                    g2[dt][i] = gv;  // g * log2 e
                    sg[dt][i] = sig;
                    if (!HAS_S) s[i] = __builtin_fmaf(qs[dt][i] * ek[dt], gv, s[i]);
                    dp[i] = __builtin_fmaf(dov[dt][i] * ev[dt], gv, dp[i]);
                }
            if (SUB) {  // the head's sums over both sub-heads
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (!HAS_S) s[i] = row_sum16(s[i]);
                    dp[i] = row_sum16(dp[i]);
                }
                pair_sum(s, dp);
            }
            // The 16 lanes' sums (dims), both quantities' chains interleaved (the fp32 mode
            // keeps one chain after the other: interleaved, its larger live set spills).
            if (!SUB && PW) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (!HAS_S) s[i] = row_sum16(s[i]);
                    dp[i] = row_sum16(dp[i]);
                }
            } else if (!SUB) {
                if (HAS_S) {
                    row_sum16_n(dp);
                } else {
                    float sd[8] = {s[0], s[1], s[2], s[3], dp[0], dp[1], dp[2], dp[3]};
                    row_sum16_n(sd);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        s[i] = sd[i];
                        dp[i] = sd[4 + i];
                    }
                }
            }
            float p[4], ds[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float dpt = dp[i] * kLn2;  // dO . v
                p[i] = HAS_S ? s2v[i] : __builtin_amdgcn_exp2f(s[i] - lse2[i]);  // s: score * log2 e
                ds[i] = p[i] * (dpt - Dv[i]);
            }
            // Phase 2: gradients.  With xq = ds q, yd = p dO:
            //   dE_k += xq g, dE_v += yd g, dQ += ds g e_k,
            //   dpre = (xq e_k + yd e_v) SiLU'(pre),  SiLU' = sig + g (1 - sig).
            float dEk[DT], dEv[DT];
            bf16x4 dpre[DT], dprel[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                dEk[dt] = 0.f;
                dEv[dt] = 0.f;
                float dvv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float gv = g2[dt][i];
                    const float xq = ds[i] * qs[dt][i];
                    const float yd = p[i] * dov[dt][i];
                    dEk[dt] = __builtin_fmaf(xq, gv, dEk[dt]);
                    dEv[dt] = __builtin_fmaf(yd, gv, dEv[dt]);
                    dq[dt][i] = __builtin_fmaf(ds[i] * gv, ek[dt], dq[dt][i]);
                    const float av = __builtin_fmaf(xq, ek[dt], yd * ev[dt]);
                    float dsil = 1.f;
                    if (SILU) {  // sig + g (1 - sig), with g = gv ln2
                        const float sig = sg[dt][i];
                        dsil = __builtin_fmaf(gv, __builtin_fmaf(-kLn2, sig, kLn2), sig);
                    }
                    dvv[i] = av * dsil;
                }
                if (PW) {  // bf16 hi + lo of each value
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        dpre[dt][i] = (__bf16)dvv[i];
                        dprel[dt][i] = (__bf16)(dvv[i] - (float)dpre[dt][i]);
                    }
                } else {  // two values per conversion
                    const bf16x2 d01 = cvt_pk_bf16(dvv[0], dvv[1]);
                    const bf16x2 d23 = cvt_pk_bf16(dvv[2], dvv[3]);
                    dpre[dt] = bf16x4{d01[0], d01[1], d23[0], d23[1]};
                }
            }
            // dE: this lane's 4 steps summed in registers; the 4 row groups (other steps)
            // are reduce-scattered with v_permlane16/32_swap so that row g holds dim tile g
            // (DT = 4) or rows 0 and 2 hold tiles 0 and 1 (DT = 2); one atomic per lane.
            const int64_t slot_row = VR ? min(meta[j].u, e_rows_of(a) - 1) : (int64_t)b * a.K + bi * SB + j;
            const int64_t erow = slot_row * D + col0 + hl * HD;
            if (DT == 4) {
                const float vk = rows4_reduce_scatter(dEk[0], dEk[1 % DT], dEk[2 % DT], dEk[3 % DT]);
                const float vv = rows4_reduce_scatter(dEv[0], dEv[1 % DT], dEv[2 % DT], dEv[3 % DT]);
                atomicAdd(a.dEk + erow + 16 * g + c16, vk * kLn2);
                atomicAdd(a.dEv + erow + 16 * g + c16, vv * kLn2);
            } else {
                const float vk = rows4_reduce_scatter2(dEk[0], dEk[1 % DT]);
                const float vv = rows4_reduce_scatter2(dEv[0], dEv[1 % DT]);
                if ((g & 1) == 0) {
                    atomicAdd(a.dEk + erow + 8 * g + c16, vk * kLn2);
                    atomicAdd(a.dEv + erow + 8 * g + c16, vv * kLn2);
                }
            }
            // dW^T[d, n] += dpre^T[d, t] c_dec[t, n]: A = dpre (rows d, k = 4 steps of a lane),
            // B = c_dec[t = 16 half + 4 g + e][n = 16 nt + c16]: one 8-byte read of the
            // transposed bf16 tile, or four 16-bit reads of a column of the fp16 tile converted
            // to bf16 (dpre needs bf16's range, so the product is bf16).
            auto cop = [&](int half, int ntg) {
                bf16x4 cb4;
                if (TT) {
                    const __bf16* ccol = cdecT_of(cur) + (j * NPAD + c16) * S::TROW + 16 * half + 4 * g;
                    cb4 = *reinterpret_cast<const bf16x4*>(ccol + 16 * ntg * S::TROW);
                } else {
                    const _Float16* ccol = cdec + (j * kTB + 16 * half + 4 * g) * S::CROW + c16;
#pragma unroll
                    for (int e = 0; e < 4; ++e) cb4[e] = (__bf16)(float)ccol[e * S::CROW + 16 * ntg];
                }
                return cb4;
            };
            if (XH) {
                bf16x4* mine = xbuf + (hl * 2 + th) * DT * 64 + lane;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) mine[dt * 64] = dpre[dt];
                __syncthreads();  // uniform: every wave takes the same slots
                const bf16x4* other = xbuf + (hl * 2 + (th ^ 1)) * DT * 64 + lane;
                bf16x4 dpo[DT];
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) dpo[dt] = other[dt * 64];
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt) {
                    const bf16x4 co = cop(th, NTW * th + nt);
                    const bf16x4 cx = cop(th ^ 1, NTW * th + nt);
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) {
                        dWacc[dt][nt] = mfma16x16x16(dpre[dt], co, dWacc[dt][nt]);
                        dWacc[dt][nt] = mfma16x16x16(dpo[dt], cx, dWacc[dt][nt]);
                    }
                }
            } else {
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt) {
                    const bf16x4 cb4 = cop(th, nt);
                    if (PW) {  // small terms first; the lo tile sits S::CT entries after the hi one
                        const __bf16* ccol = cdecT_of(cur) + S::CT + (j * NPAD + c16) * S::TROW + 16 * th + 4 * g;
                        const bf16x4 cl4 = *reinterpret_cast<const bf16x4*>(ccol + 16 * nt * S::TROW);
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) {
                            dWacc[dt][nt] = mfma16x16x16(dprel[dt], cb4, dWacc[dt][nt]);
                            dWacc[dt][nt] = mfma16x16x16(dpre[dt], cl4, dWacc[dt][nt]);
                        }
                    }
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) dWacc[dt][nt] = mfma16x16x16(dpre[dt], cb4, dWacc[dt][nt]);
                }
            }
        }
        if (bi + 1 < nb) {
            prod.template store<TT, S::CROW, S::TROW, PG, PW, S::CDEC, S::CT>(t0, cb, powt, meta_of(bi + 1), cdec_of(cur ^ 1), cdecT_of(cur ^ 1),
                                                E_of(cur ^ 1), WID, ctile);
            store_scores(S2_of(cur ^ 1));
            if (bi + 2 < nb) flash_batch_meta<SB>(a, b, bi + 2, kend, win, meta_of(bi + 2));
        }
        wait_e_lds();
        __syncthreads();
    }

    // dQ (the gate carried log2 e, the query 1/sqrt(hd)) and dW.
    const float qf = kLn2 * qscale;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = t0 + 16 * th + 4 * g + i;
        if (t >= a.L || !active) continue;
        float* dst = a.dQ + (((int64_t)b * a.H + h) * a.L + t) * HDR + sub0;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) dst[16 * dt + c16] = dq[dt][i] * qf;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            const int n = 16 * ((XH ? NTW * th : 0) + nt) + c16;
            if (n >= a.N || !active) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                atomicAdd(&a.dW[(int64_t)n * D + h * HDR + sub0 + 16 * dt + 4 * g + i], dWacc[dt][nt][i]);
        }
#undef cdec_of
#undef cdecT_of
#undef E_of
#undef S2_of
#undef meta_of
}

template <int HD, int NS, int SB, bool XH, bool PG, bool PW, bool SUB = false>
static size_t bwd_lds_bytes() {
    constexpr int WID = kBwdHeads * HD;
    return 2 * (Stage<32 * NS, SB, (SB > 1 || XH || PG), PG, PW>::bytes(WID) + (size_t)SB * kBwdHeads * kTB * 4) +
           (size_t)(PG ? 2 : 1) * kBwdHeads * (HD / 16) * NS * 64 * 16 + kMetaRing * SB * sizeof(BatchMeta) +
           kMaxWin * 8 + 65 * 32 * NS * 4 + 16 + (XH ? (size_t)kBwdHeads * 2 * (HD / 16) * 64 * 8 : 0) +
           (SUB ? (size_t)2 * kBwdHeads * 2 * 32 * 4 : 0);
}

template <int HD, int NS, int SB, bool PG = false, bool PW = false, bool SUB = false>
static int launch_bwd(const FlashArgsV& a0, bool vr, hipStream_t st) {
    FlashArgsV a = a0;
    // heads per group: the largest divisor of H that is at most four (with SUB two heads,
    // whose four sub-heads take the four wave pairs)
    int hpg = 1;
    for (int d = SUB ? kBwdHeads / 2 : kBwdHeads; d > 1; --d)
        if (a.H % d == 0) { hpg = d; break; }
    a.head_groups = a.H / hpg;
    constexpr int NPAD = 32 * NS;
    constexpr int WID = kBwdHeads * HD;
    const int nthr = 64 * 2 * kBwdHeads;
    const int mi = (SB * (kTB / 4) * (NPAD / 4) + nthr - 1) / nthr;
    const int me = (SB * 2 * (WID / 4) + nthr - 1) / nthr;
    // dW_pe tiles per wave: a DT x NTW block of 16x16 fp32 accumulators stays at 64
    // registers; twice that many tiles take the half-wave dpre exchange (XH).
    constexpr int NT = NPAD / 16;
    constexpr int NTW = NT < 256 / HD ? NT : 256 / HD;
    constexpr bool XH = NT > NTW;
    static_assert(NT == NTW || NT == 2 * NTW, "at most two half-waves per head");
    const size_t lds = bwd_lds_bytes<HD, NS, SB, XH, PG, PW, SUB>();
    if (lds > 160 * 1024)
        return fail(MB_ERR_UNSUPPORTED, "mb_flash_ema_bwd: hd=%d, N=%d needs %zu B of LDS", HD, a.N, lds);
    const int ntb = (a.L + kTB - 1) / kTB;
    dim3 grid(a.B * ntb * a.head_groups);
#define MB_BWD_PICK(MI, ME, VR)                                                                  \
    (a.S2in ? (a.silu ? flash_ema_bwd_kernel<HD, NS, SB, MI, ME, true, true, NTW, XH, VR, PG, PW, SUB>       \
                      : flash_ema_bwd_kernel<HD, NS, SB, MI, ME, false, true, NTW, XH, VR, PG, PW, SUB>)     \
            : (a.silu ? flash_ema_bwd_kernel<HD, NS, SB, MI, ME, true, false, NTW, XH, VR, PG, PW, SUB>      \
                      : flash_ema_bwd_kernel<HD, NS, SB, MI, ME, false, false, NTW, XH, VR, PG, PW, SUB>))
    const FlashArgs& base = a;
#define MB_BWD(MI, ME)                                                                            \
    do {                                                                                          \
        const int rc_ = vr ? launch_with_lds(MB_BWD_PICK(MI, ME, true), grid, nthr, lds, st,        \
                                             "mb_flash_ema_bwd", a)                               \
                           : launch_with_lds(MB_BWD_PICK(MI, ME, false), grid, nthr, lds, st,       \
                                             "mb_flash_ema_bwd", base);                           \
        if (rc_) return rc_;                                                                      \
    } while (0)
    // The embedding rows go through registers (ME >= 1).  Staging them by LDS DMA (ME = 0, as
    // the split-gate forward does) needs a vmcnt(0) wait before each batch's barrier, which
    // also waits for the batch's dE atomics: 24.91 -> 25.31 ms at configuration 2.
    if (mi <= 1 && me <= 1) MB_BWD(1, 1);
    else if (mi <= 2 && me <= 1) MB_BWD(2, 1);
    else if (mi <= 2 && me <= 2) MB_BWD(2, 2);
    else return fail(MB_ERR_UNSUPPORTED, "mb_flash_ema_bwd: N=%d too wide", a.N);
#undef MB_BWD
#undef MB_BWD_PICK
    return check_launch("mb_flash_ema_bwd");
}

int flash_validate(const char* who, const FlashArgs& a, int hd);

}  // namespace mb

using namespace mb;

extern "C" int mb_flash_ema_bwd(const float* Q, int64_t q_sb, int64_t q_sh, int64_t q_sl,
                                int64_t q_sd, const float* dO, const int64_t* x, int64_t x_sb,
                                int64_t x_sl, const float* E_k, const float* E_v,
                                const float* W_pe, const float* rhos, const int64_t* unique,
                                const float* C_bounds, const float* O, const float* LSE, int B,
                                int H, int L, int hd, int K, int N, int Np, int nc, int Br,
                                int64_t V_total, int flags, const float* scores, float* dQ,
                                float* dE_k, float* dE_v, float* dW_pe, void* stream) {
    FlashArgsV a{};
    a.Q = Q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_sl = q_sl; a.q_sd = q_sd;
    a.dO = dO; a.x = x; a.x_sb = x_sb; a.x_sl = x_sl;
    a.Ek = E_k; a.Ev = E_v; a.W = W_pe; a.rhos = rhos; a.unique = unique; a.Cb = C_bounds;
    a.Oin = O; a.LSEin = LSE;
    a.B = B; a.H = H; a.L = L; a.hd = hd; a.K = K; a.N = N; a.Np = Np; a.Br = Br; a.nc = nc;
    a.v_total = (flags & MB_FLASH_ABSENT_MASS) ? (float)V_total : -1.0f;
    a.silu = (flags & MB_FLASH_SILU) ? 1 : 0;
    a.dQ = dQ; a.dEk = dE_k; a.dEv = dE_v; a.dW = dW_pe;
    a.S2in = scores;
    const bool vr = (flags & MB_FLASH_VOCAB_ROWS) != 0;
    a.e_rows = vr ? V_total : 0;
    int rc = flash_validate("mb_flash_ema_bwd", a, hd);
    if (rc) return rc;
    MB_REQUIRE(!vr || V_total >= 1, "mb_flash_ema_bwd: MB_FLASH_VOCAB_ROWS needs V_total >= 1 rows");
    // dE_k, dE_v and dW_pe are accumulated with atomics, so they are cleared first -- also
    // when there is no step to accumulate (B or L zero), which leaves them zero; every dQ
    // element is written once.
    const int64_t D = (int64_t)H * hd;
    const int64_t erows = K > 0 ? (vr ? V_total : (int64_t)B * K) : 0;
    MB_REQUIRE(dW_pe, "mb_flash_ema_bwd: null dW_pe");
    MB_REQUIRE(erows == 0 || (dE_k && dE_v), "mb_flash_ema_bwd: null dE_k / dE_v");
    hipStream_t st = (hipStream_t)stream;
    if ((rc = zero_fill(dW_pe, (int64_t)N * D, st))) return rc;
    if (erows > 0) {
        if ((rc = zero_fill(dE_k, erows * D, st))) return rc;
        if ((rc = zero_fill(dE_v, erows * D, st))) return rc;
    }
    if (B == 0 || L == 0) return MB_OK;
    MB_REQUIRE(Q && dO && x && rhos && unique && O && LSE && W_pe && dQ,
               "mb_flash_ema_bwd: null pointer");
    MB_REQUIRE(K == 0 || (E_k && E_v && C_bounds), "mb_flash_ema_bwd: null slot pointer");
    const int NS = (N + 31) / 32;
    const int gm = flash_gate_mode("mb_flash_ema_bwd", flags, N, hd);
    if (gm < 0) return gm;
    if (gm == 2) {
        // hi + lo tiles of both kinds and both W fragment sets in LDS: one slot per batch
        if (hd == 64) return NS == 1 ? launch_bwd<64, 1, 1, true, true>(a, vr, st) : launch_bwd<64, 2, 1, true, true>(a, vr, st);
        return NS == 1 ? launch_bwd<32, 1, 1, true, true>(a, vr, st) : launch_bwd<32, 2, 1, true, true>(a, vr, st);
    }
    if (gm == 1) {  // the gate's lo tile and W_lo beside the hi ones
        if (hd == 64) return NS == 1 ? launch_bwd<64, 1, 4, true>(a, vr, st) : launch_bwd<64, 2, 2, true>(a, vr, st);
        return NS == 1 ? launch_bwd<32, 1, 4, true>(a, vr, st) : launch_bwd<32, 2, 2, true>(a, vr, st);
    }
    if (hd == 128) {  // two 64-dim sub-heads per head
        if (NS == 1) return launch_bwd<64, 1, 4, false, false, true>(a, vr, st);
        if (NS == 2) return launch_bwd<64, 2, 4, false, false, true>(a, vr, st);
        return launch_bwd<64, 4, 1, false, false, true>(a, vr, st);
    }
    if (hd == 64) {
        if (NS == 1) return launch_bwd<64, 1, 4>(a, vr, st);
        if (NS == 2) return launch_bwd<64, 2, 4>(a, vr, st);
        return launch_bwd<64, 4, 1>(a, vr, st);
    }
    if (NS == 1) return launch_bwd<32, 1, 4>(a, vr, st);
    if (NS == 2) return launch_bwd<32, 2, 4>(a, vr, st);
    return launch_bwd<32, 4, 2>(a, vr, st);
}
