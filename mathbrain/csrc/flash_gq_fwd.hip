// Flash-EMA attention forward with the query gating folded into its prologue:
// mb_flash_ema_fwd_gq computes, per workgroup, Q = q_proj(LayerNorm(x_q * SiLU((C_seq + 1)
// W_pe))) (mathbrain/triton_fused_gating.py:179-197 and model.py:75) in LDS and registers,
// then runs the flash_ema_fwd_kernel slot loop on it.  The gating kernel, the q_proj GEMM
// and Q's round trip through HBM drop out of the forward pass.  (A backward that computed
// Q in-kernel the same way was measured 11 % slower than mb_flash_ema_bwd reading it: its
// 1792 workgroups each stream 512 KB of q_proj.weight; the backward takes Q from a GEMM.)
#include "flash_fwd_kernel.h"

namespace mb {

int flash_validate(const char* who, const FlashArgs& a, int hd);

// The prologue keeps the workgroup's [32, D] x_ln tile in LDS; its q_proj contraction runs
// over D in steps of 32.
constexpr int kGQMaxD = 1024;

static int gq_validate(const char* who, const FlashArgsG& a) {
    const int D = a.H * a.hd;
    MB_REQUIRE(a.xq && a.Wq, "%s: null x_q or q_proj weight", who);
    MB_REQUIRE(a.Cq && a.lnw && a.lnb, "%s: null C_seq or ln_q parameters", who);
    if (D > kGQMaxD || D % 32)
        return fail(MB_ERR_UNSUPPORTED, "%s: d_model %d (supported: multiples of 32 up to %d)", who, D, kGQMaxD);
    MB_REQUIRE(a.xq_sb >= 0 && a.xq_sl >= D, "%s: x rows overlap (step stride %lld < d_model %d)", who,
               (long long)a.xq_sl, D);
    MB_REQUIRE(a.c_sl >= a.N, "%s: C_seq rows overlap (step stride %lld < N %d)", who,
               (long long)a.c_sl, a.N);
    MB_REQUIRE(a.eps > 0.f, "%s: LayerNorm eps %g must be > 0", who, (double)a.eps);
    return MB_OK;
}

}  // namespace mb

using namespace mb;

extern "C" int mb_flash_ema_fwd_gq(const float* x_q, int64_t xq_sb, int64_t xq_sl, const float* C_seq,
                                   int64_t c_sb, int64_t c_sl, const float* ln_w, const float* ln_b,
                                   float eps, const float* W_q, const int64_t* x, int64_t x_sb, int64_t x_sl,
                                   const float* E_k, const float* E_v, const float* W_pe, const float* rhos,
                                   const int64_t* unique, const float* C_bounds, int B, int H, int L, int hd,
                                   int K, int N, int Np, int nc, int Br, int64_t V_total, int flags,
                                   float* O, float* LSE, void* stream) {
    FlashArgsG a{};
    a.xq = x_q; a.xq_sb = xq_sb; a.xq_sl = xq_sl;
    a.Cq = C_seq; a.c_sb = c_sb; a.c_sl = c_sl;
    a.lnw = ln_w; a.lnb = ln_b; a.eps = eps; a.Wq = W_q;
    a.x = x; a.x_sb = x_sb; a.x_sl = x_sl;
    a.Ek = E_k; a.Ev = E_v; a.W = W_pe; a.rhos = rhos; a.unique = unique; a.Cb = C_bounds;
    a.B = B; a.H = H; a.L = L; a.hd = hd; a.K = K; a.N = N; a.Np = Np; a.Br = Br; a.nc = nc;
    a.v_total = (flags & MB_FLASH_ABSENT_MASS) ? (float)V_total : -1.0f;
    a.silu = (flags & MB_FLASH_SILU) ? 1 : 0;
    a.O = O; a.LSE = LSE;
    const bool vr = (flags & MB_FLASH_VOCAB_ROWS) != 0;
    a.e_rows = vr ? V_total : 0;
    int rc = flash_validate("mb_flash_ema_fwd_gq", a, hd);
    if (rc) return rc;
    if (hd > 64) return fail(MB_ERR_UNSUPPORTED, "mb_flash_ema_fwd_gq: head_dim %d (supported: 32, 64)", hd);
    if ((rc = gq_validate("mb_flash_ema_fwd_gq", a))) return rc;
    MB_REQUIRE(!vr || V_total >= 1, "mb_flash_ema_fwd_gq: MB_FLASH_VOCAB_ROWS needs V_total >= 1 rows");
    if (B == 0 || L == 0) return MB_OK;
    MB_REQUIRE(x && rhos && unique && O && LSE && W_pe, "mb_flash_ema_fwd_gq: null pointer");
    MB_REQUIRE(K == 0 || (E_k && E_v && C_bounds), "mb_flash_ema_fwd_gq: null slot pointer");
    hipStream_t st = (hipStream_t)stream;
    const int NS = (N + 31) / 32;
    const int gm = flash_gate_mode("mb_flash_ema_fwd_gq", flags, N, hd);
    if (gm < 0) return gm;
    if (gm > 0) {
        const bool full = gm == 2;  // the fp32 mode corrects every rate tile
        if (hd == 64)
            return NS == 1 ? launch_fwd<64, 1, 4, true, true>(a, vr, st, nullptr, 0, nullptr, full)
                           : launch_fwd<64, 2, 2, true, true>(a, vr, st, nullptr, 0, nullptr, full);
        return NS == 1 ? launch_fwd<32, 1, 4, true, true>(a, vr, st, nullptr, 0, nullptr, full)
                       : launch_fwd<32, 2, 2, true, true>(a, vr, st, nullptr, 0, nullptr, full);
    }
    if (hd == 64) {
        if (NS == 1) return launch_fwd<64, 1, 4, false, true>(a, vr, st);
        if (NS == 2) return launch_fwd<64, 2, 4, false, true>(a, vr, st);
        return launch_fwd<64, 4, 2, false, true>(a, vr, st);
    }
    if (NS == 1) return launch_fwd<32, 1, 4, false, true>(a, vr, st);
    if (NS == 2) return launch_fwd<32, 2, 4, false, true>(a, vr, st);
    return launch_fwd<32, 4, 2, false, true>(a, vr, st);
}
