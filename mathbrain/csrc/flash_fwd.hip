// Flash-EMA gated cross-attention forward on gfx950: the entry point mb_flash_ema_fwd (the
// kernel itself is in flash_fwd_kernel.h).
#include "flash_fwd_kernel.h"

namespace mb {

// Host-side validation shared with the backward entry point.
int flash_validate(const char* who, const FlashArgs& a, int hd) {
    MB_REQUIRE(a.B >= 0 && a.L >= 0 && a.K >= 0, "%s: negative B=%d, L=%d or K=%d", who, a.B, a.L, a.K);
    MB_REQUIRE(a.H >= 1, "%s: H=%d must be >= 1", who, a.H);
    MB_REQUIRE(a.N >= 1 && a.Np >= a.N, "%s: need 1 <= N=%d <= Np=%d", who, a.N, a.Np);
    if (hd != 32 && hd != 64 && hd != 128)
        return fail(MB_ERR_UNSUPPORTED, "%s: head_dim %d (supported: 32, 64, 128)", who, hd);
    if (a.H > 64) return fail(MB_ERR_UNSUPPORTED, "%s: %d heads (supported: 1..64)", who, a.H);
    if (a.N > 128) return fail(MB_ERR_UNSUPPORTED, "%s: N=%d > 128", who, a.N);
    MB_REQUIRE(a.Br >= 1, "%s: Br=%d must be >= 1", who, a.Br);
    if (!(a.Br <= 32 || a.Br == 64))
        return fail(MB_ERR_UNSUPPORTED, "%s: Br=%d (supported: <= 32 or 64)", who, a.Br);
    const int nc_need = a.L > 0 ? (a.L + a.Br - 1) / a.Br : 1;
    MB_REQUIRE(a.nc >= nc_need, "%s: C_bounds has %d chunks, L=%d with Br=%d needs %d", who, a.nc,
               a.L, a.Br, nc_need);
    return MB_OK;
}

}  // namespace mb

using namespace mb;

// Picks the kernel instantiation for (hd, N, flags) and launches it, or with ws_need only
// plans the slot split (see launch_fwd).
static int fwd_dispatch(const FlashArgsV& a, int hd, int N, int flags, bool vr, hipStream_t st, float* part,
                        int64_t ws_bytes, int64_t* ws_need) {
    const int NS = (N + 31) / 32;
    const int gm = flash_gate_mode("mb_flash_ema_fwd", flags, N, hd);
    if (gm < 0) return gm;
    if (gm > 0) {
        // the split gate (both modes take it in the forward): hi + lo counter tiles and each
        // wave's W_lo fragments in LDS; three slots per batch fill LDS at N = 64, head_dim 64.
        // The fp32 mode corrects every rate tile, the default the large-counter ones.
        const bool full = gm == 2;
        if (hd == 64)
            return NS == 1 ? launch_fwd<64, 1, 4, true>(a, vr, st, part, ws_bytes, ws_need, full)
                           : launch_fwd<64, 2, 3, true>(a, vr, st, part, ws_bytes, ws_need, full);
        return NS == 1 ? launch_fwd<32, 1, 4, true>(a, vr, st, part, ws_bytes, ws_need, full)
                       : launch_fwd<32, 2, 4, true>(a, vr, st, part, ws_bytes, ws_need, full);
    }
    if (hd == 128) {  // two waves per head, one 16-step tile each
        if (NS == 1) return launch_fwd<128, 1, 4>(a, vr, st, part, ws_bytes, ws_need);
        if (NS == 2) return launch_fwd<128, 2, 4>(a, vr, st, part, ws_bytes, ws_need);
        return launch_fwd<128, 4, 2>(a, vr, st, part, ws_bytes, ws_need);
    }
    if (hd == 64) {
        if (NS == 1) return launch_fwd<64, 1, 4>(a, vr, st, part, ws_bytes, ws_need);
        if (NS == 2) return launch_fwd<64, 2, 4>(a, vr, st, part, ws_bytes, ws_need);
        return launch_fwd<64, 4, 2>(a, vr, st, part, ws_bytes, ws_need);
    }
    if (NS == 1) return launch_fwd<32, 1, 4>(a, vr, st, part, ws_bytes, ws_need);
    if (NS == 2) return launch_fwd<32, 2, 4>(a, vr, st, part, ws_bytes, ws_need);
    return launch_fwd<32, 4, 2>(a, vr, st, part, ws_bytes, ws_need);
}

extern "C" int64_t mb_flash_ema_fwd_workspace(int B, int H, int L, int hd, int K, int N, int flags) {
    FlashArgsV a{};
    a.B = B; a.H = H; a.L = L; a.hd = hd; a.K = K; a.N = N; a.Np = N; a.Br = 64;
    a.nc = L > 0 ? (L + 63) / 64 : 1;
    a.silu = (flags & MB_FLASH_SILU) ? 1 : 0;
    if (flash_validate("mb_flash_ema_fwd_workspace", a, hd)) return -1;
    if (B <= 0 || L <= 0) return 0;
    int64_t need = 0;
    if (fwd_dispatch(a, hd, N, flags, (flags & MB_FLASH_VOCAB_ROWS) != 0, nullptr, nullptr, 0, &need)) return -1;
    return need;
}

extern "C" int mb_flash_ema_fwd(const float* Q, int64_t q_sb, int64_t q_sh, int64_t q_sl,
                                int64_t q_sd, const int64_t* x, int64_t x_sb, int64_t x_sl,
                                const float* E_k, const float* E_v, const float* W_pe,
                                const float* rhos, const int64_t* unique, const float* C_bounds,
                                int B, int H, int L, int hd, int K, int N, int Np, int nc, int Br,
                                int64_t V_total, int flags, float* O, float* LSE, float* scores,
                                void* workspace, int64_t workspace_bytes, void* stream) {
    FlashArgsV a{};
    a.Q = Q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_sl = q_sl; a.q_sd = q_sd;
    a.x = x; a.x_sb = x_sb; a.x_sl = x_sl;
    a.Ek = E_k; a.Ev = E_v; a.W = W_pe; a.rhos = rhos; a.unique = unique; a.Cb = C_bounds;
    a.B = B; a.H = H; a.L = L; a.hd = hd; a.K = K; a.N = N; a.Np = Np; a.Br = Br; a.nc = nc;
    a.v_total = (flags & MB_FLASH_ABSENT_MASS) ? (float)V_total : -1.0f;
    a.silu = (flags & MB_FLASH_SILU) ? 1 : 0;
    a.O = O; a.LSE = LSE;
    a.S2out = scores;
    const bool vr = (flags & MB_FLASH_VOCAB_ROWS) != 0;
    a.e_rows = vr ? V_total : 0;
    int rc = flash_validate("mb_flash_ema_fwd", a, hd);
    if (rc) return rc;
    MB_REQUIRE(!vr || V_total >= 1, "mb_flash_ema_fwd: MB_FLASH_VOCAB_ROWS needs V_total >= 1 rows");
    MB_REQUIRE(workspace_bytes >= 0, "mb_flash_ema_fwd: negative workspace size %lld", (long long)workspace_bytes);
    MB_REQUIRE(((uintptr_t)workspace & 15) == 0, "mb_flash_ema_fwd: workspace must be 16-byte aligned");
    if (B == 0 || L == 0) return MB_OK;
    MB_REQUIRE(Q && x && rhos && unique && O && LSE && W_pe, "mb_flash_ema_fwd: null pointer");
    MB_REQUIRE(K == 0 || (E_k && E_v && C_bounds), "mb_flash_ema_fwd: null slot pointer");
    return fwd_dispatch(a, hd, N, flags, vr, (hipStream_t)stream, static_cast<float*>(workspace),
                        workspace ? workspace_bytes : 0, nullptr);
}
