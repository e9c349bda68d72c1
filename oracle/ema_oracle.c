/*
 * TEST INFRASTRUCTURE ONLY -- never linked into, or called by, the product.
 *
 * Plain-C restatement of the reference's two EMA counter scans, used by the
 * tests, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the
 * checker.  Every function follows the reference step by step, in the same
 * order and in the same precision (fp32), so that the HIP kernels can be held
 * against it.
 *
 *   mbo_query_scan       <- compute_query_ema_history_pt
 *                           (mathbrain/triton_ema_query.py:67-117)
 *   mbo_boundary_states  <- _c_boundary_scan + precompute_boundaries
 *                           (mathbrain/triton_flash_ema.py:29-78, 81-113)
 *
 * Pinning: both functions are checked against the reference's own known
 * answers (tests/test_doc_boundary.py:71-134, tests/test_pipeline_thorough.py
 * :191-271, tests/test_gold_standard.py:113-160) and against the closed forms
 *   C_seq[t]    = c0[x_t] rho^t + sum_{s<t, x_s=x_t} rho^(t-s)
 *   C_bound[j]  = c0 rho^(jBr) + sum_{s<jBr, x_s=u} rho^(jBr-1-s)
 * evaluated independently in tests/test_oracle_scan.py.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fused multiply-add,
 * so that every product and sum is rounded the way the reference's torch
 * CPU path rounds it).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* compute_query_ema_history_pt (triton_ema_query.py:67-117).
 *
 * x        [B, L] token ids
 * rhos     [N]
 * c_init   [B, K, N] or NULL, c_init_keys [B, K] or NULL (-1 = padding,
 *          mapped to the dummy row V as at triton_ema_query.py:81)
 * doc_ids  [B, L] or NULL
 * C_seq    [B, L, N] output
 *
 * Returns 0, or -1 when the scratch state cannot be allocated.
 */
int mbo_query_scan(const int64_t *x, int B, int L, const float *rhos, int N,
                   int64_t V, const float *c_init, const int64_t *c_init_keys,
                   int K, const int64_t *doc_ids, float *C_seq) {
    const int64_t R = V + 1; /* vocab rows plus the dummy row (:78-80) */
    float *T_last = (float *)malloc(sizeof(float) * R);
    float *C_last = (float *)malloc(sizeof(float) * R * N);
    int32_t *D_last = (int32_t *)malloc(sizeof(int32_t) * R);
    if (!T_last || !C_last || !D_last) {
        free(T_last); free(C_last); free(D_last);
        return -1;
    }
    for (int b = 0; b < B; ++b) {
        /* :78-80 */
        for (int64_t v = 0; v < R; ++v) { T_last[v] = -1000000.0f; D_last[v] = -1; }
        memset(C_last, 0, sizeof(float) * R * N);
        /* :82-89 -- scatter_ in key order, so a repeated key keeps the last row */
        if (c_init && c_init_keys) {
            for (int k = 0; k < K; ++k) {
                int64_t key = c_init_keys[(int64_t)b * K + k];
                int64_t row = (key == -1) ? V : key;
                T_last[row] = 0.0f;
                memcpy(C_last + row * N, c_init + ((int64_t)b * K + k) * N, sizeof(float) * N);
                if (doc_ids) D_last[row] = (int32_t)doc_ids[(int64_t)b * L + 0];
            }
        }
        /* :94-115 */
        for (int t = 0; t < L; ++t) {
            int64_t xt = x[(int64_t)b * L + t];
            float t_last = T_last[xt];
            float steps = (float)t - t_last;          /* (t - t_last).float() */
            float *cl = C_last + xt * N;
            float *out = C_seq + ((int64_t)b * L + t) * N;
            float keep = 1.0f;
            if (doc_ids) {
                int32_t cur = (int32_t)doc_ids[(int64_t)b * L + t];
                int same = (D_last[xt] == cur) || (t_last < 0.0f);
                keep = same ? 1.0f : 0.0f;
                D_last[xt] = cur;
            }
            for (int n = 0; n < N; ++n) {
                float decay = powf(rhos[n], steps);  /* rhos ** decay_steps */
                float c = cl[n] * decay;
                if (doc_ids) c = c * keep;
                out[n] = c;
                cl[n] = c + 1.0f;
            }
            T_last[xt] = (float)t;
        }
    }
    free(T_last); free(C_last); free(D_last);
    return 0;
}

/* _c_boundary_scan (triton_flash_ema.py:29-78): the key-side EMA state of every
 * slot u_k = unique[b,k] at the start of each Br-step chunk, stored BEFORE the
 * chunk is processed (:56-61), with C <- C*rho + I(x_t == u_k) per step (:77-78)
 * and an optional reset at document boundaries (:69-75).
 *
 * out [B, nc, K, N] with nc = max(1, ceil(L/Br)); c_init [B,K,N] or NULL (zeros).
 */
void mbo_boundary_states(const int64_t *x, const int64_t *unique, int B, int L, int K,
                         const float *rhos, int N, int Br, const float *c_init,
                         const int64_t *doc_ids, float *out) {
    int nc = (L + Br - 1) / Br;
    if (nc < 1) nc = 1;
    float *C = (float *)malloc(sizeof(float) * N);
    for (int b = 0; b < B; ++b) {
        for (int k = 0; k < K; ++k) {
            int64_t uk = unique[(int64_t)b * K + k];
            for (int n = 0; n < N; ++n)
                C[n] = c_init ? c_init[((int64_t)b * K + k) * N + n] : 0.0f;
            int64_t prev_doc = doc_ids ? doc_ids[(int64_t)b * L] : -1;
            for (int ch = 0; ch < nc; ++ch) {
                float *o = out + (((int64_t)b * nc + ch) * K + k) * N;
                memcpy(o, C, sizeof(float) * N);
                for (int i = 0; i < Br; ++i) {
                    int t = ch * Br + i;
                    int mt = t < L;
                    int64_t xt = mt ? x[(int64_t)b * L + t] : -1;
                    if (doc_ids) {
                        int64_t cur = mt ? doc_ids[(int64_t)b * L + t] : -1;
                        int boundary = (cur != prev_doc) && (t > 0) && mt;
                        float keep = boundary ? 0.0f : 1.0f;
                        for (int n = 0; n < N; ++n) C[n] = C[n] * keep;
                        prev_doc = cur;
                    }
                    float match = (mt && xt == uk) ? 1.0f : 0.0f;
                    for (int n = 0; n < N; ++n) C[n] = C[n] * rhos[n] + match;
                }
            }
        }
    }
    free(C);
}
