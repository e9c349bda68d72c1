// EMA counter scans on gfx950: the query-side scan (C_seq) and the key-side chunk-start
// states (C_bounds).
//
// Both rest on one per-sequence index built in LDS: the positions of the sequence sorted
// by (token, position), so that every token's occurrences form a contiguous "chain".
// The recurrence C <- C*rho^dt (+1 per occurrence) only ever couples positions of the
// same chain, so chains are independent and all chains of all sequences run in parallel:
// a group of lanes owns one chain and one slice of the N decay rates, keeps the counter
// in registers and walks the chain, writing each output row with one vector store.
// Nothing of size V (vocabulary) is ever touched, unlike the reference, which zero-fills a
// [B, V+1, N] state every call (mathbrain/triton_ema_query.py:141-142).
#include "common.h"

namespace mb {

constexpr int kScanThreads = 1024;
constexpr int kMaxScanL = 8192;
constexpr int kBoundSlotsPerBlock = 64;
constexpr size_t kMaxLds = 160 * 1024;

// ---- per-sequence sorted index ---------------------------------------------------------------

// Loads x[b, 0:L) into `keys` as (token << pb | position), pads to n (power of two) with the
// all-ones key, and sorts ascending.
template <typename KeyT>
__device__ void build_sorted_positions(const int64_t* __restrict__ x, int64_t sb, int64_t sl,
                                       int b, int L, int n, int pb, KeyT* keys) {
    const KeyT tokmask = (pb == 0) ? ~KeyT(0) : ((~KeyT(0)) >> pb);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        KeyT k = ~KeyT(0);
        if (i < L) {
            const uint64_t tok = (uint64_t)x[(int64_t)b * sb + (int64_t)i * sl];
            k = ((KeyT)tok & tokmask) << pb | (KeyT)i;
        }
        keys[i] = k;
    }
    __syncthreads();
    block_bitonic_sort(keys, n);
}

// First index in sorted keys[0:L) whose token is >= tok (tok given unshifted).
template <typename KeyT>
__device__ inline int lower_bound_token(const KeyT* keys, int L, int pb, uint64_t tok) {
    int lo = 0, hi = L;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((uint64_t)(keys[mid] >> pb) < tok) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// ---- query scan ---------------------------------------------------------------------------

template <typename KeyT, int VEC>
__global__ void __launch_bounds__(kScanThreads)
ema_query_scan_kernel(const int64_t* __restrict__ x, int64_t sb, int64_t sl, int L,
                      const float* __restrict__ rhos, int N, const float* __restrict__ c_init,
                      const int64_t* __restrict__ c_init_keys, int K,
                      const int64_t* __restrict__ doc_ids, float* __restrict__ C_seq,
                      float* state_out, int32_t* __restrict__ stamp_out, int pb, int slice_w) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int b = blockIdx.x;
    const int slice = blockIdx.y;
    const int n = next_pow2(L);
    KeyT* keys = reinterpret_cast<KeyT*>(smem);
    int* chain_start = reinterpret_cast<int*>(keys + n);  // [L + 1]
    int* chain_key = chain_start + (L + 1);               // [L]
    uint32_t* lpt = reinterpret_cast<uint32_t*>(chain_key + L);  // [n]
    int* scratch = reinterpret_cast<int*>(lpt + n);        // [64]

    build_sorted_positions<KeyT>(x, sb, sl, b, L, n, pb, keys);

    // Chain heads: first element of each token run.  Chain c = sorted range
    // [chain_start[c], chain_start[c+1]).
    const int per = (L + blockDim.x - 1) / blockDim.x;
    const int i0 = threadIdx.x * per;
    const int i1 = min(i0 + per, L);
    int cnt = 0;
    for (int i = i0; i < i1; ++i)
        cnt += (i == 0 || (keys[i] >> pb) != (keys[i - 1] >> pb));
    int n_chains;
    int c = block_exclusive_scan(cnt, scratch, n_chains);
    for (int i = i0; i < i1; ++i)
        if (i == 0 || (keys[i] >> pb) != (keys[i - 1] >> pb)) chain_start[c++] = i;
    if (threadIdx.x == 0) chain_start[n_chains] = L;
    for (int j = threadIdx.x; j < n_chains; j += blockDim.x) chain_key[j] = -1;
    if (stamp_out && slice == 0)
        for (int k = threadIdx.x; k < K; k += blockDim.x) stamp_out[(int64_t)b * K + k] = -1;
    __syncthreads();

    // Each key row seeds the chain of its token (the last duplicate key wins, as a
    // sequential scatter_ leaves it, triton_ema_query.py:146-149).
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        const int64_t u = c_init_keys[(int64_t)b * K + k];
        if (u < 0) continue;
        const int i = lower_bound_token(keys, L, pb, (uint64_t)u);
        if (i < L && (uint64_t)(keys[i] >> pb) == (uint64_t)u) {
            int lo = 0, hi = n_chains;  // chain whose start is i
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (chain_start[mid] <= i) lo = mid; else hi = mid;
            }
            atomicMax(&chain_key[lo], k);
        }
    }
    // Longest chains first, so the serial walks of frequent tokens start early.
    const int cp = next_pow2(n_chains);
    for (int j = threadIdx.x; j < cp; j += blockDim.x) {
        uint32_t v = 0xFFFFFFFFu;
        if (j < n_chains) {
            const uint32_t len = (uint32_t)(chain_start[j + 1] - chain_start[j]);
            v = ((0xFFFFu - len) << 16) | (uint32_t)j;
        }
        lpt[j] = v;
    }
    __syncthreads();
    block_bitonic_sort(lpt, cp);

    // Walk the chains: a group of `lanes` lanes owns one chain and VEC*lanes decay rates.
    const int lanes = slice_w / VEC;
    const int groups = blockDim.x / lanes;
    const int g = threadIdx.x / lanes;
    if (g >= groups) return;
    const int n0 = slice * slice_w + (threadIdx.x % lanes) * VEC;
    const bool active = n0 < N;
    float l2hi[VEC], l2lo[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
        l2hi[v] = 0.0f;
        l2lo[v] = 0.0f;
        if (active && n0 + v < N) log2_split(rhos[n0 + v], l2hi[v], l2lo[v]);
    }
    const KeyT posmask = (pb == 0) ? KeyT(0) : ((KeyT(1) << pb) - 1);
    for (int r = g; r < n_chains; r += groups) {
        const int ch = (int)(lpt[r] & 0xFFFFu);
        const int beg = chain_start[ch];
        const int end = chain_start[ch + 1];
        const int key = chain_key[ch];
        float cv[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) cv[v] = 0.0f;
        if (key >= 0 && active) {
            const float* src = c_init + ((int64_t)b * K + key) * N + n0;
            if (VEC == 4) {
                const float4 q = *reinterpret_cast<const float4*>(src);
                cv[0] = q.x; cv[1] = q.y; cv[2] = q.z; cv[3] = q.w;
            } else {
#pragma unroll
                for (int v = 0; v < VEC; ++v) cv[v] = src[v];
            }
        }
        bool has_prev = key >= 0;
        int64_t d_last = (doc_ids && has_prev) ? doc_ids[(int64_t)b * L] : 0;
        int t_last = 0;
        for (int j = beg; j < end; ++j) {
            const int pos = (int)(keys[j] & posmask);
            const int steps = pos - t_last;
#pragma unroll
            for (int v = 0; v < VEC; ++v) cv[v] = cv[v] * pow_steps(l2hi[v], l2lo[v], steps);
            if (doc_ids) {
                const int64_t cur = doc_ids[(int64_t)b * L + pos];
                if (has_prev && d_last != cur) {
#pragma unroll
                    for (int v = 0; v < VEC; ++v) cv[v] = cv[v] * 0.0f;
                }
                d_last = cur;
                has_prev = true;
            }
            if (active) {
                float* dst = C_seq + ((int64_t)b * L + pos) * N + n0;
                if (VEC == 4) {
                    *reinterpret_cast<float4*>(dst) = make_float4(cv[0], cv[1], cv[2], cv[3]);
                } else {
#pragma unroll
                    for (int v = 0; v < VEC; ++v)
                        if (n0 + v < N) dst[v] = cv[v];
                }
            }
#pragma unroll
            for (int v = 0; v < VEC; ++v) cv[v] = cv[v] + 1.0f;
            t_last = pos;
        }
        if (key >= 0) {
            if (state_out && active) {
                float* dst = state_out + ((int64_t)b * K + key) * N + n0;
#pragma unroll
                for (int v = 0; v < VEC; ++v)
                    if (n0 + v < N) dst[v] = cv[v];
            }
            if (stamp_out && slice == 0 && (threadIdx.x % lanes) == 0)
                stamp_out[(int64_t)b * K + key] = t_last;
        }
    }
}

// ---- key-side chunk-start states -----------------------------------------------------------

template <typename KeyT>
__global__ void __launch_bounds__(kScanThreads)
ema_boundary_kernel(const int64_t* __restrict__ x, int64_t sb, int64_t sl, int L,
                    const int64_t* __restrict__ unique, int K, const float* __restrict__ rhos,
                    int N, int Br, int nc, const float* __restrict__ c_init, int64_t cis,
                    const int64_t* __restrict__ doc_ids, float* __restrict__ out, int Np,
                    int pb) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int b = blockIdx.x;
    const int k0 = blockIdx.y * kBoundSlotsPerBlock;
    const int n = next_pow2(L);
    KeyT* keys = reinterpret_cast<KeyT*>(smem);
    int* resets = reinterpret_cast<int*>(keys + n);  // [L] positions where the document changes
    int* scratch = resets + L;                       // [64]

    build_sorted_positions<KeyT>(x, sb, sl, b, L, n, pb, keys);

    int n_resets = 0;
    if (doc_ids) {
        const int per = (L + blockDim.x - 1) / blockDim.x;
        const int i0 = threadIdx.x * per;
        const int i1 = min(i0 + per, L);
        const int64_t* d = doc_ids + (int64_t)b * L;
        int cnt = 0;
        for (int i = max(i0, 1); i < i1; ++i) cnt += d[i] != d[i - 1];
        int c = block_exclusive_scan(cnt, scratch, n_resets);
        for (int i = max(i0, 1); i < i1; ++i)
            if (d[i] != d[i - 1]) resets[c++] = i;
        __syncthreads();
    }

    const KeyT posmask = (pb == 0) ? KeyT(0) : ((KeyT(1) << pb) - 1);
    const int kcount = min(kBoundSlotsPerBlock, K - k0);
    for (int idx = threadIdx.x; idx < kcount * Np; idx += blockDim.x) {
        const int k = k0 + idx / Np;
        const int col = idx % Np;
        float* o = out + ((int64_t)b * nc * K + k) * Np + col;
        const int64_t cstride = (int64_t)K * Np;
        if (col >= N) {
            for (int j = 0; j < nc; ++j) o[j * cstride] = 0.0f;
            continue;
        }
        float hi, lo;
        log2_split(rhos[col], hi, lo);
        float c = c_init ? c_init[((int64_t)b * K + k) * cis + col] : 0.0f;
        const int64_t u = unique[(int64_t)b * K + k];
        int mi = 0, me = 0;  // this slot's chain in the sorted positions
        if (u >= 0) {
            mi = lower_bound_token(keys, L, pb, (uint64_t)u);
            me = lower_bound_token(keys, L, pb, (uint64_t)u + 1);
        }
        int ri = 0;
        int t_cur = 0;  // c is the state before step t_cur
        for (int j = 0; j < nc; ++j) {
            const int tb = j * Br;
            // Events before the chunk start, in time order: a document reset at r zeroes the
            // state before step r; an occurrence at s adds 1 after step s's decay.
            while (true) {
                const int s = (mi < me) ? (int)(keys[mi] & posmask) : INT32_MAX;
                const int r = (ri < n_resets) ? resets[ri] : INT32_MAX;
                if (r <= s && r < tb) {
                    c = 0.0f;
                    t_cur = r;
                    ++ri;
                } else if (s < tb) {
                    c = c * pow_steps(hi, lo, s + 1 - t_cur) + 1.0f;
                    t_cur = s + 1;
                    ++mi;
                } else {
                    break;
                }
            }
            c = c * pow_steps(hi, lo, tb - t_cur);
            t_cur = tb;
            o[j * cstride] = c;
        }
    }
}

template <typename F>
static int set_lds(F kernel, size_t bytes) {
    if (bytes > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail((int)e, "hipFuncSetAttribute(max dynamic LDS = %zu) failed: %s", bytes,
                        hipGetErrorString(e));
        }
    }
    return MB_OK;
}

}  // namespace mb

using namespace mb;

extern "C" int mb_ema_query_scan(const int64_t* x, int64_t x_stride_b, int64_t x_stride_l, int B,
                                 int L, const float* rhos, int N, int64_t vocab_size,
                                 const float* c_init, const int64_t* c_init_keys, int K,
                                 const int64_t* doc_ids, float* C_seq, float* state_out,
                                 int32_t* stamp_out, void* stream) {
    MB_REQUIRE(B >= 0 && L >= 0, "mb_ema_query_scan: negative B=%d or L=%d", B, L);
    MB_REQUIRE(N >= 1, "mb_ema_query_scan: N=%d must be >= 1", N);
    if (!c_init || !c_init_keys) K = 0;
    MB_REQUIRE(K >= 0, "mb_ema_query_scan: negative K=%d", K);
    if (B == 0 || L == 0) return MB_OK;
    MB_REQUIRE(x && rhos && C_seq, "mb_ema_query_scan: x, rhos and C_seq must be non-null");
    if (L > kMaxScanL)
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_query_scan: L=%d exceeds the on-chip limit %d", L,
                    kMaxScanL);
    const int pb = ceil_log2(L);
    const bool wide = vocab_size > 0 && (pb >= 32 || (uint64_t)vocab_size > (1ull << (32 - pb)));
    const int n = next_pow2(L);
    const size_t key_bytes = wide ? 8 : 4;
    const size_t lds = n * key_bytes + (size_t)(2 * L + 1) * 4 + (size_t)n * 4 + 64 * 4;
    if (lds > kMaxLds)
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_query_scan: L=%d with vocab %lld needs %zu B of LDS",
                    L, (long long)vocab_size, lds);
    const bool vec4 = (N % 4) == 0;
    int slice_w = N >= 32 ? 32 : N;
    if (vec4) slice_w = (slice_w + 3) & ~3;
    const int ns = (N + slice_w - 1) / slice_w;
    dim3 grid(B, ns);
    hipStream_t st = (hipStream_t)stream;
#define MB_LAUNCH_SCAN(KT, V)                                                                  \
    do {                                                                                       \
        auto kfn = ema_query_scan_kernel<KT, V>;                                               \
        int rc = set_lds(kfn, lds);                                                            \
        if (rc) return rc;                                                                     \
        hipLaunchKernelGGL(kfn, grid, dim3(kScanThreads), lds, st, x, x_stride_b, x_stride_l, L, \
                           rhos, N, c_init, c_init_keys, K, doc_ids, C_seq, state_out,          \
                           stamp_out, pb, slice_w);                                            \
    } while (0)
    if (wide) {
        if (vec4) MB_LAUNCH_SCAN(uint64_t, 4); else MB_LAUNCH_SCAN(uint64_t, 1);
    } else {
        if (vec4) MB_LAUNCH_SCAN(uint32_t, 4); else MB_LAUNCH_SCAN(uint32_t, 1);
    }
#undef MB_LAUNCH_SCAN
    return check_launch("mb_ema_query_scan");
}

extern "C" int mb_ema_boundary_states(const int64_t* x, int64_t x_stride_b, int64_t x_stride_l,
                                      int B, int L, const int64_t* unique, int K,
                                      const float* rhos, int N, int Br, const float* c_init,
                                      int64_t c_init_stride_k, const int64_t* doc_ids,
                                      float* C_bounds, int Np, void* stream) {
    MB_REQUIRE(B >= 0 && L >= 0 && K >= 0, "mb_ema_boundary_states: negative B=%d, L=%d or K=%d", B,
               L, K);
    MB_REQUIRE(N >= 1 && Np >= N, "mb_ema_boundary_states: need 1 <= N=%d <= Np=%d", N, Np);
    MB_REQUIRE(Br >= 1, "mb_ema_boundary_states: Br=%d must be >= 1", Br);
    MB_REQUIRE(!c_init || c_init_stride_k >= N, "mb_ema_boundary_states: c_init row stride %lld < N",
               (long long)c_init_stride_k);
    if (B == 0 || K == 0) return MB_OK;
    MB_REQUIRE(unique && rhos && C_bounds, "mb_ema_boundary_states: null pointer");
    MB_REQUIRE(L == 0 || x, "mb_ema_boundary_states: x is null");
    if (L > kMaxScanL)
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_boundary_states: L=%d exceeds the on-chip limit %d",
                    L, kMaxScanL);
    const int nc = L > 0 ? (L + Br - 1) / Br : 1;
    const int Lk = L > 0 ? L : 1;  // an empty sequence still stores c0 once
    const int pb = ceil_log2(Lk);
    const int n = next_pow2(Lk);
    const size_t key_bytes = 8;  // slot ids are int64 and unbounded by any vocab size here
    const size_t lds = n * key_bytes + (size_t)Lk * 4 + 64 * 4;
    if (lds > kMaxLds)
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_boundary_states: L=%d needs %zu B of LDS", L, lds);
    dim3 grid(B, (K + kBoundSlotsPerBlock - 1) / kBoundSlotsPerBlock);
    auto kfn = ema_boundary_kernel<uint64_t>;
    int rc = set_lds(kfn, lds);
    if (rc) return rc;
    hipLaunchKernelGGL(kfn, grid, dim3(kScanThreads), lds, (hipStream_t)stream, x, x_stride_b,
                       x_stride_l, L, unique, K, rhos, N, Br, nc, c_init, c_init_stride_k, doc_ids,
                       C_bounds, Np, pb);
    return check_launch("mb_ema_boundary_states");
}
