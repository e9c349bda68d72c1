// EMA counter scans on gfx950: the query-side scan (C_seq) and the key-side chunk-start
// states (C_bounds).
//
// The query scan sorts each sequence's positions by (token, position) in LDS, so that
// every token's occurrences form a contiguous "chain": the recurrence
// C <- C*rho^dt (+1 per occurrence) only couples positions of one chain, so lane groups
// walk chains in parallel, writing each output row with one vector store.  The key-side
// states need no sort: a wave follows one slot and finds its occurrences in each window
// with a ballot.  Nothing of size V (vocabulary) is ever touched, unlike the reference,
// which zero-fills a [B, V+1, N] state every call (mathbrain/triton_ema_query.py:141-142).
#include "common.h"

#include <algorithm>

namespace mb {

constexpr int kScanThreads = 1024;
constexpr int kMaxScanL = 8192;
constexpr size_t kMaxLds = 160 * 1024;

// ---- query scan ---------------------------------------------------------------------------
//
// After the sort, chain c is the sorted range [chain_start[c], chain_start[c+1]) and the
// recurrence along it, in pre-increment values C_j = C_seq at the chain's j-th position,
//   C_1 = c0 rho^t_1,   C_j = (C_{j-1} + 1) rho^(t_j - t_{j-1})
// is linear.  Chains are cut into segments of at most S elements, so that no lane group
// walks more than S steps however frequent a token is (the top Zipf token of a 2048-token
// sequence occurs ~190 times).  Pass A walks every segment that is not its chain's last
// one from zero and keeps its local sum at the segment's last element,
//   agg_k = sum_{j in segment k, j < last} rho^(t_last - t_j),
// in LDS.  Pass B walks every segment again and writes C_seq; segment i of a chain first
// rebuilds its carry-in from the chain's earlier aggregates,
//   C_last(k) = (C_last(k-1) + 1) rho^(t_last(k) - t_last(k-1)) + agg_k,
// (C_last(-1) + 1 := c0 at t = 0), which costs i <= L/S steps.  With doc_ids, a segment
// that contains a document change drops its carry (flag kept beside the aggregate).

template <int VEC>
struct Vec {
    float v[VEC];
};

template <int VEC>
__device__ inline Vec<VEC> load_vec(const float* src, bool ok, int n0, int N) {
    Vec<VEC> r;
#pragma unroll
    for (int i = 0; i < VEC; ++i) r.v[i] = 0.f;
    if (!ok) return r;
    if (VEC == 4) {
        const float4 q = *reinterpret_cast<const float4*>(src);
        r.v[0] = q.x; r.v[1] = q.y; r.v[2] = q.z; r.v[3] = q.w;
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i)
            if (n0 + i < N) r.v[i] = src[i];
    }
    return r;
}

template <int VEC>
__device__ inline void store_vec(float* dst, const float* v, int n0, int N) {
    if (VEC == 4) {
        *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i)
            if (n0 + i < N) dst[i] = v[i];
    }
}

// x^e for an integer e >= 0 by binary exponentiation in double precision.
__device__ inline double powi(double x, int e) {
    double r = 1.0;
    while (e) {
        if (e & 1) r *= x;
        x *= x;
        e >>= 1;
    }
    return r;
}

// Radix sort rounds per wave (64 keys each): 2 cover L <= 2048 with 16 waves, and that
// variant is register-light enough for two workgroups per CU; 8 cover L <= 8192.
constexpr int kScanRoundsSmall = 2;
constexpr int kScanRoundsLarge = 8;

// Byte offsets of the per-sequence index inside dynamic LDS.  The radix sort's scratch,
// the slot lookup's element->chain map and the power tables are live at different times
// and share space.
struct ScanLds {
    size_t keys, chain_start, chain_seg, seg_chain, nf_seg, chain_key, r1;
    size_t sort_b, sort_cnt;             // during the sort (from the end of keys)
    size_t elem_chain, scan_scratch;     // during the chain build and slot lookup (r1)
    size_t agg, aggr, lowT, highT;       // during the walks (r1)
    size_t total;
    __host__ __device__ ScanLds(int L, int key_bytes, int nthr, int nf_max, int slice_w, int nH) {
        auto al = [](size_t o) { return (o + 15) & ~(size_t)15; };
        keys = 0;
        size_t o = al((size_t)L * key_bytes);
        const size_t after_keys = o;
        chain_start = o; o += (size_t)(L + 1) * 2;
        chain_seg = o;   o += (size_t)(L + 1) * 2;
        seg_chain = o;   o += (size_t)L * 2;
        nf_seg = o;      o += (size_t)nf_max * 2;
        o = al(o);
        chain_key = o;   o += (size_t)L * 4;
        r1 = o = al(o);
        elem_chain = r1;
        agg = r1;
        aggr = agg + (size_t)nf_max * slice_w * 4;
        lowT = al(aggr + (size_t)nf_max * 4);
        highT = lowT + (size_t)64 * slice_w * 4;
        const size_t walk_end = highT + (size_t)nH * slice_w * 4;
        scan_scratch = al(elem_chain + (size_t)L * 2);
        const size_t lookup_end = scan_scratch + 64 * 4;
        sort_b = after_keys;
        sort_cnt = al(sort_b + (size_t)L * key_bytes);
        const size_t sort_end = sort_cnt + (size_t)(4 * nthr + 64) * 4;
        total = al(walk_end > lookup_end ? walk_end : lookup_end);
        if (sort_end > total) total = al(sort_end);
    }
};

// Query scan: one workgroup per (sequence b, slice of slice_w decay rates).
//   1. keys = (token << pb | position) in position order, stably radix-sorted by token:
//      chain c = the sorted range [chain_start[c], chain_start[c+1]) of one token.
//   2. chains are cut into segments of at most S elements; c_init keys are matched to
//      their chains.
//   3. pass A: local aggregates of the non-final segments; pass B: every segment rebuilds
//      its carry-in from its chain's earlier aggregates and writes its C_seq rows.
// rho^d comes from two LDS tables per rate, rho^(d mod 64) * rho^(64 floor(d / 64)),
// each entry a correctly rounded float of a double-precision power.
template <typename KeyT, int VEC, bool DOCS, int MAXR>
__global__ void __launch_bounds__(kScanThreads) __attribute__((amdgpu_waves_per_eu(MAXR <= 2 ? 8 : 1)))
ema_query_scan_kernel(const int64_t* __restrict__ x, int64_t sb, int64_t sl, int L,
                      const float* __restrict__ rhos, int N, const float* __restrict__ c_init,
                      const int64_t* __restrict__ c_init_keys, int K,
                      const int64_t* __restrict__ doc_ids, float* __restrict__ C_seq,
                      float* state_out, int32_t* __restrict__ stamp_out, int pb, int tok_bits,
                      int slice_w, int S, int nf_max) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int b = blockIdx.x;
    const int slice = blockIdx.y;
    const int nH = (L - 1) / 64 + 1;
    const ScanLds lay(L, (int)sizeof(KeyT), blockDim.x, nf_max, slice_w, nH);
    KeyT* keys = reinterpret_cast<KeyT*>(smem + lay.keys);
    uint16_t* chain_start = reinterpret_cast<uint16_t*>(smem + lay.chain_start);
    uint16_t* chain_seg = reinterpret_cast<uint16_t*>(smem + lay.chain_seg);
    uint16_t* seg_chain = reinterpret_cast<uint16_t*>(smem + lay.seg_chain);
    uint16_t* nf_seg = reinterpret_cast<uint16_t*>(smem + lay.nf_seg);
    int* chain_key = reinterpret_cast<int*>(smem + lay.chain_key);
    uint16_t* elem_chain = reinterpret_cast<uint16_t*>(smem + lay.elem_chain);
    float* agg = reinterpret_cast<float*>(smem + lay.agg);
    int* aggr = reinterpret_cast<int*>(smem + lay.aggr);
    float* lowT = reinterpret_cast<float*>(smem + lay.lowT);
    float* highT = reinterpret_cast<float*>(smem + lay.highT);
    int* scratch;

    // 1. sorted (token, position) keys
    {
        const KeyT tokmask = (pb == 0) ? ~KeyT(0) : ((~KeyT(0)) >> pb);
        for (int i = threadIdx.x; i < L; i += blockDim.x) {
            const uint64_t tok = (uint64_t)x[(int64_t)b * sb + (int64_t)i * sl];
            keys[i] = ((KeyT)tok & tokmask) << pb | (KeyT)i;
        }
        __syncthreads();
        KeyT* sorted = block_radix_sort<MAXR>(keys, reinterpret_cast<KeyT*>(smem + lay.sort_b),
                                                        reinterpret_cast<int*>(smem + lay.sort_cnt), L,
                                                        pb, tok_bits);
        if (sorted != keys) {
            for (int i = threadIdx.x; i < L; i += blockDim.x) keys[i] = sorted[i];
            __syncthreads();
        }
    }
    scratch = reinterpret_cast<int*>(smem + lay.scan_scratch);

    // chain heads (first element of each token run), element -> chain map
    const int per = (L + blockDim.x - 1) / blockDim.x;
    const int i0 = threadIdx.x * per;
    const int i1 = min(i0 + per, L);
    int cnt = 0;
    for (int i = i0; i < i1; ++i) cnt += (i == 0 || (keys[i] >> pb) != (keys[i - 1] >> pb));
    int n_chains;
    int c = block_exclusive_scan(cnt, scratch, n_chains);
    for (int i = i0; i < i1; ++i) {
        if (i == 0 || (keys[i] >> pb) != (keys[i - 1] >> pb)) chain_start[c++] = (uint16_t)i;
        elem_chain[i] = (uint16_t)(c - 1);
    }
    if (threadIdx.x == 0) chain_start[n_chains] = (uint16_t)L;
    if (stamp_out && slice == 0)
        for (int k = threadIdx.x; k < K; k += blockDim.x) stamp_out[(int64_t)b * K + k] = -1;
    __syncthreads();

    // 2. segments: chain c owns segments [chain_seg[c], chain_seg[c+1])
    const int cper = (n_chains + blockDim.x - 1) / blockDim.x;
    const int c0i = threadIdx.x * cper;
    const int c1i = min(c0i + cper, n_chains);
    int nseg = 0;
    for (int cc = c0i; cc < c1i; ++cc) nseg += (chain_start[cc + 1] - chain_start[cc] + S - 1) / S;
    int n_segs;
    int so = block_exclusive_scan(nseg, scratch, n_segs);
    for (int cc = c0i; cc < c1i; ++cc) {
        chain_seg[cc] = (uint16_t)so;
        chain_key[cc] = -1;
        const int ns = (chain_start[cc + 1] - chain_start[cc] + S - 1) / S;
        for (int q = 0; q < ns; ++q) seg_chain[so + q] = (uint16_t)cc;
        for (int q = 0; q + 1 < ns; ++q) nf_seg[so - cc + q] = (uint16_t)(so + q);
        so += ns;
    }
    if (threadIdx.x == 0) chain_seg[n_chains] = (uint16_t)n_segs;
    __syncthreads();

    // each key row seeds the chain of its token; the last duplicate key wins, as a
    // sequential scatter_ leaves it (triton_ema_query.py:146-149).  Four lookups per
    // thread run in lockstep so their dependent LDS reads overlap.
    for (int kb = threadIdx.x; kb < K; kb += 4 * blockDim.x) {
        uint64_t tok[4];
        int lo[4], hi[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int k = kb + r * blockDim.x;
            const int64_t u = k < K ? c_init_keys[(int64_t)b * K + k] : (int64_t)-1;
            tok[r] = (uint64_t)u;
            lo[r] = 0;
            hi[r] = u < 0 ? 0 : L;
        }
        for (int it = 0; it < 32; ++it) {
            bool any = false;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (lo[r] < hi[r]) {
                    const int mid = (lo[r] + hi[r]) >> 1;
                    if ((uint64_t)(keys[mid] >> pb) < tok[r]) lo[r] = mid + 1; else hi[r] = mid;
                    any = true;
                }
            }
            if (!any) break;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int k = kb + r * blockDim.x;
            if (k < K && (int64_t)tok[r] >= 0 && lo[r] < L && (uint64_t)(keys[lo[r]] >> pb) == tok[r])
                atomicMax(&chain_key[elem_chain[lo[r]]], k);
        }
    }
    __syncthreads();  // elem_chain is dead from here; r1 now holds the tables and aggregates

    // power tables of this slice's rates
    for (int i = threadIdx.x; i < (64 + nH) * slice_w; i += blockDim.x) {
        const int j = i / slice_w;
        const int r = i % slice_w;
        const int nn = slice * slice_w + r;
        float v = 0.f;
        if (nn < N) {
            const double rho = (double)rhos[nn];
            v = (float)(j < 64 ? powi(rho, j) : powi(powi(rho, 64), j - 64));
        }
        lowT[i] = v;  // highT follows lowT: entry j >= 64 is rho^(64 (j - 64))
    }

    const int lanes = slice_w / VEC;
    const int groups = blockDim.x / lanes;
    const int g = threadIdx.x / lanes;
    const int lane_r = (threadIdx.x % lanes) * VEC;  // rate offset inside the slice
    const int n0 = slice * slice_w + lane_r;
    const bool active = n0 < N && g < groups;
    const KeyT posmask = (pb == 0) ? KeyT(0) : ((KeyT(1) << pb) - 1);
    auto pos_of = [&](int j) { return (int)(keys[j] & posmask); };
    auto doc_of = [&](int pos) { return doc_ids[(int64_t)b * L + pos]; };
    // rho^d for this lane's VEC rates
    auto powv = [&](int d, float* pw) {
        const float* lo = lowT + (d & 63) * slice_w + lane_r;
        const float* hi = highT + (d >> 6) * slice_w + lane_r;
        if (VEC == 4) {
            const float4 a = *reinterpret_cast<const float4*>(lo);
            const float4 h = *reinterpret_cast<const float4*>(hi);
            pw[0] = a.x * h.x; pw[1] = a.y * h.y; pw[2] = a.z * h.z; pw[3] = a.w * h.w;
        } else {
#pragma unroll
            for (int v = 0; v < VEC; ++v) pw[v] = lo[v] * hi[v];
        }
    };
    float* const Cb = C_seq + (int64_t)b * L * N + n0;
    __syncthreads();

    // 3a. pass A: local aggregates of the non-final segments
    const int n_nf = n_segs - n_chains;
    if (g < groups) {
        for (int f = g; f < n_nf; f += groups) {
            const int s = nf_seg[f];
            const int cc = seg_chain[s];
            const int qi = s - chain_seg[cc];
            const int beg = chain_start[cc] + qi * S;
            float h[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v) h[v] = 0.f;
            int reset = 0;
            int tp = pos_of(beg);
            int64_t dprev = 0;
            if (DOCS) {
                const bool has_prev = qi > 0 || chain_key[cc] >= 0;
                const int64_t dcur = doc_of(tp);
                const int64_t dref = qi > 0 ? doc_of(pos_of(beg - 1)) : doc_of(0);
                reset = has_prev && dref != dcur;
                dprev = dcur;
            }
            for (int j = beg + 1; j < beg + S; ++j) {
                const int t = pos_of(j);
                float pw[VEC];
                powv(t - tp, pw);
#pragma unroll
                for (int v = 0; v < VEC; ++v) h[v] = (h[v] + 1.0f) * pw[v];
                if (DOCS) {
                    const int64_t dcur = doc_of(t);
                    if (dcur != dprev) {
                        reset = 1;
#pragma unroll
                        for (int v = 0; v < VEC; ++v) h[v] = 0.f;
                    }
                    dprev = dcur;
                }
                tp = t;
            }
#pragma unroll
            for (int v = 0; v < VEC; ++v) agg[f * slice_w + lane_r + v] = h[v];
            if (DOCS && lane_r == 0) aggr[f] = reset;
        }
    }
    __syncthreads();

    // 3b. pass B: every segment, from its carry-in, writes C_seq rows (and the final
    // state).  A group takes its segments kBatch at a time and issues their c_init row
    // loads first.
    constexpr int kBatch = MAXR <= 2 ? 2 : 4;
    if (g < groups) {
        for (int s0 = g; s0 < n_segs; s0 += kBatch * groups) {
            Vec<VEC> c0v[kBatch];
            int keyv[kBatch];
#pragma unroll
            for (int r = 0; r < kBatch; ++r) {
                const int s = s0 + r * groups;
                keyv[r] = s < n_segs ? chain_key[seg_chain[s]] : -1;
                c0v[r] = load_vec<VEC>(c_init + ((int64_t)b * K + (keyv[r] >= 0 ? keyv[r] : 0)) * N + n0,
                                       keyv[r] >= 0 && active, n0, N);
            }
#pragma unroll
            for (int r = 0; r < kBatch; ++r) {
                const int s = s0 + r * groups;
                if (s >= n_segs) break;
                const int cc = seg_chain[s];
                const int key = keyv[r];
                const int cs = chain_start[cc];
                const int ce = chain_start[cc + 1];
                const int f0 = chain_seg[cc] - cc;  // non-final index of the chain's first segment
                const int qi = s - chain_seg[cc];
                const int beg = cs + qi * S;
                const int end = min(beg + S, ce);
                // post-increment state P at time tp entering the chain: c0 at t = 0
                float P[VEC];
#pragma unroll
                for (int v = 0; v < VEC; ++v) P[v] = c0v[r].v[v];
                int tp = 0;
                bool has_prev = key >= 0;
                int64_t dprev = 0;
                if (DOCS && has_prev) dprev = doc_of(0);
                for (int k = 0; k < qi; ++k) {  // carry through the chain's earlier segments
                    const int tl = pos_of(cs + (k + 1) * S - 1);
                    const bool drop = DOCS && aggr[f0 + k];
                    float pw[VEC];
                    powv(tl - tp, pw);
#pragma unroll
                    for (int v = 0; v < VEC; ++v)
                        P[v] = (drop ? 0.f : P[v] * pw[v]) + agg[(f0 + k) * slice_w + lane_r + v] + 1.0f;
                    tp = tl;
                }
                if (DOCS && qi > 0) {
                    dprev = doc_of(tp);
                    has_prev = true;
                }
                int t = tp;
                for (int j = beg; j < end; ++j) {
                    t = pos_of(j);
                    float cv[VEC];
                    powv(t - tp, cv);
#pragma unroll
                    for (int v = 0; v < VEC; ++v) cv[v] *= P[v];
                    if (DOCS) {
                        const int64_t dcur = doc_of(t);
                        if (has_prev && dcur != dprev) {
#pragma unroll
                            for (int v = 0; v < VEC; ++v) cv[v] = 0.f;
                        }
                        dprev = dcur;
                        has_prev = true;
                    }
                    if (active && t < L) store_vec<VEC>(Cb + t * N, cv, n0, N);
#pragma unroll
                    for (int v = 0; v < VEC; ++v) P[v] = cv[v] + 1.0f;
                    tp = t;
                }
                if (end == ce && key >= 0) {
                    if (state_out && active)
                        store_vec<VEC>(state_out + ((int64_t)b * K + key) * N + n0, P, n0, N);
                    if (stamp_out && slice == 0 && lane_r == 0) stamp_out[(int64_t)b * K + key] = t;
                }
            }
        }
    }
}

// ---- key-side chunk-start states -----------------------------------------------------------
//
// One workgroup per (sequence b, block of kBoundSlots slots); wave w takes slots w,
// w + nwaves, ... and its lanes the decay rates (lane, lane + 64, ...).  The sequence's
// tokens sit in LDS.  Between two chunk starts the window [(j-1) Br, j Br) is walked in
// pieces of at most 64 steps: one ballot of (token == slot id) gives the piece's
// occurrence mask and the state advances as
//   C <- C rho^len + sum_{p in mask} rho^(len - 1 - p)
// (an occurrence adds 1 after its step's decay: triton_flash_ema.py:56-78).  A document
// change at r zeroes the state before step r (:69-75): the piece drops the carried state
// and the occurrences before its last change.  No sort is needed.

constexpr int kBoundThreads = 512;
constexpr int kBoundSlots = 32;

// 64 bits of the bitmask `bits` starting at bit `pos` (bits beyond the array read as 0:
// the array carries one spare word).
__device__ inline uint64_t bits64_at(const uint64_t* bits, int pos) {
    const int w = pos >> 6;
    const int off = pos & 63;
    uint64_t v = bits[w] >> off;
    if (off) v |= bits[w + 1] << (64 - off);
    return v;
}

template <int RPL>
__global__ void __launch_bounds__(kBoundThreads)
ema_boundary_kernel(const int64_t* __restrict__ x, int64_t sb, int64_t sl, int L,
                    const int64_t* __restrict__ unique, int K, const float* __restrict__ rhos,
                    int N, int Br, int nc, const float* __restrict__ c_init, int64_t cis,
                    const int64_t* __restrict__ doc_ids, float* __restrict__ out, int Np) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nwords = (L >> 6) + 2;
    int64_t* tok = reinterpret_cast<int64_t*>(smem);                 // [L]
    uint64_t* rbits = reinterpret_cast<uint64_t*>(tok + L);          // [nwords] document changes
    const int b = blockIdx.x;
    const int k0 = blockIdx.y * kBoundSlots;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int nw = blockDim.x >> 6;

    for (int i = threadIdx.x; i < L; i += blockDim.x) tok[i] = x[(int64_t)b * sb + (int64_t)i * sl];
    // bit p: the document changes at step p (doc[p] != doc[p - 1], p >= 1)
    for (int w = wave; w < nwords; w += nw) {
        const int p = 64 * w + lane;
        bool chg = false;
        if (doc_ids && p >= 1 && p < L)
            chg = doc_ids[(int64_t)b * L + p] != doc_ids[(int64_t)b * L + p - 1];
        const uint64_t m = __ballot(chg);
        if (lane == 0) rbits[w] = m;
    }
    float hi[RPL], lo[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        hi[r] = 0.f;
        lo[r] = 0.f;
        const int n = lane + 64 * r;
        if (n < N) log2_split(rhos[n], hi[r], lo[r]);
    }
    __syncthreads();

    const int64_t cstride = (int64_t)K * Np;
    for (int kk = wave; kk < kBoundSlots; kk += nw) {
        const int k = k0 + kk;
        if (k >= K) break;
        const int64_t u = unique[(int64_t)b * K + k];
        float c[RPL];
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const int n = lane + 64 * r;
            c[r] = (c_init && n < N) ? c_init[((int64_t)b * K + k) * cis + n] : 0.f;
        }
        float* o = out + ((int64_t)b * nc * K + k) * Np;
        auto store = [&](float* dst) {
#pragma unroll
            for (int r = 0; r < RPL; ++r) {
                const int n = lane + 64 * r;
                if (n < Np) dst[n] = n < N ? c[r] : 0.f;
            }
        };
        store(o);
        for (int j = 1; j < nc; ++j) {
            for (int ps = (j - 1) * Br; ps < j * Br; ps += 64) {
                const int len = min(64, j * Br - ps);
                const bool hit = lane < len && u >= 0 && tok[ps + lane] == u;
                uint64_t m = __ballot(hit);
                bool drop = false;
                if (doc_ids) {
                    uint64_t rb = bits64_at(rbits, ps);
                    if (len < 64) rb &= (1ull << len) - 1;
                    if (rb) {
                        const int rl = 63 - __builtin_clzll(rb);  // last change in the piece
                        drop = true;
                        m &= ~((1ull << rl) - 1);
                    }
                }
#pragma unroll
                for (int r = 0; r < RPL; ++r) c[r] = drop ? 0.f : c[r] * pow_steps(hi[r], lo[r], len);
                while (m) {  // uniform across the wave
                    const int p = __builtin_ctzll(m);
                    m &= m - 1;
#pragma unroll
                    for (int r = 0; r < RPL; ++r) c[r] += pow_steps(hi[r], lo[r], len - 1 - p);
                }
            }
            store(o + j * cstride);
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
    // token bits the radix sort orders by: those of vocab_size - 1 (ids are < vocab_size)
    int tok_bits = (wide ? 64 : 32) - pb;
    if (vocab_size > 0) {
        int vb = 1;
        while (vb < 63 && (vocab_size - 1) >> vb) ++vb;
        tok_bits = std::min(tok_bits, vb);
    }
    const bool vec4 = (N % 4) == 0;
    int slice_w = N >= 32 ? 32 : N;
    if (vec4) slice_w = (slice_w + 3) & ~3;
    const int ns = (N + slice_w - 1) / slice_w;
    // segment length: at most kMaxNonFinal non-final segments per sequence
    constexpr int kMaxNonFinal = 128;
    const int S = std::max(16, (L + kMaxNonFinal - 1) / kMaxNonFinal);
    const int nf_max = L / S;
    const int nH = (L - 1) / 64 + 1;
    const ScanLds lay(L, wide ? 8 : 4, kScanThreads, nf_max, slice_w, nH);
    if (lay.total > kMaxLds)
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_query_scan: L=%d with vocab %lld needs %zu B of LDS",
                    L, (long long)vocab_size, lay.total);
    dim3 grid(B, ns);
    hipStream_t st = (hipStream_t)stream;
#define MB_LAUNCH_SCAN(KT, V, DOCS)                                                            \
    do {                                                                                       \
        auto kfn = L <= 64 * kScanRoundsSmall * (kScanThreads / 64)                            \
                       ? ema_query_scan_kernel<KT, V, DOCS, kScanRoundsSmall>                  \
                       : ema_query_scan_kernel<KT, V, DOCS, kScanRoundsLarge>;                 \
        int rc = set_lds(kfn, lay.total);                                                      \
        if (rc) return rc;                                                                     \
        hipLaunchKernelGGL(kfn, grid, dim3(kScanThreads), lay.total, st, x, x_stride_b,        \
                           x_stride_l, L, rhos, N, c_init, c_init_keys, K, doc_ids, C_seq,     \
                           state_out, stamp_out, pb, tok_bits, slice_w, S, nf_max);            \
    } while (0)
#define MB_LAUNCH_SCAN_D(KT, V)                                     \
    do {                                                            \
        if (doc_ids) MB_LAUNCH_SCAN(KT, V, true);                   \
        else MB_LAUNCH_SCAN(KT, V, false);                          \
    } while (0)
    if (wide) {
        if (vec4) MB_LAUNCH_SCAN_D(uint64_t, 4); else MB_LAUNCH_SCAN_D(uint64_t, 1);
    } else {
        if (vec4) MB_LAUNCH_SCAN_D(uint32_t, 4); else MB_LAUNCH_SCAN_D(uint32_t, 1);
    }
#undef MB_LAUNCH_SCAN_D
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
    const int nc = L > 0 ? (L + Br - 1) / Br : 1;  // an empty sequence still stores c0 once
    const size_t lds = (size_t)L * 8 + (size_t)((L >> 6) + 2) * 8;
    if (lds > kMaxLds)
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_boundary_states: L=%d needs %zu B of LDS", L, lds);
    if (Np > 256)
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_boundary_states: Np=%d > 256", Np);
    dim3 grid(B, (K + kBoundSlots - 1) / kBoundSlots);
    hipStream_t st = (hipStream_t)stream;
#define MB_LAUNCH_BOUND(RPL)                                                                   \
    do {                                                                                       \
        auto kfn = ema_boundary_kernel<RPL>;                                                   \
        int rc = set_lds(kfn, lds);                                                            \
        if (rc) return rc;                                                                     \
        hipLaunchKernelGGL(kfn, grid, dim3(kBoundThreads), lds, st, x, x_stride_b, x_stride_l, \
                           L, unique, K, rhos, N, Br, nc, c_init, c_init_stride_k, doc_ids,    \
                           C_bounds, Np);                                                      \
    } while (0)
    if (Np <= 64) MB_LAUNCH_BOUND(1);
    else if (Np <= 128) MB_LAUNCH_BOUND(2);
    else MB_LAUNCH_BOUND(4);
#undef MB_LAUNCH_BOUND
    return check_launch("mb_ema_boundary_states");
}
