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
// After the sort, chain c is the sorted range [chain_start[c], chain_start[c+1]) of one
// token, and the recurrence along it, in pre-increment values C_j = C_seq at the chain's
// j-th position,
//   C_1 = c0 rho^t_1,   C_j = (C_{j-1} + 1) rho^(t_j - t_{j-1})
// is linear.  The sorted order is cut every S elements (S a power of two): lane group g
// walks the range [g S, (g + 1) S) in lockstep with the other groups of its wave, S steps
// for every group however the chains fall.  A range that starts inside a chain needs the
// chain's state at its start: pass A walks, for every cut m that falls inside a chain, the
// chain's piece that the cut closes, from zero, and keeps its local sum at the piece's last
// element j_m = m S - 1,
//   agg_m = sum_{j in piece, j < j_m} rho^(t_{j_m} - t_j),
// in LDS.  Pass B rebuilds a range's carry-in from the chain's earlier cuts,
//   P(m) = P(m') rho^(t_{j_m} - t_{j_m'}) + agg_m + 1     (post-increment state at t_{j_m}),
// (P := c0 at t = 0 before the first cut), which costs at most L/S steps.  With doc_ids, a
// piece that contains a document change drops its carry (flag kept beside the aggregate).

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
        st_stream4(dst, make_float4(v[0], v[1], v[2], v[3]));
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i)
            if (n0 + i < N) st_stream(dst + i, v[i]);
    }
}

// Makes every register of `a` ready here.  Vector-memory waits count loads and stores in
// one in-order counter, so a load's first use after some stores also waits for those
// stores; settling a chunk's loads before its stores leaves the walk with no such waits.
template <typename T, int n>
__device__ inline void settle(T (&a)[n]) {
#pragma unroll
    for (int i = 0; i < n; ++i) asm volatile("" : "+v"(a[i]));
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

// Radix sort rounds per wave (64 keys each): 2 cover L <= 2048 with 16 waves, 8 cover
// L <= 8192.  A thread holds at most MAXR tokens of its sequence.
constexpr int kScanRoundsSmall = 2;
constexpr int kScanRoundsLarge = 8;
// Loads issued before the sort so that its LDS phases hide their latency: c_init key ids
// (K <= 4 * 1024 in registers, more are fetched during the lookup) and power-table entries.
constexpr int kKeyPrefetch = 4;
constexpr int kTablePrefetch = 4;

// Byte offsets of the per-sequence index inside dynamic LDS.  The sorted keys take Lp =
// 2^ceil(log2 L) entries (the tail holds all-ones sentinels for the lookup); the radix
// sort's scratch overlaps everything after them.
// Hash grouping: a token with at least long_run(L) positions (at most kMaxLongRuns such
// tokens) is ranked through a position bitmap instead of by counting.
constexpr int kMaxLongRuns = 128;
// (T = ceil(L / kMaxLongRuns), at least 16: then at most L / T <= kMaxLongRuns runs reach T)
__host__ __device__ inline int long_run(int L) {
    const int t = (L + kMaxLongRuns - 1) / kMaxLongRuns;
    return t > 16 ? t : 16;
}

struct ScanLds {
    size_t keys, chain_start, elem_chain, chain_key, agg, aggr, lowT, highT, scan_scratch, chain_prev;
    size_t sort_b, sort_cnt;
    size_t htab, hcnt, hpre, hpos, hbits, hlpre, hnl;  // grouping by hash (lgTS > 0)
    size_t total;
    // rows of the power tables and of the cut aggregates hold 1 << lgRow floats (the slice
    // width rounded up to a power of two, so that row addressing is a shift)
    __host__ __device__ ScanLds(int L, int Lp, int key_bytes, int nthr, int ncut, int nH, int lgRow,
                                int lgTS = 0, bool piece = false) {
        auto al = [](size_t o) { return (o + 15) & ~(size_t)15; };
        keys = 0;
        size_t o = al((size_t)Lp * key_bytes);
        const size_t after_keys = o;
        chain_start = o;  o += (size_t)(L + 1) * 2;
        elem_chain = o;   o += (size_t)L * 2;
        chain_key = o = al(o);
        o += (size_t)L * 4;
        agg = o;          o += (size_t)(ncut + 1) * 4 << lgRow;
        aggr = o;         o += (size_t)(ncut + 1) * 4;
        lowT = o = al(o);
        highT = lowT + ((size_t)64 * 4 << lgRow);
        o = highT + ((size_t)nH * 4 << lgRow);
        scan_scratch = o = al(o);
        o += 64 * 4;
        // piece mode: per chain, the last position of its token before the piece (or -1)
        chain_prev = o = al(o);
        if (piece) o += (size_t)(L + 1) * 4;
        total = al(o);
        sort_b = after_keys;
        sort_cnt = al(sort_b + (size_t)L * key_bytes);
        htab = hcnt = hpre = hpos = hbits = hlpre = hnl = 0;
        if (lgTS > 0) {  // the hash tables live beside the index; no sort scratch
            const size_t W = (size_t)(L + 63) / 64;  // bitmap words of a long run
            htab = total;
            hcnt = htab + ((size_t)4 << lgTS);
            hpre = hcnt + ((size_t)4 << lgTS);
            hpos = hpre + ((size_t)4 << lgTS);
            hbits = al(hpos + (size_t)(L + 8) * 2);
            hlpre = hbits + kMaxLongRuns * W * 8;
            hnl = al(hlpre + kMaxLongRuns * W * 2);
            total = al(hnl + 4);
        } else {
            const size_t sort_end = al(sort_cnt + (size_t)(4 * nthr + 64) * 4);
            if (sort_end > total) total = sort_end;
        }
    }
};

// Table slot of a 32-bit token key (multiplicative hash, top lgTS bits).
__device__ inline int hash_slot(uint32_t key, int lgTS) {
    return (int)((key * 0x9E3779B1u) >> (32 - lgTS));
}
constexpr uint32_t kHashEmpty = 0xFFFFFFFFu;

// Query scan: one workgroup per (sequence b, slice of slice_w decay rates).
//   0. this thread's tokens, c_init key ids and power-table entries go to registers;
//   1. keys = (token << pb | position) in position order, stably radix-sorted by token;
//   2. one block scan numbers the chains (element -> chain map, chain starts); the power
//      tables go to LDS;
//   3. c_init keys are matched to their chains (the last duplicate wins);
//   4. each lane group gathers its range's first chunk and issues its c_init row loads;
//      pass A computes the cut aggregates meanwhile;
//   5. pass B: every group walks its range and writes the C_seq rows (and the final state
//      and stamp at each chain's last element).
// rho^d comes from two LDS tables per rate, rho^(d mod 64) * rho^(64 floor(d / 64)),
// each entry a correctly rounded float of a double-precision power.
// PIECE: the launch scans steps [T0, T0 + L) of sequences of Ltot steps (longer sequences
// run as consecutive pieces, one launch each): a chain whose token occurred before T0 starts
// from that occurrence's post-increment state C_seq[b, s] + 1 decayed by rho^(T0 - s), with
// s = last_pos[b, token] (kept by query_piece_last_kernel between launches), and a key's c0
// enters decayed by rho^T0; positions and stamps are absolute.  Without PIECE, T0 = 0 and
// Ltot = L.
template <typename KeyT, int VEC, bool DOCS, int MAXR, bool HASH, bool PIECE = false>
__global__ void __launch_bounds__(kScanThreads)
ema_query_scan_kernel(const int64_t* __restrict__ x, int64_t sb, int64_t sl, int L,
                      const float* __restrict__ rhos, int N, const float* __restrict__ c_init,
                      const int64_t* __restrict__ c_init_keys, int K,
                      const int64_t* __restrict__ doc_ids, float* __restrict__ C_seq,
                      float* state_out, int32_t* __restrict__ stamp_out, int pb, int tok_bits,
                      int slice_w, int lgS, int ncut, int lgTS, int T0, int Ltot,
                      const int32_t* __restrict__ last_pos, int64_t V) {
    static_assert(!HASH || sizeof(KeyT) == 4, "hash grouping keys are 32-bit tokens");
    // elements per unrolled chunk of a pass-B walk; their c_init rows (and with doc_ids
    // their documents) sit in registers
    constexpr int CH = DOCS ? 4 : 8;
    extern __shared__ __align__(16) unsigned char smem[];
    const int b = blockIdx.x;
    const int slice = blockIdx.y;
    const int nthr = blockDim.x;
    const int nH = (L - 1) / 64 + 1;
    const int Lp = 1 << pb;
    const int lgRow = ceil_log2(slice_w);
    const ScanLds lay(L, Lp, (int)sizeof(KeyT), nthr, ncut, nH, lgRow, HASH ? lgTS : 0, PIECE);
    KeyT* keys = reinterpret_cast<KeyT*>(smem + lay.keys);
    uint16_t* chain_start = reinterpret_cast<uint16_t*>(smem + lay.chain_start);
    uint16_t* elem_chain = reinterpret_cast<uint16_t*>(smem + lay.elem_chain);
    int* chain_key = reinterpret_cast<int*>(smem + lay.chain_key);
    float* agg = reinterpret_cast<float*>(smem + lay.agg);
    int* aggr = reinterpret_cast<int*>(smem + lay.aggr);
    float* lowT = reinterpret_cast<float*>(smem + lay.lowT);
    float* highT = reinterpret_cast<float*>(smem + lay.highT);
    int* scratch = reinterpret_cast<int*>(smem + lay.scan_scratch);
    int* chain_prev = reinterpret_cast<int*>(smem + lay.chain_prev);
    const int S = 1 << lgS;
    if (!PIECE) {
        T0 = 0;
        Ltot = L;
    }
    // last position of `token` before T0, or -1 (ids outside [0, V) count as never seen)
    auto prev_of = [&](uint64_t token) -> int {
        return PIECE && token < (uint64_t)V ? last_pos[(int64_t)b * V + (int64_t)token] : -1;
    };

    // 0. early loads: tokens, c_init key ids, rates; then the power-table entries
    // (double-precision work that overlaps the loads' latency)
    uint64_t tokv[MAXR];
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
        const int i = threadIdx.x + r * nthr;
        tokv[r] = i < L ? (uint64_t)x[(int64_t)b * sb + (int64_t)(T0 + i) * sl] : 0;
    }
    int64_t pre_key[kKeyPrefetch];
#pragma unroll
    for (int r = 0; r < kKeyPrefetch; ++r) {
        const int k = threadIdx.x + r * nthr;
        pre_key[r] = k < K ? c_init_keys[(int64_t)b * K + k] : (int64_t)-1;
    }
    const int n_tab = (64 + nH) * slice_w;
    auto table_value = [](int j, double rho) -> float {
        return (float)(j < 64 ? powi(rho, j) : powi(powi(rho, 64), j - 64));
    };
    auto table_rate = [&](int i) { return slice * slice_w + i % slice_w; };
    float pre_tab[kTablePrefetch];
#pragma unroll
    for (int r = 0; r < kTablePrefetch; ++r) {
        const int i = threadIdx.x + r * nthr;
        pre_tab[r] = rhos[min(table_rate(i), N - 1)];
    }
    // The four loads issue together and are waited for once, here: left to itself the
    // compiler moves each load into the guarded computation below and waits for it there,
    // one memory round trip after the other.
    settle(pre_tab);
#pragma unroll
    for (int r = 0; r < kTablePrefetch; ++r) {
        const int i = threadIdx.x + r * nthr;
        if (!(i < n_tab && table_rate(i) < N)) pre_tab[r] = 0.f;
    }
    const int64_t doc0 = DOCS ? doc_ids[(int64_t)b * Ltot] : 0;
#pragma unroll
    for (int r = 0; r < kTablePrefetch; ++r) {
        const int i = threadIdx.x + r * nthr;
        pre_tab[r] = i < n_tab ? table_value(i / slice_w, (double)pre_tab[r]) : 0.f;
    }

    // Power tables into LDS (highT follows lowT: entry j >= 64 is rho^(64 (j - 64))).
    auto store_tables = [&]() {
        auto table_slot = [&](int i) { return ((i / slice_w) << lgRow) + i % slice_w; };
#pragma unroll
        for (int r = 0; r < kTablePrefetch; ++r) {
            const int i = threadIdx.x + r * nthr;
            if (i < n_tab) lowT[table_slot(i)] = pre_tab[r];
        }
        for (int i = threadIdx.x + kTablePrefetch * nthr; i < n_tab; i += nthr)
            lowT[table_slot(i)] = table_rate(i) < N ? table_value(i / slice_w, (double)rhos[table_rate(i)]) : 0.f;
    };
    // 3'. (hash path) each key row seeds the chain of its token by probing the token table
    // (every taken slot holds a token of the sequence); the last duplicate key wins, as a
    // sequential scatter_ leaves it (triton_ema_query.py:146-149).  Token ids compare as the
    // keys hold them: a key id above tok_lim or negative is never matched.
    auto hash_lookup = [&]() {
        const uint64_t tok_lim = (uint64_t)(KeyT)~KeyT(0) >> pb;
        const uint32_t* htab = reinterpret_cast<const uint32_t*>(smem + lay.htab);
        const int* hpre = reinterpret_cast<const int*>(smem + lay.hpre);
        const int TS = 1 << lgTS;
        for (int kb = threadIdx.x; kb < K; kb += kKeyPrefetch * nthr) {
#pragma unroll
            for (int r = 0; r < kKeyPrefetch; ++r) {
                const int k = kb + r * nthr;
                const int64_t u = kb == (int)threadIdx.x ? pre_key[r]
                                                         : (k < K ? c_init_keys[(int64_t)b * K + k] : (int64_t)-1);
                if (k < K && u >= 0 && (uint64_t)u <= tok_lim) {
                    const uint32_t key = (uint32_t)u;
                    int h = hash_slot(key, lgTS);
                    uint32_t cur;
                    // ends at an empty slot: at most L of the TS >= 2L slots are taken
                    while ((cur = htab[h]) != kHashEmpty && cur != key) h = (h + 1) & (TS - 1);
                    if (cur == key) atomicMax(&chain_key[hpre[h] >> 16], k);
                }
            }
        }
    };

    if constexpr (HASH) {
        // 1'. group the positions by token without sorting: a hash table of 2^lgTS >= 2L
        // slots gives each distinct token a slot (linear probing) and its count; one block
        // scan of (count, nonempty) packed in an int (low 16 bits: positions before the slot,
        // high 16 bits: chains before it) gives every token its run [base, base + count) of
        // the grouped order and its chain number.  The atomic placement leaves a run
        // unordered, so each position then counts the run's earlier positions (runs are
        // short except for the most frequent tokens) and lands at base + that rank: every
        // chain lists its positions in order, as the passes below need.  The key word keeps
        // the chain number where the sort keeps the token.
        uint32_t* htab = reinterpret_cast<uint32_t*>(smem + lay.htab);
        int* hcnt = reinterpret_cast<int*>(smem + lay.hcnt);
        int* hpre = reinterpret_cast<int*>(smem + lay.hpre);
        uint16_t* hpos = reinterpret_cast<uint16_t*>(smem + lay.hpos);
        uint64_t* hbits = reinterpret_cast<uint64_t*>(smem + lay.hbits);
        uint16_t* hlpre = reinterpret_cast<uint16_t*>(smem + lay.hlpre);
        int* hnl = reinterpret_cast<int*>(smem + lay.hnl);
        const int TS = 1 << lgTS;
        const int W = (L + 63) >> 6;
        const int T = long_run(L);
        for (int i = threadIdx.x; i < TS; i += nthr) {
            htab[i] = kHashEmpty;
            hcnt[i] = 0;
        }
        for (int i = threadIdx.x; i < kMaxLongRuns * W; i += nthr) hbits[i] = 0;
        if (threadIdx.x == 0) *hnl = 0;
        // the power tables and the stamps' initial -1 now: nothing of the grouping overlaps
        // them, and their stores then need no phase (and barrier) of their own
        store_tables();
        if (stamp_out && slice == 0 && T0 == 0)
            for (int k = threadIdx.x; k < K; k += nthr) stamp_out[(int64_t)b * K + k] = -1;
        __syncthreads();
        const uint32_t tokmask = 0xFFFFFFFFu >> pb;
        int slot[MAXR], urank[MAXR];
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
            const int i = threadIdx.x + r * nthr;
            slot[r] = 0;
            urank[r] = 0;
            if (i < L) {
                const uint32_t key = (uint32_t)tokv[r] & tokmask;  // never kHashEmpty (pb >= 1)
                int h = hash_slot(key, lgTS);
                // ends: at most L of the TS >= 2L slots are ever taken
                while (true) {
                    const uint32_t old = atomicCAS(&htab[h], kHashEmpty, key);
                    if (old == kHashEmpty || old == key) break;
                    h = (h + 1) & (TS - 1);
                }
                slot[r] = h;
                urank[r] = atomicAdd(&hcnt[h], 1);
            }
        }
        __syncthreads();
        const int per = (TS + nthr - 1) / nthr;
        const int s0 = threadIdx.x * per;
        int sum = 0;
        for (int q = 0; q < per; ++q) {
            const int c = s0 + q < TS ? hcnt[s0 + q] : 0;
            sum += c + (c > 0 ? 1 << 16 : 0);
        }
        int total;
        int run = block_exclusive_scan(sum, scratch, total);
        for (int q = 0; q < per; ++q) {
            if (s0 + q < TS) {
                const int c = hcnt[s0 + q];
                hpre[s0 + q] = run;
                run += c + (c > 0 ? 1 << 16 : 0);
                // a long run gets a bitmap (its number + 1 above the count; at most L / T
                // <= kMaxLongRuns runs have T positions)
                if (c >= T) hcnt[s0 + q] = c | ((atomicAdd(hnl, 1) + 1) << 16);
                if (c > 0) {  // this token's chain: its start and, until a key claims it, no key
                    const int pre = hpre[s0 + q];
                    chain_start[pre >> 16] = (uint16_t)(pre & 0xFFFF);
                    chain_key[pre >> 16] = -1;
                }
            }
        }
        if (threadIdx.x == 0) chain_start[total >> 16] = (uint16_t)L;
        __syncthreads();
        hash_lookup();
        // short runs: unordered placement; long runs: one bit per position
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
            const int i = threadIdx.x + r * nthr;
            if (i < L) {
                const int lid = hcnt[slot[r]] >> 16;
                if (lid) atomicOr(&hbits[(lid - 1) * W + (i >> 6)], 1ull << (i & 63));
                else hpos[(hpre[slot[r]] & 0xFFFF) + urank[r]] = (uint16_t)i;
            }
        }
        __syncthreads();
        {  // positions of a long run before each of its bitmap words (W <= 64: a wave per run)
            const int lane = threadIdx.x & 63;
            const int nl = *hnl;
            for (int lr = threadIdx.x >> 6; lr < nl; lr += nthr >> 6) {
                const int c = lane < W ? __popcll(hbits[lr * W + lane]) : 0;
                const int ex = wave_inclusive_scan(c) - c;
                if (lane < W) hlpre[lr * W + lane] = (uint16_t)ex;
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
            const int i = threadIdx.x + r * nthr;
            if (i < L) {
                const int pre = hpre[slot[r]];
                const int base = pre & 0xFFFF;
                const int cid = pre >> 16;
                const int cw = hcnt[slot[r]];
                int rank = 0;
                if (cw >> 16) {  // the run's positions below i: bitmap words before, then bits
                    const int wi = ((cw >> 16) - 1) * W + (i >> 6);
                    rank = (int)hlpre[wi] + __popcll(hbits[wi] & ((1ull << (i & 63)) - 1ull));
                } else {  // fewer than T positions: count the earlier ones, eight reads
                    // in flight at a time (hpos has 8 spare entries past L)
                    for (int q = 0; q < cw; q += 8) {
                        uint16_t v[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[e] = hpos[base + q + e];
#pragma unroll
                        for (int e = 0; e < 8; ++e) rank += (q + e < cw && v[e] < i) ? 1 : 0;
                    }
                }
                const int j = base + rank;
                keys[j] = (KeyT)cid << pb | (KeyT)i;
                elem_chain[j] = (uint16_t)cid;
                if (PIECE && rank == 0) chain_prev[cid] = prev_of(tokv[r]);  // the chain's head
            }
        }
        for (int i = L + threadIdx.x; i < Lp; i += nthr) keys[i] = ~KeyT(0);
    } else {
    // 1. sorted (token, position) keys, then all-ones sentinels up to Lp
    {
        const KeyT tokmask = (pb == 0) ? ~KeyT(0) : ((~KeyT(0)) >> pb);
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
            const int i = threadIdx.x + r * nthr;
            if (i < L) keys[i] = ((KeyT)tokv[r] & tokmask) << pb | (KeyT)i;
        }
        __syncthreads();
        KeyT* sorted = block_radix_sort<MAXR>(keys, reinterpret_cast<KeyT*>(smem + lay.sort_b),
                                              reinterpret_cast<int*>(smem + lay.sort_cnt), L, pb,
                                              tok_bits);
        if (sorted != keys) {
            for (int i = threadIdx.x; i < L; i += nthr) keys[i] = sorted[i];
            __syncthreads();
        }
        for (int i = L + threadIdx.x; i < Lp; i += nthr) keys[i] = ~KeyT(0);
    }

    }

    // 2. chain ids from one scan of head counts, element -> chain map, chain starts (from
    // the sort); the power tables (highT follows lowT: entry j >= 64 is rho^(64 (j - 64)))
    {
        if constexpr (!HASH) {
        const int per = (L + nthr - 1) / nthr;
        const int i0 = threadIdx.x * per;
        const int i1 = min(i0 + per, L);
        auto chain_head = [&](int i) { return i == 0 || (keys[i] >> pb) != (keys[i - 1] >> pb); };
        int cnt = 0;
        for (int i = i0; i < i1; ++i) cnt += chain_head(i);
        int n_chains;
        int c = block_exclusive_scan(cnt, scratch, n_chains);
        for (int i = i0; i < i1; ++i) {
            if (chain_head(i)) {
                chain_start[c] = (uint16_t)i;
                chain_key[c] = -1;
                if (PIECE) chain_prev[c] = prev_of((uint64_t)(keys[i] >> pb));
                ++c;
            }
            elem_chain[i] = (uint16_t)(c - 1);
        }
        if (threadIdx.x == 0) chain_start[n_chains] = (uint16_t)L;
        }
        if constexpr (!HASH) {
            store_tables();
            if (stamp_out && slice == 0 && T0 == 0)
                for (int k = threadIdx.x; k < K; k += nthr) stamp_out[(int64_t)b * K + k] = -1;
        }
        __syncthreads();
    }

    // 3. each key row seeds the chain of its token; the last duplicate key wins, as a
    // sequential scatter_ leaves it (triton_ema_query.py:146-149).  Lower bounds by halving
    // steps over the Lp sentinel-padded keys: no bounds test, so a thread's lookups keep
    // their LDS reads in flight together.
    // Token ids compare in KeyT.  A key id that no sorted token can equal (negative, or
    // wider than the key layout's token field) searches for all-ones and is never matched.
    const uint64_t tok_lim = (uint64_t)(KeyT)~KeyT(0) >> pb;  // largest token the keys hold
    if constexpr (!HASH)  // (the hash path matched its keys right after the grouping's scan)
    for (int kb = threadIdx.x; kb < K; kb += kKeyPrefetch * nthr) {
        KeyT tok[kKeyPrefetch];
        int lo[kKeyPrefetch];
        bool valid[kKeyPrefetch];
#pragma unroll
        for (int r = 0; r < kKeyPrefetch; ++r) {
            const int k = kb + r * nthr;
            const int64_t u = kb == (int)threadIdx.x ? pre_key[r]
                                                     : (k < K ? c_init_keys[(int64_t)b * K + k] : (int64_t)-1);
            valid[r] = k < K && u >= 0 && (uint64_t)u <= tok_lim;
            tok[r] = valid[r] ? (KeyT)u : ~KeyT(0);
            lo[r] = 0;  // every key before lo is below tok
        }
        for (int step = Lp >> 1; step > 0; step >>= 1) {
#pragma unroll
            for (int r = 0; r < kKeyPrefetch; ++r)
                lo[r] += (KeyT)(keys[lo[r] + step - 1] >> pb) < tok[r] ? step : 0;
        }
#pragma unroll
        for (int r = 0; r < kKeyPrefetch; ++r) {
            lo[r] += (KeyT)(keys[lo[r]] >> pb) < tok[r] ? 1 : 0;
            if (valid[r] && lo[r] < L && (KeyT)(keys[lo[r]] >> pb) == tok[r])
                atomicMax(&chain_key[elem_chain[lo[r]]], kb + r * nthr);
        }
    }
    if constexpr (!HASH) __syncthreads();

    const int lanes = slice_w / VEC;
    const int groups = nthr / lanes;
    const int g = threadIdx.x / lanes;
    const int lane_r = (threadIdx.x % lanes) * VEC;  // rate offset inside the slice
    const int n0 = slice * slice_w + lane_r;
    const bool active = n0 < N && g < groups;
    const KeyT posmask = (pb == 0) ? KeyT(0) : ((KeyT(1) << pb) - 1);
    auto pos_of = [&](int j) { return (int)(keys[j] & posmask); };
    auto doc_of = [&](int pos) { return doc_ids[(int64_t)b * Ltot + T0 + pos]; };
    auto doc_abs = [&](int pos) { return doc_ids[(int64_t)b * Ltot + pos]; };
    // rho^d for this lane's VEC rates
    auto powv = [&](int d, float* pw) {
        const float* lo = lowT + ((d & 63) << lgRow) + lane_r;
        const float* hi = highT + ((d >> 6) << lgRow) + lane_r;
        if (VEC == 4) {
            const float4 a = *reinterpret_cast<const float4*>(lo);
            const float4 h = *reinterpret_cast<const float4*>(hi);
            pw[0] = a.x * h.x; pw[1] = a.y * h.y; pw[2] = a.z * h.z; pw[3] = a.w * h.w;
        } else {
#pragma unroll
            for (int v = 0; v < VEC; ++v) pw[v] = lo[v] * hi[v];
        }
    };
    // row offsets as 24-bit products from per-sequence bases (the host checks L * N and
    // K * N against 2^31 and K against 2^24)
    float* const Cb = C_seq + ((int64_t)b * Ltot + T0) * N;
    const float* const c0b = c_init + (int64_t)b * K * N;
    float* const stb = state_out ? state_out + (int64_t)b * K * N : nullptr;
    auto row = [&](int r) { return (int)__umul24((unsigned)r, (unsigned)N) + n0; };

    // 4. this group's sorted range [ra, re) (the host picks S so that no group has two),
    // its first chunk's walk starts and their c_init rows.  A walk starts at the range's
    // first element and at every chain head; `key` -1 marks a start without a key row.
    const int ra = g * S;
    const int re = g < groups && ra < L ? min(ra + S, L) : ra;
    Vec<VEC> c0v[CH];
    int keyv[CH];
    int64_t docv[CH];
    // PIECE: the chain's previous occurrence before T0 (-1: none) and, with doc_ids, the
    // document its carry belongs to (that occurrence's, or the sequence's first)
    int prevv[CH];
    int64_t pdocv[CH];
    uint32_t startm = 0, lastm = 0;  // bit e: element c + e starts a walk / ends its chain
    auto gather = [&](int c) {
        startm = lastm = 0;
        int prev = c > 0 ? elem_chain[c - 1] : -1;
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int j = c + e;
            const bool in = j < re;
            const int cid = in ? elem_chain[j] : prev;
            const int nxt = in && j + 1 < L ? elem_chain[j + 1] : -1;
            const bool start = in && (j == ra || cid != prev);
            startm |= (start ? 1u : 0u) << e;
            lastm |= (in && nxt != cid ? 1u : 0u) << e;
            keyv[e] = start ? chain_key[cid] : -1;
            prevv[e] = PIECE && start ? chain_prev[cid] : -1;
            if (PIECE && prevv[e] >= 0)  // the carry: C_seq at the previous occurrence
                c0v[e] = load_vec<VEC>(C_seq + ((int64_t)b * Ltot + prevv[e]) * N + n0, active, n0, N);
            else
                c0v[e] = load_vec<VEC>(c0b + row(keyv[e] >= 0 ? keyv[e] : 0), start && keyv[e] >= 0 && active,
                                       n0, N);
            if (DOCS) docv[e] = in ? doc_of(pos_of(j)) : 0;
            if (DOCS && PIECE) pdocv[e] = prevv[e] >= 0 ? doc_abs(prevv[e]) : doc0;
            prev = cid;
        }
    };
    if (ra < re) gather(ra);

    // pass A: the aggregate of the chain piece that each interior cut closes (cut g + 1
    // closes this group's range)
    for (int m = 1 + g; g < groups && m <= ncut; m += groups) {
        const int last = m << lgS;
        const int cc = elem_chain[last - 1];
        if (cc != elem_chain[last]) continue;  // a chain starts at the cut
        const int cs = chain_start[cc];
        const int beg = max(cs, last - S);
        float h[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) h[v] = 0.f;
        int reset = 0;
        int tp = pos_of(beg);
        int64_t dprev = 0;
        if (DOCS) {
            const bool first = beg == cs;
            const int cprev = PIECE ? chain_prev[cc] : -1;
            const bool has_prev = !first || chain_key[cc] >= 0 || cprev >= 0;
            const int64_t dcur = doc_of(tp);
            const int64_t dref = first ? (cprev >= 0 ? doc_abs(cprev) : doc0) : doc_of(pos_of(beg - 1));
            reset = has_prev && dref != dcur;
            dprev = dcur;
        }
        int tn = pos_of(min(beg + 1, last - 1));
        for (int j = beg + 1; j < last; ++j) {
            const int t = tn;
            tn = pos_of(min(j + 1, last - 1));  // next position, read one step ahead
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
        for (int v = 0; v < VEC; ++v) agg[(m << lgRow) + lane_r + v] = h[v];
        if (DOCS && lane_r == 0) aggr[m] = reset;
    }
    __syncthreads();

    // 5. pass B: the walk, CH elements per chunk; P is the post-increment state at time tp.
    // The range's first element starts from its chain's c0 and, when the range starts inside
    // the chain, the carries through the chain's cuts in (cs, ra].
    // PIECE: a chain's start state at the piece's step 0 (tp = 0): its previous occurrence's
    // C_seq + 1, or its key's c0, decayed over the steps since (log2 rho split in two floats).
    float l2hi[VEC], l2lo[VEC];
    if (PIECE) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
            l2hi[v] = l2lo[v] = 0.f;
            if (n0 + v < N) log2_split(rhos[n0 + v], l2hi[v], l2lo[v]);
        }
    }
    auto seed = [&](int e, float* Pv) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) Pv[v] = c0v[e].v[v];
        if (PIECE && T0 > 0) {
            const bool carry = prevv[e] >= 0;
            const int d = T0 - (carry ? prevv[e] : 0);
#pragma unroll
            for (int v = 0; v < VEC; ++v) Pv[v] = (Pv[v] + (carry ? 1.0f : 0.0f)) * pow_steps(l2hi[v], l2lo[v], d);
        }
    };
    float P[VEC];
    seed(0, P);
    int tp = 0;
    int key = keyv[0];
    bool has_prev = key >= 0 || prevv[0] >= 0;
    int64_t dprev = DOCS && PIECE ? pdocv[0] : doc0;
    if (ra < re) {
        const int cs = chain_start[elem_chain[ra]];
        for (int m = (cs >> lgS) + 1; m <= g; ++m) {
            const int tl = pos_of((m << lgS) - 1);
            const bool drop = DOCS && aggr[m];
            float pw[VEC];
            powv(tl - tp, pw);
#pragma unroll
            for (int v = 0; v < VEC; ++v)
                P[v] = (drop ? 0.f : P[v] * pw[v]) + agg[(m << lgRow) + lane_r + v] + 1.0f;
            tp = tl;
        }
        if (DOCS && ra > cs) {
            dprev = doc_of(tp);
            has_prev = true;
        }
        startm &= ~1u;
    }
    for (int c = ra; c < re; c += CH) {
        if (c != ra) gather(c);
#pragma unroll
        for (int e = 0; e < CH; ++e) settle(c0v[e].v);
        if (DOCS) settle(docv);
        int tn = pos_of(c);
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int j = c + e;
            if (j < re) {
                const int t = tn;
                tn = pos_of(min(j + 1, re - 1));  // next position, read one step ahead
                if ((startm >> e) & 1) {
                    seed(e, P);
                    tp = 0;
                    key = keyv[e];
                    has_prev = key >= 0 || prevv[e] >= 0;
                    dprev = DOCS && PIECE ? pdocv[e] : doc0;
                }
                float cv[VEC];
                powv(t - tp, cv);
#pragma unroll
                for (int v = 0; v < VEC; ++v) cv[v] *= P[v];
                if (DOCS) {
                    const int64_t dcur = docv[e];
                    if (has_prev && dcur != dprev) {
#pragma unroll
                        for (int v = 0; v < VEC; ++v) cv[v] = 0.f;
                    }
                    dprev = dcur;
                    has_prev = true;
                }
                if (active && t < L) store_vec<VEC>(Cb + row(t), cv, n0, N);
#pragma unroll
                for (int v = 0; v < VEC; ++v) P[v] = cv[v] + 1.0f;
                tp = t;
                if (((lastm >> e) & 1) && key >= 0) {
                    if (stb && active) store_vec<VEC>(stb + row(key), P, n0, N);
                    if (stamp_out && slice == 0 && lane_r == 0) stamp_out[(int64_t)b * K + key] = T0 + t;
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
// and the occurrences before its last change.  No sort is needed.  A wave advances its
// eight slots together, chunk by chunk, so the workgroup writes each chunk's 64
// consecutive state rows (16 KB) at about the same time (measured at configuration 2:
// 32 slots per workgroup 48.2 us, 64 slots 39.9 us, 128 slots 42.5 us).

constexpr int kBoundThreads = 512;
constexpr int kBoundSlots = 64;
constexpr int kBoundWin = 8192;  // tokens staged in LDS at a time

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
    // The tokens (and document-change bits) of a window [w0, w0 + WL) of the sequence sit in
    // LDS: the whole sequence when L <= kBoundWin, else windows that move forward as the
    // pieces reach their end (all waves walk the same pieces, so they move together).
    const int WL = min(L, kBoundWin);
    const int nwords = (WL >> 6) + 2;
    int64_t* tok = reinterpret_cast<int64_t*>(smem);                 // [WL]
    uint64_t* rbits = reinterpret_cast<uint64_t*>(tok + WL);         // [nwords] document changes
    const int b = blockIdx.x;
    const int k0 = blockIdx.y * kBoundSlots;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int nw = blockDim.x >> 6;
    constexpr int SPW = kBoundSlots / (kBoundThreads / 64);  // slots per wave
    static_assert(kBoundSlots % (kBoundThreads / 64) == 0, "whole slots per wave");

    // The wave's slot ids and initial states first: vector-memory waits count loads and
    // stores in one in-order counter, so a slot's loads issued after the previous slot's
    // stores would wait for those stores too.
    int64_t uu[SPW];
    float ci[SPW][RPL];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        const int k = k0 + wave + s * (kBoundThreads / 64);
        uu[s] = k < K ? unique[(int64_t)b * K + k] : (int64_t)-1;
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const int n = lane + 64 * r;
            ci[s][r] = (c_init && k < K && n < N) ? c_init[((int64_t)b * K + k) * cis + n] : 0.f;
        }
    }

    // Stages the window starting at w0: tok[i] = x[w0 + i]; bit i: the document changes at
    // step w0 + i (doc[p] != doc[p - 1], p >= 1).
    int w0 = 0;
    auto stage = [&](int start) {
        w0 = start;
        for (int i = threadIdx.x; i < WL; i += blockDim.x)
            tok[i] = w0 + i < L ? x[(int64_t)b * sb + (int64_t)(w0 + i) * sl] : (int64_t)-1;
        for (int w = wave; w < nwords; w += nw) {
            const int p = w0 + 64 * w + lane;
            bool chg = false;
            if (doc_ids && p >= 1 && p < L)
                chg = doc_ids[(int64_t)b * L + p] != doc_ids[(int64_t)b * L + p - 1];
            const uint64_t m = __ballot(chg);
            if (lane == 0) rbits[w] = m;
        }
    };
    stage(0);
    float hi[RPL], lo[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        hi[r] = 0.f;
        lo[r] = 0.f;
        const int n = lane + 64 * r;
        if (n < N) log2_split(rhos[n], hi[r], lo[r]);
    }
    // rho^64, the decay over a whole piece, as a float pair (hi + lo): the state is scaled by
    // it once per piece, so a rounding of rho^64 itself would bias it by the same factor every
    // piece (1.2e-5 relative by step 16384 in a single float); the pair leaves the per-piece
    // rounding of the product, which does not accumulate in one direction.
    // A chunk of Br steps is walked as pieces of 64 and one last piece of brem steps, so
    // these are the only two lengths (brem = 64 when 64 divides Br).
    const int brem = Br - 64 * ((Br - 1) / 64);
    float p64[RPL], p64l[RPL], prem[RPL], preml[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
        const int n = lane + 64 * r;
        const double l2 = n < N ? log2((double)rhos[n]) : 0.0;
        const double pd = n < N ? exp2(64.0 * l2) : 0.0;
        const double pr = n < N ? exp2((double)brem * l2) : 0.0;
        p64[r] = (float)pd;
        p64l[r] = (float)(pd - (double)p64[r]);
        prem[r] = (float)pr;
        preml[r] = (float)(pr - (double)prem[r]);
    }
    __syncthreads();

    const int64_t cstride = (int64_t)K * Np;
    // Chunk-outer, slot-inner: the wave advances its SPW slots (independent chains) by one
    // chunk at a time, so the workgroup writes chunk j's 32 consecutive rows together and
    // one token read per piece serves all SPW slots.  Each slot's state sees the same
    // operations in the same order as a slot walked alone.
    float c[SPW][RPL];
    float* o[SPW];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
        const int k = k0 + wave + s * (kBoundThreads / 64);
        o[s] = k < K ? out + ((int64_t)b * nc * K + k) * Np : nullptr;
#pragma unroll
        for (int r = 0; r < RPL; ++r) c[s][r] = ci[s][r];
    }
    auto store = [&](int s, int64_t off) {
        if (!o[s]) return;  // (uniform: a slot past K)
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
            const int n = lane + 64 * r;
            if (n < Np) o[s][off + n] = n < N ? c[s][r] : 0.f;
        }
    };
#pragma unroll
    for (int s = 0; s < SPW; ++s) store(s, 0);
    // Pieces run back to back (the next starts at ps + len); each piece's tokens are read
    // one piece ahead, so the LDS read is not on the chain of state updates.
    const int pend = (nc - 1) * Br;
    int64_t tnext = (pend > 0 && lane < L) ? tok[lane] : (int64_t)-1;
    for (int j = 1; j < nc; ++j) {
        for (int ps = (j - 1) * Br; ps < j * Br; ps += 64) {
            // a piece and the next one read [ps, ps + 128): move the window to start at ps
            // when that runs past it (the current piece's tokens were read one piece ahead;
            // every wave is done with the old window at the barrier)
            if (ps + 128 > w0 + WL && w0 + WL < L) {
                __syncthreads();
                stage(ps);
                __syncthreads();
            }
            const int len = min(64, j * Br - ps);
            const int64_t tv = tnext;
            const int pn = ps + len;
            tnext = (pn < pend && pn + lane < L) ? tok[pn + lane - w0] : (int64_t)-1;
            bool drop = false;
            uint64_t keep = ~0ull;
            if (doc_ids) {
                uint64_t rb = bits64_at(rbits, ps - w0);
                if (len < 64) rb &= (1ull << len) - 1;
                if (rb) {
                    const int rl = 63 - __builtin_clzll(rb);  // last change in the piece
                    drop = true;
                    keep = ~((1ull << rl) - 1);
                }
            }
            float pw[RPL], pwl[RPL];
#pragma unroll
            for (int r = 0; r < RPL; ++r) {  // len is 64 or brem
                pw[r] = len == 64 ? p64[r] : prem[r];
                pwl[r] = len == 64 ? p64l[r] : preml[r];
            }
#pragma unroll
            for (int s = 0; s < SPW; ++s) {
                const bool hit = lane < len && uu[s] >= 0 && tv == uu[s];
                uint64_t m = __ballot(hit) & keep;
#pragma unroll
                for (int r = 0; r < RPL; ++r)
                    c[s][r] = drop ? 0.f : __builtin_fmaf(c[s][r], pw[r], c[s][r] * pwl[r]);
                while (m) {  // uniform across the wave
                    const int p = __builtin_ctzll(m);
                    m &= m - 1;
#pragma unroll
                    for (int r = 0; r < RPL; ++r) c[s][r] += pow_steps(hi[r], lo[r], len - 1 - p);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < SPW; ++s) store(s, j * cstride);
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

namespace mb {

// Pieces of a long query scan: steps [T0, T0 + kScanPiece) per launch (hash grouping fits LDS
// at this length); kMaxScanL and shorter sequences run in one launch.
constexpr int kScanPiece = 2048;

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

// last_pos[b, x[b, t]] = the largest t in [T0, T0 + Lp) (ids outside [0, V) are skipped).
__global__ void query_piece_last_kernel(const int64_t* __restrict__ x, int64_t sb, int64_t sl, int T0,
                                        int Lp, int64_t V, int32_t* __restrict__ last_pos) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= Lp) return;
    const int64_t u = x[(int64_t)b * sb + (int64_t)(T0 + i) * sl];
    if (u >= 0 && u < V) atomicMax(&last_pos[(int64_t)b * V + u], T0 + i);
}

// One launch of the query scan over steps [T0, T0 + L) of sequences of Ltot steps (PIECE
// when last_pos is given).
static int query_scan_launch(const int64_t* x, int64_t x_stride_b, int64_t x_stride_l, int B, int L,
                             const float* rhos, int N, int64_t vocab_size, const float* c_init,
                             const int64_t* c_init_keys, int K, const int64_t* doc_ids, float* C_seq,
                             float* state_out, int32_t* stamp_out, int T0, int Ltot,
                             const int32_t* last_pos, hipStream_t st) {
    const bool piece = last_pos != nullptr;
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
    // segment length S: a power of two >= 16 that gives each lane group of pass B at most
    // one sorted range of S elements
    const int groups = kScanThreads / (slice_w / (vec4 ? 4 : 1));
    int lgS = 4;
    while (((L - 1) >> lgS) + 1 > groups) ++lgS;
    const int ncut = (L - 1) >> lgS;
    const int nH = (L - 1) / 64 + 1;
    // Grouping by hash when the token keys are 32-bit and its tables fit beside the index
    // (2^lgTS >= 2L slots); otherwise by the radix sort.
    const int lgTS = pb + 1;
    const ScanLds lay_hash(L, 1 << pb, 4, kScanThreads, ncut, nH, ceil_log2(slice_w), lgTS, piece);
    const bool hash = !wide && pb >= 1 && L <= 64 * 64 && lay_hash.total <= kMaxLds;
    const ScanLds lay = hash ? lay_hash
                             : ScanLds(L, 1 << pb, wide ? 8 : 4, kScanThreads, ncut, nH, ceil_log2(slice_w), 0, piece);
    if (lay.total > kMaxLds)
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_query_scan: L=%d with vocab %lld needs %zu B of LDS",
                    L, (long long)vocab_size, lay.total);
    dim3 grid(B, ns);
#define MB_LAUNCH_SCAN_P(KT, V_, DOCS, HASH, PIECE)                                             \
    do {                                                                                       \
        auto kfn = L <= 64 * kScanRoundsSmall * (kScanThreads / 64)                            \
                       ? ema_query_scan_kernel<KT, V_, DOCS, kScanRoundsSmall, HASH, PIECE>    \
                       : ema_query_scan_kernel<KT, V_, DOCS, kScanRoundsLarge, HASH, PIECE>;   \
        int rc = set_lds(kfn, lay.total);                                                      \
        if (rc) return rc;                                                                     \
        hipLaunchKernelGGL(kfn, grid, dim3(kScanThreads), lay.total, st, x, x_stride_b,        \
                           x_stride_l, L, rhos, N, c_init, c_init_keys, K, doc_ids, C_seq,     \
                           state_out, stamp_out, pb, tok_bits, slice_w, lgS, ncut, lgTS, T0,    \
                           Ltot, last_pos, vocab_size);                                        \
    } while (0)
#define MB_LAUNCH_SCAN_H(KT, V_, DOCS, HASH)                                                    \
    do {                                                                                       \
        if (piece) MB_LAUNCH_SCAN_P(KT, V_, DOCS, HASH, true);                                  \
        else MB_LAUNCH_SCAN_P(KT, V_, DOCS, HASH, false);                                       \
    } while (0)
#define MB_LAUNCH_SCAN(KT, V_, DOCS)                                                            \
    do {                                                                                       \
        if (hash) MB_LAUNCH_SCAN_H(KT, V_, DOCS, true);                                        \
        else MB_LAUNCH_SCAN_H(KT, V_, DOCS, false);                                            \
    } while (0)
#define MB_LAUNCH_SCAN_D(KT, V_)                                    \
    do {                                                            \
        if (doc_ids) MB_LAUNCH_SCAN(KT, V_, true);                  \
        else MB_LAUNCH_SCAN(KT, V_, false);                         \
    } while (0)
    if (wide) {  // (never hashed)
#define MB_LAUNCH_SCAN_W(V_, DOCS) MB_LAUNCH_SCAN_H(uint64_t, V_, DOCS, false)
        if (vec4) {
            if (doc_ids) MB_LAUNCH_SCAN_W(4, true); else MB_LAUNCH_SCAN_W(4, false);
        } else {
            if (doc_ids) MB_LAUNCH_SCAN_W(1, true); else MB_LAUNCH_SCAN_W(1, false);
        }
#undef MB_LAUNCH_SCAN_W
    } else {
        if (vec4) MB_LAUNCH_SCAN_D(uint32_t, 4); else MB_LAUNCH_SCAN_D(uint32_t, 1);
    }
#undef MB_LAUNCH_SCAN_D
#undef MB_LAUNCH_SCAN
#undef MB_LAUNCH_SCAN_H
#undef MB_LAUNCH_SCAN_P
    return check_launch("mb_ema_query_scan");
}

}  // namespace mb

extern "C" int64_t mb_ema_query_scan_workspace(int B, int L, int64_t vocab_size) {
    if (B < 0 || L < 0) {
        fail(MB_ERR_INVALID_ARGUMENT, "mb_ema_query_scan_workspace: negative B=%d or L=%d", B, L);
        return -1;
    }
    if (L <= kMaxScanL || B == 0) return 0;
    if (vocab_size < 1) {
        fail(MB_ERR_UNSUPPORTED, "mb_ema_query_scan_workspace: L=%d > %d needs vocab_size >= 1", L, kMaxScanL);
        return -1;
    }
    return (int64_t)B * vocab_size * 4;
}

extern "C" int mb_ema_query_scan_ws(const int64_t* x, int64_t x_stride_b, int64_t x_stride_l, int B, int L,
                                    const float* rhos, int N, int64_t vocab_size, const float* c_init,
                                    const int64_t* c_init_keys, int K, const int64_t* doc_ids, float* C_seq,
                                    float* state_out, int32_t* stamp_out, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
    MB_REQUIRE(B >= 0 && L >= 0, "mb_ema_query_scan: negative B=%d or L=%d", B, L);
    MB_REQUIRE(N >= 1, "mb_ema_query_scan: N=%d must be >= 1", N);
    if (!c_init || !c_init_keys) K = 0;
    MB_REQUIRE(K >= 0, "mb_ema_query_scan: negative K=%d", K);
    if (B == 0 || L == 0) return MB_OK;
    MB_REQUIRE(x && rhos && C_seq, "mb_ema_query_scan: x, rhos and C_seq must be non-null");
    if ((int64_t)std::min(L, kMaxScanL) * N >= (1ll << 31) || (int64_t)K * N >= (1ll << 31) || K >= (1 << 24))
        return fail(MB_ERR_UNSUPPORTED, "mb_ema_query_scan: L=%d, K=%d, N=%d: rows of one scan must "
                    "stay below 2^31 elements (and K below 2^24)", L, K, N);
    hipStream_t st = (hipStream_t)stream;
    if (L <= kMaxScanL)
        return query_scan_launch(x, x_stride_b, x_stride_l, B, L, rhos, N, vocab_size, c_init, c_init_keys, K,
                                 doc_ids, C_seq, state_out, stamp_out, 0, L, nullptr, st);
    // Longer sequences: pieces of kScanPiece steps, one launch each, the last positions of
    // every token so far in the workspace ([B, vocab_size] int32) between them.
    const int64_t need = mb_ema_query_scan_workspace(B, L, vocab_size);
    if (need < 0) return MB_ERR_UNSUPPORTED;
    if (!workspace || workspace_bytes < need)
        return fail(MB_ERR_WORKSPACE, "mb_ema_query_scan: L=%d > %d runs in pieces and needs %lld B of "
                    "workspace (mb_ema_query_scan_workspace), got %lld", L, kMaxScanL, (long long)need,
                    (long long)(workspace ? workspace_bytes : 0));
    MB_REQUIRE(((uintptr_t)workspace & 3) == 0, "mb_ema_query_scan: workspace must be 4-byte aligned");
    MB_REQUIRE((int64_t)L + kScanPiece < (1ll << 31), "mb_ema_query_scan: L=%d too long", L);
    int32_t* last_pos = static_cast<int32_t*>(workspace);
    const int64_t n = (int64_t)B * vocab_size;
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)), dim3(256), 0, st,
                       last_pos, n, (int32_t)-1);
    int rc = check_launch("mb_ema_query_scan (workspace fill)");
    if (rc) return rc;
    for (int T0 = 0; T0 < L; T0 += kScanPiece) {
        const int Lp = std::min(kScanPiece, L - T0);
        rc = query_scan_launch(x, x_stride_b, x_stride_l, B, Lp, rhos, N, vocab_size, c_init, c_init_keys, K,
                               doc_ids, C_seq, state_out, stamp_out, T0, L, last_pos, st);
        if (rc) return rc;
        if (T0 + Lp < L) {
            hipLaunchKernelGGL(query_piece_last_kernel, dim3((Lp + 255) / 256, B), dim3(256), 0, st, x,
                               x_stride_b, x_stride_l, T0, Lp, vocab_size, last_pos);
            rc = check_launch("mb_ema_query_scan (last positions)");
            if (rc) return rc;
        }
    }
    return MB_OK;
}

extern "C" int mb_ema_query_scan(const int64_t* x, int64_t x_stride_b, int64_t x_stride_l, int B,
                                 int L, const float* rhos, int N, int64_t vocab_size,
                                 const float* c_init, const int64_t* c_init_keys, int K,
                                 const int64_t* doc_ids, float* C_seq, float* state_out,
                                 int32_t* stamp_out, void* stream) {
    return mb_ema_query_scan_ws(x, x_stride_b, x_stride_l, B, L, rhos, N, vocab_size, c_init, c_init_keys, K,
                                doc_ids, C_seq, state_out, stamp_out, nullptr, 0, stream);
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
    MB_REQUIRE((int64_t)L + 128 < (1ll << 31), "mb_ema_boundary_states: L=%d too long", L);
    const int nc = L > 0 ? (L + Br - 1) / Br : 1;  // an empty sequence still stores c0 once
    const int WL = std::min(L, kBoundWin);
    const size_t lds = (size_t)WL * 8 + (size_t)((WL >> 6) + 2) * 8;
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
