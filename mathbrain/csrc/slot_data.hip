// Device-side producers of the hot path's inputs: the corpus EMA states that
// preprocess_corpus writes (mathbrain/data.py:276-303) and the collated batch that
// WikiTextMMapDataset.__getitem__ + dynamic_collate_fn build on the host
// (data.py:93-148, 207-232).  The corpus (tokens, document ids, the next-occurrence
// index and the [T, N] states) stays resident in HBM; a batch is three small launches.
#include <climits>
#include <mutex>

#include "common.h"

namespace mb {
namespace {

// ---- corpus states ------------------------------------------------------------------------
//
// The positions, sorted by (document segment, token) with ascending positions inside a
// key, form one chain per key.  Along the sorted order each occurrence e applies
//     s -> a_e * s + 1,   a_e = rho^(p_e - p_{e-1}) when e-1 has the same key, else 0,
// and states[p_e] is the result.  The sorted order is cut into units of kUnit occurrences:
// pass 1 composes each unit's maps (one wave per unit, lanes over rates), pass 2 scans the
// unit compositions per rate, pass 3 re-walks each unit from its incoming state and writes
// the state rows.  Both walks read the sorted positions and keys contiguously (16 B per
// occurrence); each occurrence costs one exp2 per rate per walk, and every state row is
// written once, 4*N contiguous bytes.

constexpr int kUnit = 1024;
constexpr int kUnitWaves = 4;
constexpr int kScanThreads = 1024;
constexpr int kMaxRates = 128;

// WALK = false: pass 1, writes the composition (A, B) of each unit into agg[2][N][n_units].
// WALK = true: pass 3, starts from s_in[N][n_units] and writes states[p][n].
template <bool WALK, int NV>
__global__ void __launch_bounds__(64 * kUnitWaves)
corpus_unit_kernel(const int64_t* __restrict__ order, const int64_t* __restrict__ chain, int64_t T,
                   const float* __restrict__ rhos, int N, int64_t n_units, float* __restrict__ agg,
                   const float* __restrict__ s_in, float* __restrict__ states) {
    const int lane = threadIdx.x & 63;
    const int64_t u = (int64_t)blockIdx.x * kUnitWaves + (threadIdx.x >> 6);
    if (u >= n_units) return;
    float hi[NV], lo[NV], A[NV], S[NV];
#pragma unroll
    for (int q = 0; q < NV; ++q) {
        const int n = lane + 64 * q;
        hi[q] = lo[q] = 0.0f;
        if (n < N) log2_split(rhos[n], hi[q], lo[q]);
        A[q] = 1.0f;
        S[q] = (WALK && n < N) ? s_in[(int64_t)n * n_units + u] : 0.0f;
    }
    const int64_t e0 = u * kUnit;
    const int64_t e1 = e0 + kUnit < T ? e0 + kUnit : T;
    // occurrence e0 - 1, the predecessor of the unit's first one
    int pp = -1;
    int64_t kp = 0;
    if (e0 > 0) {
        const int64_t q = order[e0 - 1];
        pp = (q >= 0 && q < T) ? (int)q : -1;
        kp = chain[e0 - 1];
    }
    for (int64_t b0 = e0; b0 < e1; b0 += 64) {
        const int64_t e = b0 + lane;
        int p = -1;
        int64_t key = 0;
        if (e < e1) {
            const int64_t q = order[e];
            p = (q >= 0 && q < T) ? (int)q : -1;
            key = chain[e];
        }
        int p_prev = __shfl_up(p, 1, 64);
        int64_t k_prev = __shfl_up(key, 1, 64);
        if (lane == 0) {
            p_prev = pp;
            k_prev = kp;
        }
        const bool link = p >= 0 && p_prev >= 0 && key == k_prev && p > p_prev;
        const int step = link ? p - p_prev : -1;
        const int cnt = (int)(e1 - b0 < 64 ? e1 - b0 : 64);
        pp = __shfl(p, cnt - 1, 64);
        kp = __shfl(key, cnt - 1, 64);
        for (int j = 0; j < cnt; ++j) {
            const int d = __builtin_amdgcn_readlane(step, j);
            const int pj = __builtin_amdgcn_readlane(p, j);
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                const float a = d < 0 ? 0.0f : pow_steps(hi[q], lo[q], d);
                if (!WALK) A[q] *= a;
                S[q] = __builtin_fmaf(a, S[q], 1.0f);
                const int n = lane + 64 * q;
                if (WALK && pj >= 0 && n < N) st_stream(states + (int64_t)pj * N + n, S[q]);
            }
        }
    }
    if (!WALK) {
#pragma unroll
        for (int q = 0; q < NV; ++q) {
            const int n = lane + 64 * q;
            if (n < N) {
                agg[(int64_t)n * n_units + u] = A[q];
                agg[((int64_t)N + n) * n_units + u] = S[q];
            }
        }
    }
}

// Pass 2: one block per rate; exclusive scan of the unit compositions, applied to the
// zero state before the first occurrence, giving each unit's incoming state.
__global__ void __launch_bounds__(kScanThreads)
corpus_scan_kernel(const float* __restrict__ agg, int64_t n_units, int N, float* __restrict__ s_in) {
    __shared__ float wa[kScanThreads / 64], wb[kScanThreads / 64];
    const int n = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* Ag = agg + (int64_t)n * n_units;
    const float* Bg = agg + ((int64_t)N + n) * n_units;
    const int64_t per = (n_units + kScanThreads - 1) / kScanThreads;
    const int64_t u0 = tid * per;
    const int64_t u1 = u0 + per < n_units ? u0 + per : n_units;
    float A = 1.0f, Bc = 0.0f;  // this thread's composition: s -> A*s + Bc
    for (int64_t u = u0; u < u1; ++u) {
        const float a = Ag[u];
        A *= a;
        Bc = __builtin_fmaf(a, Bc, Bg[u]);
    }
    // inclusive scan over the wave: (A, B) after (A', B') = (A*A', A*B' + B)
    float iA = A, iB = Bc;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const float oA = __shfl_up(iA, d, 64), oB = __shfl_up(iB, d, 64);
        if (lane >= d) {
            iB = __builtin_fmaf(iA, oB, iB);
            iA *= oA;
        }
    }
    if (lane == 63) {
        wa[w] = iA;
        wb[w] = iB;
    }
    __syncthreads();
    // state after all earlier waves, starting from 0
    float s = 0.0f;
    for (int k = 0; k < w; ++k) s = __builtin_fmaf(wa[k], s, wb[k]);
    // state after the earlier lanes of this wave: exclusive = inclusive of lane - 1
    const float eA = __shfl_up(iA, 1, 64), eB = __shfl_up(iB, 1, 64);
    if (lane > 0) s = __builtin_fmaf(eA, s, eB);
    for (int64_t u = u0; u < u1; ++u) {
        s_in[(int64_t)n * n_units + u] = s;
        s = __builtin_fmaf(Ag[u], s, Bg[u]);
    }
}

// ---- batch builder -----------------------------------------------------------------------

constexpr int kMarkBlocks = 16;
constexpr int kMarkThreads = 256;
constexpr int kCompactThreads = 1024;
constexpr int kCompactPer = 4;
constexpr int kRowsPerWave = 8;

__device__ inline bool row_ok(int64_t d0, int64_t s0, int64_t e0, int64_t T) {
    return d0 >= 0 && d0 <= s0 && s0 < e0 && e0 <= T;
}

__global__ void slot_clear_kernel(int32_t* __restrict__ last, int32_t* __restrict__ slot_of, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        last[i] = -1;
        slot_of[i] = 0;
    }
}

// Row b: every position p of tokens[doc_start:start) whose token does not occur again
// before start records itself as that token's last history occurrence; every token of
// tokens[start:end) is flagged as a chunk token (slot_of = 1).
__global__ void __launch_bounds__(kMarkThreads)
slot_mark_kernel(const int32_t* __restrict__ tokens, const int32_t* __restrict__ next_pos, int64_t T,
                 int64_t V, const int64_t* __restrict__ doc_start, const int64_t* __restrict__ start,
                 const int64_t* __restrict__ end, int32_t* __restrict__ last,
                 int32_t* __restrict__ slot_of) {
    const int b = blockIdx.y;
    const int64_t d0 = doc_start[b], s0 = start[b], e0 = end[b];
    if (!row_ok(d0, s0, e0, T)) return;
    int32_t* lb = last + (int64_t)b * V;
    int32_t* fb = slot_of + (int64_t)b * V;
    for (int64_t p = d0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < e0;
         p += (int64_t)gridDim.x * blockDim.x) {
        const int v = tokens[p];
        if (v < 0 || v >= V) continue;
        if (p < s0) {
            if ((int64_t)next_pos[p] >= s0) lb[v] = (int32_t)p;
        } else {
            fb[v] = 1;
        }
    }
}

// One block per row: chunk tokens get slots 0.. in id order, history-only tokens the
// slots after them, in id order.
__global__ void __launch_bounds__(kCompactThreads)
slot_compact_kernel(int64_t V, const int64_t* __restrict__ doc_start, const int64_t* __restrict__ start,
                    const int64_t* __restrict__ end, int64_t T, const int32_t* __restrict__ last,
                    int32_t* __restrict__ slot_of, int64_t* __restrict__ slot_tok,
                    int32_t* __restrict__ counts) {
    __shared__ int scratch[64];
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int32_t* lb = last + (int64_t)b * V;
    int32_t* fb = slot_of + (int64_t)b * V;
    int64_t* tb = slot_tok + (int64_t)b * V;
    const bool ok = row_ok(doc_start[b], start[b], end[b], T);
    int c = 0;
    if (ok)
        for (int64_t v = tid; v < V; v += kCompactThreads) c += fb[v] == 1;
    int n_chunk;
    block_exclusive_scan(c, scratch, n_chunk);
    int base_c = 0, base_h = 0;
    constexpr int kTile = kCompactThreads * kCompactPer;
    for (int64_t v0 = 0; v0 < V; v0 += kTile) {
        int f[kCompactPer];
        int sum = 0;
#pragma unroll
        for (int i = 0; i < kCompactPer; ++i) {
            const int64_t v = v0 + (int64_t)tid * kCompactPer + i;
            f[i] = 0;
            if (ok && v < V) {
                const int ic = fb[v] == 1;
                f[i] = ic | ((!ic && lb[v] >= 0) << 16);
            }
            sum += f[i];
        }
        int tot;
        int ex = block_exclusive_scan(sum, scratch, tot);
#pragma unroll
        for (int i = 0; i < kCompactPer; ++i) {
            const int64_t v = v0 + (int64_t)tid * kCompactPer + i;
            if (v < V) {
                int slot = -1;
                if (f[i] & 1) slot = base_c + (ex & 0xFFFF);
                else if (f[i] >> 16) slot = n_chunk + base_h + (ex >> 16);
                fb[v] = slot;
                if (slot >= 0) tb[slot] = v;
            }
            ex += f[i];
        }
        base_c += tot & 0xFFFF;
        base_h += tot >> 16;
    }
    if (tid == 0) {
        counts[2 * b] = n_chunk;
        counts[2 * b + 1] = n_chunk + base_h;
    }
}

// c_base, slot list and pad mask: each wave fills kRowsPerWave consecutive (b, k) rows.
// Lanes 0..kRowsPerWave-1 first look up their row's slot token and last occurrence, so the
// state rows of all kRowsPerWave rows are fetched together.
__global__ void __launch_bounds__(256)
slot_fill_kernel(const float* __restrict__ states, const float* __restrict__ rhos, int N, int64_t T,
                 int64_t V, const int64_t* __restrict__ start, const int32_t* __restrict__ last,
                 const int64_t* __restrict__ slot_tok, const int32_t* __restrict__ counts, int B,
                 int K_max, int64_t* __restrict__ unique_slots, uint8_t* __restrict__ pad_mask,
                 float* __restrict__ c_base) {
    const int lane = threadIdx.x & 63;
    const int64_t rows = (int64_t)B * K_max;
    const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kRowsPerWave;
    if (r0 >= rows) return;
    float hi[kMaxRates / 64], lo[kMaxRates / 64];
#pragma unroll
    for (int q = 0; q < kMaxRates / 64; ++q) {
        const int n = lane + 64 * q;
        hi[q] = lo[q] = 0.0f;
        if (n < N) log2_split(rhos[n], hi[q], lo[q]);
    }
    // lane j < kRowsPerWave: row r0 + j's token, source position and decay steps
    int my_p = -1, my_steps = 0, my_valid = 0;
    int64_t my_v = 0;
    {
        const int64_t r = r0 + lane;
        if (lane < kRowsPerWave && r < rows) {
            const int b = (int)(r / K_max), k = (int)(r % K_max);
            if (k < counts[2 * b + 1]) {
                my_valid = 1;
                const int64_t v = slot_tok[(int64_t)b * V + k];
                my_v = v;
                if (v >= 0 && v < V) {
                    const int p = last[(int64_t)b * V + v];
                    const int64_t s0 = start[b];
                    if (p >= 0 && p < T && p < s0) {
                        my_p = p;
                        my_steps = (int)(s0 - p);
                    }
                }
            }
            unique_slots[r] = my_valid ? my_v : 0;
            pad_mask[r] = (uint8_t)my_valid;
        }
    }
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) {
        const int64_t r = r0 + j;
        if (r >= rows) break;
        const int p = __builtin_amdgcn_readlane(my_p, j);
        const int steps = __builtin_amdgcn_readlane(my_steps, j);
        float* dst = c_base + r * N;
#pragma unroll
        for (int q = 0; q < kMaxRates / 64; ++q) {
            const int n = lane + 64 * q;
            if (n < N)
                dst[n] = p >= 0 ? states[(int64_t)p * N + n] * pow_steps(hi[q], lo[q], steps) : 0.0f;
        }
    }
}

// Chunk rows: tokens, document ids and the slot of every chunk position.
__global__ void __launch_bounds__(256)
slot_chunk_kernel(const int32_t* __restrict__ tokens, const int32_t* __restrict__ doc_ids, int64_t T,
                  int64_t V, const int64_t* __restrict__ doc_start, const int64_t* __restrict__ start,
                  const int64_t* __restrict__ end, const int32_t* __restrict__ slot_of, int B, int L,
                  int64_t* __restrict__ chunks, int64_t* __restrict__ doc_out,
                  int64_t* __restrict__ inverse) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * L) return;
    const int b = (int)(i / L), t = (int)(i % L);
    const int64_t d0 = doc_start[b], s0 = start[b], e0 = end[b];
    int64_t tok = 0, doc = -1, inv = 0;
    if (row_ok(d0, s0, e0, T) && s0 + t < e0) {
        const int v = tokens[s0 + t];
        tok = v;
        doc = doc_ids[s0 + t];
        if (v >= 0 && v < V) {
            const int sl = slot_of[(int64_t)b * V + v];
            inv = sl >= 0 ? sl : 0;
        }
    }
    chunks[i] = tok;
    doc_out[i] = doc;
    inverse[i] = inv;
}

int64_t units_for(int64_t T) { return (T + kUnit - 1) / kUnit; }

}  // namespace
}  // namespace mb

using namespace mb;

// Device scratch of mb_corpus_states_noalloc.  Each GPU the library runs on holds its own
// copy from module load until the process ends; host code reaches it only through the
// address hipGetSymbolAddress returns on that device (the array's name in host code is a
// stand-in, not a device address).
constexpr int64_t kNoAllocScratchBytes = 32ll << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace mb {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];
// Per device, the event recorded after the last call's final pass: the next call's stream
// waits for it, so that calls on different streams take the scratch array one after the
// other instead of overwriting each other's aggregates.
hipEvent_t g_scratch_done[kMaxScratchDevices];

// The current device's address of `scratch`, looked up once per device (with that device
// current) and kept.
int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail((int)e, "mb_corpus_states_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(MB_ERR_UNSUPPORTED, "mb_corpus_states_noalloc: device %d beyond %d", dev, kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail((int)(e != hipSuccess ? e : hipErrorInvalidSymbol),
                        "mb_corpus_states_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        hipEvent_t ev = nullptr;
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess)
            return fail((int)e, "mb_corpus_states_noalloc: hipEventCreateWithFlags: %s", hipGetErrorString(e));
        g_scratch_done[dev] = ev;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MB_OK;
}

// The three passes of mb_corpus_states over a workspace of mb_corpus_states_workspace bytes.
int corpus_states_run(const int64_t* order, const int64_t* chain, int64_t T, const float* rhos,
                      int N, float* states, void* work, hipStream_t st) {
    const int64_t nu = units_for(T);
    float* agg = (float*)work;
    float* s_in = agg + nu * 2 * N;
    const dim3 ugrid((unsigned)((nu + kUnitWaves - 1) / kUnitWaves));
    const dim3 ublock(64 * kUnitWaves);
    if (N <= 64) {
        hipLaunchKernelGGL((corpus_unit_kernel<false, 1>), ugrid, ublock, 0, st, order, chain, T,
                           rhos, N, nu, agg, nullptr, nullptr);
    } else {
        hipLaunchKernelGGL((corpus_unit_kernel<false, 2>), ugrid, ublock, 0, st, order, chain, T,
                           rhos, N, nu, agg, nullptr, nullptr);
    }
    int rc = check_launch("mb_corpus_states (unit compositions)");
    if (rc) return rc;
    hipLaunchKernelGGL(corpus_scan_kernel, dim3(N), dim3(kScanThreads), 0, st, agg, nu, N, s_in);
    if ((rc = check_launch("mb_corpus_states (unit scan)"))) return rc;
    if (N <= 64) {
        hipLaunchKernelGGL((corpus_unit_kernel<true, 1>), ugrid, ublock, 0, st, order, chain, T,
                           rhos, N, nu, nullptr, s_in, states);
    } else {
        hipLaunchKernelGGL((corpus_unit_kernel<true, 2>), ugrid, ublock, 0, st, order, chain, T,
                           rhos, N, nu, nullptr, s_in, states);
    }
    return check_launch("mb_corpus_states (state rows)");
}

}  // namespace
}  // namespace mb

extern "C" int64_t mb_corpus_states_workspace(int64_t T, int N) {
    if (T <= 0 || N <= 0) return 0;
    return units_for(T) * (int64_t)N * 3 * (int64_t)sizeof(float);
}

extern "C" int mb_corpus_states(const int64_t* order, const int64_t* chain, int64_t T,
                                const float* rhos, int N, float* states, void* work,
                                int64_t work_bytes, void* stream) {
    MB_REQUIRE(T >= 0, "mb_corpus_states: negative T=%lld", (long long)T);
    MB_REQUIRE(N >= 1 && N <= kMaxRates, "mb_corpus_states: N=%d must be in [1, %d]", N, kMaxRates);
    MB_REQUIRE(T <= INT_MAX, "mb_corpus_states: T=%lld exceeds the int32 position range",
               (long long)T);
    if (T == 0) return MB_OK;
    MB_REQUIRE(order && chain && rhos && states,
               "mb_corpus_states: order, chain, rhos and states must be non-null");
    const int64_t need = mb_corpus_states_workspace(T, N);
    if (!work || work_bytes < need)
        return fail(MB_ERR_WORKSPACE, "mb_corpus_states: workspace of %lld B given, %lld B needed",
                    (long long)work_bytes, (long long)need);
    return corpus_states_run(order, chain, T, rhos, N, states, work, (hipStream_t)stream);
}

extern "C" int mb_corpus_states_noalloc(const int64_t* order, const int64_t* chain, int64_t T,
                                        const float* rhos, int N, float* states, void* stream) {
    MB_REQUIRE(T >= 0, "mb_corpus_states_noalloc: negative T=%lld", (long long)T);
    MB_REQUIRE(N >= 1 && N <= kMaxRates, "mb_corpus_states_noalloc: N=%d must be in [1, %d]", N,
               kMaxRates);
    MB_REQUIRE(T <= INT_MAX, "mb_corpus_states_noalloc: T=%lld exceeds the int32 position range",
               (long long)T);
    const int64_t need = mb_corpus_states_workspace(T, N);
    if (need > kNoAllocScratchBytes)
        return fail(MB_ERR_WORKSPACE,
                    "mb_corpus_states_noalloc: T=%lld at N=%d needs %lld B of scratch, more than the "
                    "%lld B this entry point holds per GPU (use mb_corpus_states with a workspace)",
                    (long long)T, N, (long long)need, (long long)kNoAllocScratchBytes);
    if (T == 0) return MB_OK;
    MB_REQUIRE(order && chain && rhos && states,
               "mb_corpus_states_noalloc: order, chain, rhos and states must be non-null");
    void* work = nullptr;
    int rc = scratch_address(&work);
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail((int)e, "mb_corpus_states_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    // Calls on one device run their passes one call after the other, in the order the host
    // makes them: each waits for the previous call's event and records its own.  (Under
    // graph capture the graph's own order applies and replays that overlap race.)
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess) {
        (void)hipGetLastError();
        cap = hipStreamCaptureStatusNone;
    }
    const bool serial = cap == hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (serial && (e = hipStreamWaitEvent(st, g_scratch_done[dev], 0)) != hipSuccess)
        return fail((int)e, "mb_corpus_states_noalloc: hipStreamWaitEvent: %s", hipGetErrorString(e));
    rc = corpus_states_run(order, chain, T, rhos, N, states, work, st);
    if (rc) return rc;
    if (serial && (e = hipEventRecord(g_scratch_done[dev], st)) != hipSuccess)
        return fail((int)e, "mb_corpus_states_noalloc: hipEventRecord: %s", hipGetErrorString(e));
    return MB_OK;
}

extern "C" int mb_slot_lists(const int32_t* tokens, const int32_t* next_pos, int64_t T, int64_t V,
                             const int64_t* doc_start, const int64_t* start, const int64_t* end, int B,
                             int32_t* last, int32_t* slot_of, int64_t* slot_tok, int32_t* counts,
                             void* stream) {
    MB_REQUIRE(B >= 0 && T >= 0 && V >= 1, "mb_slot_lists: bad sizes B=%d T=%lld V=%lld", B,
               (long long)T, (long long)V);
    MB_REQUIRE(T <= INT_MAX && V <= INT_MAX, "mb_slot_lists: T=%lld or V=%lld exceeds int32",
               (long long)T, (long long)V);
    if (B == 0) return MB_OK;
    MB_REQUIRE(tokens && next_pos && doc_start && start && end && last && slot_of && slot_tok && counts,
               "mb_slot_lists: null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    const int64_t n = (int64_t)B * V;
    const int64_t cb = (n + 255) / 256;
    hipLaunchKernelGGL(slot_clear_kernel, dim3((unsigned)(cb < 4096 ? cb : 4096)), dim3(256), 0, st,
                       last, slot_of, n);
    int rc = check_launch("mb_slot_lists (clear)");
    if (rc) return rc;
    hipLaunchKernelGGL(slot_mark_kernel, dim3(kMarkBlocks, B), dim3(kMarkThreads), 0, st, tokens,
                       next_pos, T, V, doc_start, start, end, last, slot_of);
    if ((rc = check_launch("mb_slot_lists (mark)"))) return rc;
    hipLaunchKernelGGL(slot_compact_kernel, dim3(B), dim3(kCompactThreads), 0, st, V, doc_start,
                       start, end, T, last, slot_of, slot_tok, counts);
    return check_launch("mb_slot_lists (compact)");
}

extern "C" int mb_slot_batch(const int32_t* tokens, const int32_t* doc_ids, const float* states,
                             const float* rhos, int N, int64_t T, int64_t V, const int64_t* doc_start,
                             const int64_t* start, const int64_t* end, int B, const int32_t* last,
                             const int32_t* slot_of, const int64_t* slot_tok, const int32_t* counts,
                             int L, int K_max, int64_t* chunks, int64_t* doc_out, int64_t* unique_slots,
                             uint8_t* pad_mask, int64_t* inverse, float* c_base, void* stream) {
    MB_REQUIRE(B >= 0 && L >= 0 && K_max >= 0 && T >= 0 && V >= 1,
               "mb_slot_batch: bad sizes B=%d L=%d K_max=%d T=%lld V=%lld", B, L, K_max,
               (long long)T, (long long)V);
    MB_REQUIRE(N >= 1 && N <= kMaxRates, "mb_slot_batch: N=%d must be in [1, %d]", N, kMaxRates);
    MB_REQUIRE(T <= INT_MAX && V <= INT_MAX, "mb_slot_batch: T=%lld or V=%lld exceeds int32",
               (long long)T, (long long)V);
    if (B == 0) return MB_OK;
    MB_REQUIRE(tokens && doc_ids && states && rhos && doc_start && start && end && last && slot_of &&
                   slot_tok && counts,
               "mb_slot_batch: null input pointer");
    hipStream_t st = (hipStream_t)stream;
    int rc;
    if (K_max > 0) {
        MB_REQUIRE(unique_slots && pad_mask && c_base, "mb_slot_batch: null slot output pointer");
        const int64_t waves = ((int64_t)B * K_max + kRowsPerWave - 1) / kRowsPerWave;
        hipLaunchKernelGGL(slot_fill_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st,
                           states, rhos, N, T, V, start, last, slot_tok, counts, B, K_max,
                           unique_slots, pad_mask, c_base);
        if ((rc = check_launch("mb_slot_batch (slots)"))) return rc;
    }
    if (L > 0) {
        MB_REQUIRE(chunks && doc_out && inverse, "mb_slot_batch: null chunk output pointer");
        const int64_t n = (int64_t)B * L;
        hipLaunchKernelGGL(slot_chunk_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           tokens, doc_ids, T, V, doc_start, start, end, slot_of, B, L, chunks,
                           doc_out, inverse);
        if ((rc = check_launch("mb_slot_batch (chunks)"))) return rc;
    }
    return MB_OK;
}
