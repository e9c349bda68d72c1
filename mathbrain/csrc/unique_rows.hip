// Per-row distinct ids on gfx950: the slot list of a chunk without loader metadata.
//
// Replaces the body of _build_unique_index (mathbrain/triton_flash_ema.py:475-507), which
// sorts each row with torch.sort, marks first occurrences and compacts them with an
// argsort.  Here one workgroup of 1024 threads owns a row: it loads the row's L ids into
// LDS as offsets from the row minimum (so only the bits the row's range needs are
// sorted), sorts them with the block radix sort, marks each key that differs from its
// predecessor, and writes the marked keys in order through one block scan, then -1 up to
// the output width.  The row's distinct count goes to counts[b].  The offsets are held as
// 32-bit keys when the row's range fits (token ids always do), which lets a row of 16384
// ids and its sort buffer fit in LDS; rows with a wider range take 64-bit keys, up to 8192.
#include "common.h"

namespace mb {
namespace {

constexpr int kUThreads = 1024;
constexpr int kUMaxL = 16384;   // 32-bit keys: 16 per thread
constexpr int kUMaxL64 = 8192;  // 64-bit keys: 8 per thread

__device__ inline uint64_t wave_min_u64(uint64_t v) {
    for (int d = 32; d >= 1; d >>= 1) {
        const uint64_t o = __shfl_xor(v, d, 64);
        v = o < v ? o : v;
    }
    return v;
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
    for (int d = 32; d >= 1; d >>= 1) {
        const uint64_t o = __shfl_xor(v, d, 64);
        v = o > v ? o : v;
    }
    return v;
}

// The row's minimum and maximum as order-preserving unsigned keys (the sign bit flipped).
__device__ inline void row_min_max(const int64_t* __restrict__ x, int64_t sb, int64_t sl, int L, int row,
                                   uint64_t& mn, uint64_t& mx) {
    __shared__ uint64_t red[2][16];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    constexpr uint64_t kFlip = 1ull << 63;
    mn = ~0ull;
    mx = 0ull;
    for (int i = tid; i < L; i += kUThreads) {
        const uint64_t k = (uint64_t)x[(int64_t)row * sb + (int64_t)i * sl] ^ kFlip;
        mn = k < mn ? k : mn;
        mx = k > mx ? k : mx;
    }
    mn = wave_min_u64(mn);
    mx = wave_max_u64(mx);
    if (lane == 0) {
        red[0][wave] = mn;
        red[1][wave] = mx;
    }
    __syncthreads();
    mn = ~0ull;
    mx = 0ull;
    for (int w = 0; w < kUThreads / 64; ++w) {
        mn = red[0][w] < mn ? red[0][w] : mn;
        mx = red[1][w] > mx ? red[1][w] : mx;
    }
}

// Keys are compared as unsigned after flipping the sign bit, which orders int64 values; a
// row is sorted as offsets from its minimum in KeyT (uint32_t when its range fits 32 bits;
// otherwise the host launches the uint64_t instantiation, L <= 8192).
template <typename KeyT, int MAXR>
__global__ void __launch_bounds__(kUThreads)
unique_rows_kernel(const int64_t* __restrict__ x, int64_t sb, int64_t sl, int L,
                   int64_t* __restrict__ out, int width, int32_t* __restrict__ counts) {
    extern __shared__ __align__(16) unsigned char smem[];
    KeyT* a = reinterpret_cast<KeyT*>(smem);
    KeyT* b = a + L;
    int* cnt = reinterpret_cast<int*>(smem + (((size_t)2 * L * sizeof(KeyT) + 15) & ~(size_t)15));
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    constexpr uint64_t kFlip = 1ull << 63;

    uint64_t mn, mx;
    row_min_max(x, sb, sl, L, row, mn, mx);
    const uint64_t range = L > 0 ? mx - mn : 0;
    if (sizeof(KeyT) < 8 && (range >> 32) != 0) {
        // (the host picks 64-bit keys for such rows; a row of another call's shape that
        // reaches here writes an empty list rather than wrong ids)
        for (int j = tid; j < width; j += kUThreads) out[(int64_t)row * width + j] = -1;
        if (tid == 0) counts[row] = -1;
        return;
    }
    int nbits = 8;
    while (nbits < 8 * (int)sizeof(KeyT) && (range >> nbits) != 0) nbits += 8;
    for (int i = tid; i < L; i += kUThreads)
        a[i] = (KeyT)(((uint64_t)x[(int64_t)row * sb + (int64_t)i * sl] ^ kFlip) - mn);
    __syncthreads();

    const KeyT* s = block_radix_sort<MAXR>(a, b, cnt, L, 0, nbits);

    // Each thread owns MAXR consecutive sorted keys: count its first occurrences, scan.
    const int i0 = tid * MAXR;
    int mine = 0;
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
        const int i = i0 + r;
        if (i < L && (i == 0 || s[i] != s[i - 1])) ++mine;
    }
    int total;
    int pos = block_exclusive_scan(mine, cnt + 4 * kUThreads, total);
    int64_t* orow = out + (int64_t)row * width;
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
        const int i = i0 + r;
        if (i < L && (i == 0 || s[i] != s[i - 1])) {
            if (pos < width) orow[pos] = (int64_t)(((uint64_t)s[i] + mn) ^ kFlip);
            ++pos;
        }
    }
    for (int j = total + tid; j < width; j += kUThreads) orow[j] = -1;
    if (tid == 0) counts[row] = total;
}

}  // namespace
}  // namespace mb

using namespace mb;

extern "C" int mb_unique_rows(const int64_t* x, int64_t x_stride_b, int64_t x_stride_l, int B,
                              int L, int64_t* out, int width, int32_t* counts, void* stream) {
    MB_REQUIRE(B >= 0 && L >= 0 && width >= 0, "mb_unique_rows: negative B=%d, L=%d or width=%d",
               B, L, width);
    if (L > kUMaxL)
        return fail(MB_ERR_UNSUPPORTED, "mb_unique_rows: L=%d > %d (the row is sorted in LDS)", L,
                    kUMaxL);
    if (B == 0) return MB_OK;
    MB_REQUIRE(out && counts && (L == 0 || x), "mb_unique_rows: null pointer");
    hipStream_t st = (hipStream_t)stream;
    // Rows up to 8192 ids take 64-bit keys, whatever their range.  Longer rows take 32-bit
    // keys: a row whose ids span 2^32 or more then gets counts[b] = -1 and an all -1 list
    // (token ids always fit).
    const bool wide = L <= kUMaxL64;
    auto launch = [&](auto kern, size_t key_bytes) -> int {
        const size_t lds = ((2 * (size_t)(L > 0 ? L : 1) * key_bytes + 15) & ~(size_t)15) +
                           (size_t)(4 * kUThreads + 48) * sizeof(int);
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail((int)e, "mb_unique_rows: LDS attribute: %s", hipGetErrorString(e));
        }
        hipLaunchKernelGGL(kern, dim3(B), dim3(kUThreads), lds, st, x, x_stride_b, x_stride_l, L, out,
                           width, counts);
        return MB_OK;
    };
    const int rc = wide ? launch(unique_rows_kernel<uint64_t, kUMaxL64 / kUThreads>, 8)
                        : launch(unique_rows_kernel<uint32_t, kUMaxL / kUThreads>, 4);
    if (rc) return rc;
    return check_launch("mb_unique_rows");
}
