// scan.hpp — device-wide inclusive scan of int32 (or int64) items with int64 running sums
// (replaces CUDA.jl's accumulate!(+) at src/forward_core.jl:231, 259 and
// src/training.jl:384). Reduce-then-scan in two launches (or the second alone when the
// producer of the items sums the tiles, device_scan_apply):
//   1. each 2048-item tile reduces its items                      (k_scan_reduce)
//   2. each tile sums the earlier tiles' sums into its offset and
//      rescans its items; tile 0 also writes the total              (k_scan_apply)
// (A third launch that scanned the tile sums once cost more than every tile summing its
// predecessors: a kernel boundary is ~4 us, the extra loads of a few hundred sums ~1 us.)
// Items come from a functor In(i) and results go to a functor Out(i, inclusive, item), so
// compaction, gathers and scatters fuse into the scan passes instead of separate kernels.
#pragma once

#include "common.hpp"

namespace tdgs {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;

// Block-wide exclusive scan of one int64 per thread; returns the exclusive prefix and
// writes the block total to *total.
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t v, int64_t* total) {
    __shared__ int64_t s_wave[kScanThreads / kWave];
    const int lane = __lane_id();
    const int wave = threadIdx.x / kWave;
    int64_t incl = v;
    for (int d = 1; d < kWave; d <<= 1) {
        const int64_t o = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) s_wave[wave] = incl;
    __syncthreads();
    int64_t wave_off = 0, tot = 0;
    for (int w = 0; w < kScanThreads / kWave; ++w) {
        const int64_t s = s_wave[w];
        if (w < wave) wave_off += s;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return wave_off + incl - v;
}

// d_limit, when not null, is a device count past which every item is zero: tiles that start
// at or after it do no work (their sum is 0 and nothing is written for them).
template <class In>
__global__ __launch_bounds__(kScanThreads) void k_scan_reduce(In in, int64_t n, int64_t* tile_sums,
                                                              const int64_t* d_limit) {
    if (d_limit && (int64_t)blockIdx.x * kScanTile >= *d_limit) {
        if (threadIdx.x == 0) tile_sums[blockIdx.x] = 0;
        return;
    }
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int64_t acc = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + k;
        if (i < n) acc += in(i);
    }
    int64_t total;
    block_exclusive_scan(acc, &total);
    if (threadIdx.x == 0) tile_sums[blockIdx.x] = total;
}

// Tile b's offset is the sum of tile_sums[0, b); tile 0 sums all ntiles and writes the
// total to *total_out (when not null).
template <class In, class Out>
__global__ __launch_bounds__(kScanThreads) void k_scan_apply(In in, Out out, int64_t n, const int64_t* tile_sums,
                                                             int64_t ntiles, int64_t* total_out,
                                                             const int64_t* d_limit) {
    const int64_t b = blockIdx.x;
    const bool past = d_limit && b * kScanTile >= *d_limit;
    if (past && b != 0) return;
    const int64_t upto = b == 0 ? ntiles : b;
    int64_t part = 0;
    for (int64_t k = threadIdx.x; k < upto; k += kScanThreads) part += tile_sums[k];
    int64_t before;
    block_exclusive_scan(part, &before);   // (only the block total is used)
    if (b == 0) {
        if (threadIdx.x == 0 && total_out) *total_out = before;
        before = 0;
    }
    if (past) return;
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    using Item = decltype(in(int64_t(0)));   // int32_t, or int64_t for two packed counts
    Item v[kScanItems];
    int64_t acc = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + k;
        v[k] = i < n ? in(i) : 0;
        acc += v[k];
    }
    int64_t total;
    int64_t run = block_exclusive_scan(acc, &total) + before;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + k;
        run += v[k];
        if (i < n) out(i, run, v[k]);
    }
}

inline size_t scan_temp_bytes_for(int64_t n) {
    return align_up((size_t)(ceil_div(n > 0 ? n : 1, kScanTile)) * sizeof(int64_t));
}

// In1 is used by the reduce pass, In2 by the apply pass (they may differ when the reduce
// pass also materialises the items, e.g. writes keep flags that the apply pass re-reads).
// d_limit (device count, may be null): items at or past it are zero and their results are
// not needed; the tiles past it are skipped.
template <class In1, class In2, class Out>
int device_scan(In1 in_reduce, In2 in_apply, Out out, int64_t n, void* temp, size_t temp_bytes,
                int64_t* d_total, hipStream_t stream, const int64_t* d_limit = nullptr) {
    const int64_t ntiles = ceil_div(n > 0 ? n : 1, kScanTile);
    if (temp_bytes < (size_t)ntiles * sizeof(int64_t) || temp == nullptr) {
        set_error("scan scratch too small: need %zu bytes, have %zu", (size_t)ntiles * 8, temp_bytes);
        return TDGS_ERR_CAPACITY;
    }
    int64_t* tile_sums = (int64_t*)temp;
    k_scan_reduce<<<(unsigned)ntiles, kScanThreads, 0, stream>>>(in_reduce, n, tile_sums, d_limit);
    TDGS_LAUNCHED();
    k_scan_apply<<<(unsigned)ntiles, kScanThreads, 0, stream>>>(in_apply, out, n, tile_sums, ntiles, d_total,
                                                                 d_limit);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

// The apply pass alone, for a producer that has already summed the items of every kScanTile
// tile into tile_sums (ceil(n / kScanTile) entries).
template <class In, class Out>
int device_scan_apply(In in, Out out, int64_t n, const int64_t* tile_sums, int64_t* d_total, hipStream_t stream,
                      const int64_t* d_limit = nullptr) {
    const int64_t ntiles = ceil_div(n > 0 ? n : 1, kScanTile);
    k_scan_apply<<<(unsigned)ntiles, kScanThreads, 0, stream>>>(in, out, n, tile_sums, ntiles, d_total, d_limit);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

// Common item/result functors.
struct ItemsU8 {
    const uint8_t* p;
    __device__ int32_t operator()(int64_t i) const { return p[i] ? 1 : 0; }
};
struct ItemsI32 {
    const int32_t* p;
    __device__ int32_t operator()(int64_t i) const { return p[i]; }
};
struct ItemsU32 {
    const uint32_t* p;
    __device__ int32_t operator()(int64_t i) const { return (int32_t)p[i]; }
};
// The same with items past n read as zero and not written (a scan launched over
// max(n, 1) items, so that an empty input still produces its total).
struct ItemsI32Bounded {
    const int32_t* p;
    int64_t n;
    __device__ int32_t operator()(int64_t i) const { return i < n ? p[i] : 0; }
};
struct WriteInclusiveI32Bounded {
    int32_t* p;
    int64_t n;
    __device__ void operator()(int64_t i, int64_t incl, int32_t) const {
        if (i < n) p[i] = (int32_t)incl;
    }
};
struct WriteInclusiveI32 {
    int32_t* p;
    __device__ void operator()(int64_t i, int64_t incl, int32_t) const { p[i] = (int32_t)incl; }
};
struct WriteExclusiveU32 {
    uint32_t* p;
    __device__ void operator()(int64_t i, int64_t incl, int32_t item) const {
        p[i] = (uint32_t)(incl - item);
    }
};

}  // namespace tdgs
