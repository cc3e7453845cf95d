// sort.hpp — stable LSD radix sort of (key, int32 value) pairs on a key bit range
// [begin_bit, end_bit), 8-bit digits; replaces CUB DeviceRadixSort::SortPairs
// (deps/cub_sort_pairs/cub_sort_pairs_wrapper.cu:31-43).
//
// One pass per digit, three launches per pass:
//   count   each 4096-key tile builds its digit histogram in LDS (wave-aggregated: one LDS
//           atomic per distinct digit per wavefront, found with 8 ballots)
//   scan    exclusive scan of the digit-major count table [256][tiles] -> global offsets
//   scatter each tile re-ranks its keys stably (same ballot match gives the rank inside the
//           wavefront; per-wave digit counts in LDS give the rank across wavefronts) and
//           writes every pair to offset[digit][tile] + rank.
// Stability: within a tile keys are ranked in index order (iteration, wave, lane), across
// tiles by the digit-major scan, so equal digits keep their input order.
#pragma once

#include "common.hpp"
#include "scan.hpp"

namespace tdgs {

constexpr int kRsThreads = 256;
constexpr int kRsItems = 16;
constexpr int kRsTile = kRsThreads * kRsItems;
constexpr int kRsBins = 256;
constexpr int kRsWaves = kRsThreads / kWave;
static_assert(kRsThreads == kRsBins, "one thread per digit bin");

// Lanes of the wavefront holding the same digit as this lane (among lanes with valid).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, int nbits, bool valid) {
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        peers &= bit ? bal : ~bal;
    }
    return peers;
}

template <class K>
__global__ __launch_bounds__(kRsThreads) void k_radix_count(const K* __restrict__ keys, int64_t n,
                                                            int shift, int nbits,
                                                            uint32_t* __restrict__ counts,
                                                            int64_t ntiles) {
    __shared__ uint32_t hist[kRsBins];
    hist[threadIdx.x] = 0;
    __syncthreads();
    const uint32_t mask = (1u << nbits) - 1u;
    const int64_t base = (int64_t)blockIdx.x * kRsTile + threadIdx.x;
    for (int k = 0; k < kRsItems; ++k) {
        const int64_t i = base + (int64_t)k * kRsThreads;
        const bool valid = i < n;
        const uint32_t d = valid ? (uint32_t)(keys[i] >> shift) & mask : 0u;
        const uint64_t peers = match_digit(d, nbits, valid);
        if (valid && (peers & lanemask_lt()) == 0) atomicAdd(&hist[d], (uint32_t)__popcll(peers));
    }
    __syncthreads();
    counts[(int64_t)threadIdx.x * ntiles + blockIdx.x] = hist[threadIdx.x];
}

template <class K>
__global__ __launch_bounds__(kRsThreads) void k_radix_scatter(
    const K* __restrict__ kin, const int32_t* __restrict__ vin, K* __restrict__ kout,
    int32_t* __restrict__ vout, int64_t n, int shift, int nbits,
    const uint32_t* __restrict__ offsets, int64_t ntiles) {
    __shared__ uint32_t running[kRsBins];
    __shared__ uint32_t wcount[kRsWaves][kRsBins];
    const int t = threadIdx.x;
    const int wave = t / kWave;
    running[t] = offsets[(int64_t)t * ntiles + blockIdx.x];
#pragma unroll
    for (int w = 0; w < kRsWaves; ++w) wcount[w][t] = 0;
    __syncthreads();
    const uint32_t mask = (1u << nbits) - 1u;
    const int64_t base = (int64_t)blockIdx.x * kRsTile + t;
    for (int k = 0; k < kRsItems; ++k) {
        const int64_t i = base + (int64_t)k * kRsThreads;
        const bool valid = i < n;
        const K key = valid ? kin[i] : (K)0;
        const int32_t val = valid ? vin[i] : 0;
        const uint32_t d = (uint32_t)(key >> shift) & mask;
        const uint64_t peers = match_digit(d, nbits, valid);
        const uint32_t rank = (uint32_t)__popcll(peers & lanemask_lt());
        if (valid && rank == 0) wcount[wave][d] = (uint32_t)__popcll(peers);
        __syncthreads();
        uint32_t pos = 0;
        if (valid) {
            pos = running[d] + rank;
            for (int w = 0; w < wave; ++w) pos += wcount[w][d];
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int w = 0; w < kRsWaves; ++w) {
            add += wcount[w][t];
            wcount[w][t] = 0;
        }
        running[t] += add;
        __syncthreads();
        if (valid) {
            kout[pos] = key;
            vout[pos] = val;
        }
    }
}

inline int radix_passes(int begin_bit, int end_bit) {
    return end_bit > begin_bit ? (end_bit - begin_bit + 7) / 8 : 0;
}

// Scratch for radix_sort_pairs (count table + its scan), excluding ping-pong buffers.
inline size_t radix_temp_bytes(int64_t n) {
    const int64_t ntiles = ceil_div(n > 0 ? n : 1, kRsTile);
    const int64_t cells = ntiles * kRsBins;
    return align_up((size_t)cells * sizeof(uint32_t)) + scan_temp_bytes_for(cells) + 256;
}

// Sort n pairs from (kin, vin) into (kout, vout) on key bits [begin_bit, end_bit).
// (alt_k, alt_v) is the ping-pong buffer. The first pass writes (kout) when the pass count is
// odd and (alt) when it is even, so kin may alias whichever of the two the first pass does
// not write (and it is never written otherwise).
template <class K>
int radix_sort_pairs(const K* kin, K* kout, const int32_t* vin, int32_t* vout, K* alt_k,
                     int32_t* alt_v, int64_t n, int begin_bit, int end_bit, void* temp,
                     size_t temp_bytes, hipStream_t stream) {
    const int passes = radix_passes(begin_bit, end_bit);
    if (n <= 0) return TDGS_OK;
    if (passes == 0) {
        if (kout != kin) TDGS_HIP(hipMemcpyAsync(kout, kin, n * sizeof(K), hipMemcpyDeviceToDevice, stream));
        if (vout != vin) TDGS_HIP(hipMemcpyAsync(vout, vin, n * sizeof(int32_t), hipMemcpyDeviceToDevice, stream));
        return TDGS_OK;
    }
    const int64_t ntiles = ceil_div(n, kRsTile);
    const int64_t cells = ntiles * kRsBins;
    Arena ar(temp, temp_bytes);
    uint32_t* counts = ar.take<uint32_t>(cells);
    const size_t sbytes = scan_temp_bytes_for(cells);
    void* stemp = ar.take<char>((int64_t)sbytes);
    if (!counts || !stemp) {
        set_error("radix sort scratch too small (%zu bytes for %lld keys)", temp_bytes, (long long)n);
        return TDGS_ERR_CAPACITY;
    }
    const K* src_k = kin;
    const int32_t* src_v = vin;
    for (int p = 0; p < passes; ++p) {
        const int shift = begin_bit + 8 * p;
        const int nbits = end_bit - shift < 8 ? end_bit - shift : 8;
        const bool to_out = ((passes - 1 - p) % 2) == 0;
        K* dk = to_out ? kout : alt_k;
        int32_t* dv = to_out ? vout : alt_v;
        k_radix_count<K><<<(unsigned)ntiles, kRsThreads, 0, stream>>>(src_k, n, shift, nbits, counts, ntiles);
        TDGS_LAUNCHED();
        TDGS_TRY(device_scan(ItemsU32{counts}, ItemsU32{counts}, WriteExclusiveU32{counts}, cells,
                             stemp, sbytes, nullptr, stream));
        k_radix_scatter<K><<<(unsigned)ntiles, kRsThreads, 0, stream>>>(src_k, src_v, dk, dv, n, shift,
                                                                         nbits, counts, ntiles);
        TDGS_LAUNCHED();
        src_k = dk;
        src_v = dv;
    }
    return TDGS_OK;
}

}  // namespace tdgs
