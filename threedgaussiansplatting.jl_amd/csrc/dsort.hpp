// dsort.hpp — the render pipeline's depth presort by sampled buckets.
//
// Input: the projection's depth key of every Gaussian slot i (the float bits of its depth;
// all ones when it is culled or empty), whose filtered index is i + 1. Output: the non-empty
// Gaussians ordered by (depth bits, fgidx) — the order the reference's stable sort of
// (tile, depth) keys gives every tile's list (forward_core.jl:605-660) — with, for every
// output index, the Gaussian's tile rectangle gathered alongside and the packed tile/block
// counts summed per count-scan tile (RsGather).
//
// Three launches instead of the eight of a 4-pass LSD radix sort over the 32-bit keys, whose
// short, latency-bound passes cost ~8 us each whatever their work:
//   k_ds_count      every workgroup first takes 255 splitters from a sample of 8192 keys
//                   (strided over the slots, written by the projection beside the keys):
//                   histogrammed in 4096 bins over its range, splitters at bin edges near
//                   equal ranks of its non-empty part, as composites (depth bits << 32 |
//                   fgidx), so that every bucket holds about 1/256 of the non-empty
//                   Gaussians however the depths are distributed. Then, per 4096-key radix
//                   tile, each key's bucket id (a binary search in the splitters, written as
//                   one byte per slot) and their histogram as a row of the count table plus
//                   16-tile group sums
//   k_ds_scatter    the stable radix pass on the bucket id (grouped offsets, as
//                   k_rs_scatter_grouped); tile 0 writes the buckets' starts
//   k_ds_buckets    one workgroup per bucket sorts its Gaussians by depth bits: up to 8192
//                   held in registers (the fewest of up to 8 per thread), an LSD pass per 9
//                   bits over only the bits in which the bucket's keys differ, each pass
//                   ranked with wavefront ballots and permuted through LDS (the keys less the
//                   bucket's smallest, so the passes cover its range); larger buckets (a
//                   skewed sample) take the same passes chunk by chunk through global memory.
//                   Then the output.
// Every pass is stable and the buckets partition the composite order, so ties in depth keep
// fgidx order: the result equals the LSD sort's bit for bit, and does not depend on the
// splitters (they only set the buckets' sizes).
#pragma once

#include "sort.hpp"

namespace tdgs {

constexpr int kDsBuckets = kRsBins;                     // 256: one 8-bit radix pass on the bucket id
constexpr int kDsThreads = 1024;                        // splitter and bucket workgroups
constexpr int kDsWaves = kDsThreads / kWave;
constexpr int kDsItems = 8;                             // keys per thread of a bucket sort (16: register spills)
constexpr int kDsCap = kDsThreads * kDsItems;           // buckets of up to 8192 Gaussians sort in LDS
constexpr int kDsSampleItems = 8;
// 8192 sampled keys: ~17 non-empty samples per bucket at 1M Gaussians, 1080p, whose largest
// bucket then holds fewer keys (the bucket sorts take as long as their largest bucket): presort
// 53.3 -> 50.7 us against 4096 samples, no faster with 16384 (2048: +3 us of sample loads less,
// but buckets up to 3.6x the mean)
constexpr int kDsSample = kDsThreads * kDsSampleItems;
using DsTile = RsTile<uint64_t>;                        // the bucket pass: 4096-key tiles, 512 threads
constexpr int kDsDigit = 512;                           // bucket sorts: 9-bit digits (2 passes cover the
                                                        // 15-20 bits a bucket's keys typically span)

// The sample of the slots' depth keys the splitters come from: sample p < kDsSample holds the
// key of slot p n / kDsSample (n > kDsSample), else of slot p < n. The writer of slot i's key
// (the projection) stores it here too when slot i is sampled: p = ceil(i kDsSample / n) is the
// only candidate (p n / kDsSample increases strictly with p), so the splitter kernel reads
// the sample contiguously instead of gathering it.
__device__ __forceinline__ void ds_sample_store(uint32_t* sample, int64_t n, int64_t i, uint32_t key) {
    if (n <= kDsSample) {
        sample[i] = key;
        return;
    }
    const int64_t p = (i * kDsSample + n - 1) / n;
    if (p < kDsSample && p * n / kDsSample == i) sample[p] = key;
}

// The bucket of composite c: the number of splitters s[0..254] (ascending) that are <= c.
__device__ __forceinline__ int ds_bucket(uint64_t c, const uint64_t* s) {
    int b = 0;
#pragma unroll
    for (int step = kDsBuckets / 2; step >= 1; step >>= 1)
        if (s[b + step - 1] <= c) b += step;
    return b;
}

// Exclusive prefix over a 1024-thread workgroup of one value per thread (tmp: kDsWaves words;
// ends with a block barrier).
__device__ __forceinline__ uint32_t ds_block_excl_scan(uint32_t a, uint32_t* tmp) {
    const int lane = __lane_id(), w = threadIdx.x / kWave;
    uint32_t incl = a;
    for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) tmp[w] = incl;
    __syncthreads();
    uint32_t off = 0;
#pragma unroll
    for (int q = 0; q < kDsWaves; ++q) off += q < w ? tmp[q] : 0u;
    __syncthreads();
    return off + incl - a;
}

// Stable rank of the keys of a 1024-thread workgroup held in registers, `it` (<= IT) per
// thread: the key of item j < it of lane l in wavefront w sits at position (w it + j) 64 + l
// and is valid when that position is below n. Leaves in pos[j] its rank among the
// wavefront's earlier keys of its digit (k >> shift) & (2^nb - 1) (nb <= log2 DB) and in
// wh[w][d] the wavefront's count of digit d, then (digit owners, threads < DB) turns wh[.][d]
// into the earlier wavefronts' counts and returns digit d's total in tot. Ends with a block
// barrier. (Each item costs nb ballots: `it` is the fewest items per thread that hold the n
// keys.)
template <int IT, int DB>
__device__ __forceinline__ void ds_rank(const uint32_t (&k)[IT], int it, int n, int shift, int nb,
                                        uint32_t (&pos)[IT], uint32_t (*wh)[DB], uint32_t& tot) {
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const uint32_t mask = (1u << nb) - 1u;
    for (int i = t; i < kDsWaves * DB; i += kDsThreads) (&wh[0][0])[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < IT; ++j) {
        if (j >= it || (w * it + j) * kWave >= n) break;   // (wave-uniform)
        const bool valid = (w * it + j) * kWave + lane < n;
        const uint32_t d = (k[j] >> shift) & mask;
        const uint64_t peers = match_digit(d, nb, valid);
        const uint64_t below = peers & lanemask_lt();
        const uint32_t c = wh[w][d];
        pos[j] = c + (uint32_t)__popcll(below);
        if (valid && below == 0) wh[w][d] = c + (uint32_t)__popcll(peers);
    }
    __syncthreads();
    tot = 0;
    if (t < DB) {
#pragma unroll
        for (int i = 0; i < kDsWaves; ++i) {
            const uint32_t c = wh[i][t];
            wh[i][t] = tot;
            tot += c;
        }
    }
    __syncthreads();
}

// Stable LSD sort of the n register-held (key, value) pairs of a 1024-thread workgroup (layout
// as ds_rank, `it` items per thread) on key bits [0, nbits), log2 DB bits a pass, permuted
// through stage (n entries of LDS); the pairs end in the same registers in sorted order.
template <int IT, int DB>
__device__ void ds_sort_regs(uint32_t (&k)[IT], int32_t (&v)[IT], int it, int n, int nbits, uint64_t* stage,
                             uint32_t (*wh)[DB], uint32_t* loc, uint32_t* tmp) {
    static_assert(DB <= kDsThreads && (DB & (DB - 1)) == 0, "one owner thread per digit");
    constexpr int W = __builtin_ctz(DB);
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    for (int shift = 0; shift < nbits; shift += W) {
        const int nb = nbits - shift < W ? nbits - shift : W;
        const uint32_t mask = (1u << nb) - 1u;
        uint32_t pos[IT], tot;
        ds_rank<IT, DB>(k, it, n, shift, nb, pos, wh, tot);
        const uint32_t start = ds_block_excl_scan(t < DB ? tot : 0u, tmp);
        if (t < DB) loc[t] = start;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            if (j < it && (w * it + j) * kWave + lane < n) {
                const uint32_t d = (k[j] >> shift) & mask;
                stage[loc[d] + wh[w][d] + pos[j]] = ((uint64_t)k[j] << 32) | (uint32_t)v[j];
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            const int p = (w * it + j) * kWave + lane;
            if (j < it && p < n) {
                const uint64_t x = stage[p];
                k[j] = (uint32_t)(x >> 32);
                v[j] = (int32_t)(uint32_t)x;
            }
        }
        __syncthreads();
    }
}

// Splitters from the sample, by one workgroup of NTH threads: the non-empty keys among the
// kDsSample sampled slots (ds_sample_store) are histogrammed in 4096 bins over their range
// [kmin, kmax]; for b < 255, spl[b] = (the lower edge of the bin holding the sample of rank
// (b + 1) ne / 256, ne non-empty samples) << 32, a composite below every key of that bin and
// above every key of the bins before it; spl[255] and, without a non-empty sample, every
// splitter are all ones. (No sort: the splitters only balance the buckets, the order does not
// depend on them.) spl, s_h (4096 words), s_mm (2) and s_w (NTH / 64) are LDS; the caller
// waits at a barrier before reading spl.
constexpr int kDsHistBits = 12;
template <int NTH>
__device__ __forceinline__ void ds_splitters(const uint32_t* __restrict__ sample, int64_t n, uint64_t* spl,
                                             uint32_t* s_h, uint32_t* s_mm, uint32_t* s_w) {
    constexpr int kBins = 1 << kDsHistBits;
    constexpr int kPer = kBins / NTH;          // bins per thread
    constexpr int kItems = kDsSample / NTH;    // sampled keys per thread
    constexpr int kWaves = NTH / kWave;
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const int ns = (int)(n < kDsSample ? n : kDsSample);
    uint32_t k[kItems];
    uint32_t mn = 0xffffffffu, mx = 0u;
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
        const int p = j * NTH + t;
        k[j] = 0xffffffffu;
        if (p < ns) k[j] = sample[p];
        if (k[j] != 0xffffffffu) {
            mn = k[j] < mn ? k[j] : mn;
            mx = k[j] > mx ? k[j] : mx;
        }
    }
#pragma unroll
    for (int q = 0; q < kPer; ++q) s_h[q * NTH + t] = 0;
    if (t == 0) {
        s_mm[0] = 0xffffffffu;
        s_mm[1] = 0u;
    }
    for (int d = kWave / 2; d >= 1; d >>= 1) {
        const uint32_t a = __shfl_xor(mn, d, kWave), b = __shfl_xor(mx, d, kWave);
        mn = a < mn ? a : mn;
        mx = b > mx ? b : mx;
    }
    __syncthreads();
    if (lane == 0 && mn <= mx) {
        atomicMin(&s_mm[0], mn);
        atomicMax(&s_mm[1], mx);
    }
    __syncthreads();
    const uint32_t kmin = s_mm[0], kmax = s_mm[1];
    if (kmin > kmax) {   // no non-empty sample (block-uniform)
        if (t < kDsBuckets) spl[t] = ~0ull;
        return;
    }
    const uint32_t span = kmax - kmin;
    const int len = span ? 32 - __clz((int)span) : 0;
    const int shift = len > kDsHistBits ? len - kDsHistBits : 0;
#pragma unroll
    for (int j = 0; j < kItems; ++j)
        if (k[j] != 0xffffffffu) atomicAdd(&s_h[(k[j] - kmin) >> shift], 1u);
    __syncthreads();
    // thread t owns bins t kPer .. t kPer + kPer - 1: their exclusive prefix over all bins
    uint32_t c[kPer], sum = 0;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        c[q] = s_h[t * kPer + q];
        sum += c[q];
    }
    uint32_t incl = sum;
    for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) s_w[w] = incl;
    __syncthreads();
    uint32_t before = incl - sum, ne = 0;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
        const uint32_t x = s_w[q];
        if (q < w) before += x;
        ne += x;
    }
    // splitter b takes the bin of the sample of rank r_b = (b + 1) ne / 256 (r_b < ne)
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const uint32_t lo = before, hi = before + c[q];
        before = hi;
        if (lo == hi) continue;
        const uint64_t edge = (uint64_t)(kmin + ((uint32_t)(t * kPer + q) << shift)) << 32;
        // the first b with r_b >= lo, then every b with r_b < hi
        int b = (int)(((uint64_t)lo * kDsBuckets) / ne);
        b = b > 0 ? b - 1 : 0;
        for (; b < kDsBuckets - 1; ++b) {
            const uint32_t r = (uint32_t)(((uint64_t)(b + 1) * ne) / kDsBuckets);
            if (r >= hi) break;
            if (r >= lo) spl[b] = edge;
        }
    }
    if (t == 0) spl[kDsBuckets - 1] = ~0ull;
}

// Per 4096-key tile: the splitters (every workgroup computes them from the sample: cheaper
// than a launch of their own), each slot's bucket id in bid (0 for an empty key) and the
// histogram of the non-empty keys' buckets, as row cnt[tile][.] and added into the group sums
// grp[tile / kRsGroup][.] (zero on entry).
__global__ __launch_bounds__(kRsThreads) void k_ds_count(const uint32_t* __restrict__ keys, int64_t n,
                                                         const uint32_t* __restrict__ sample, uint8_t* __restrict__ bid,
                                                         uint32_t* __restrict__ cnt, uint32_t* __restrict__ grp) {
    __shared__ uint64_t s_spl[kDsBuckets];
    __shared__ uint32_t s_hist[1 << kDsHistBits];
    __shared__ uint32_t s_mm[2];
    __shared__ uint32_t s_w[kRsThreads / kWave];
    __shared__ uint32_t s_h[kRsBins];
    const int t = threadIdx.x;
    constexpr int IT = DsTile::kItems;
    const int64_t base = (int64_t)blockIdx.x * DsTile::kTile + t;
    uint32_t key[IT];
#pragma unroll
    for (int j = 0; j < IT; ++j) {
        const int64_t i = base + (int64_t)j * kRsThreads;
        key[j] = i < n ? keys[i] : 0xffffffffu;
    }
    if (t < kDsBuckets) s_h[t] = 0;
    ds_splitters<kRsThreads>(sample, n, s_spl, s_hist, s_mm, s_w);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < IT; ++j) {
        const int64_t i = base + (int64_t)j * kRsThreads;
        const bool valid = key[j] != 0xffffffffu;
        const uint32_t d = valid ? (uint32_t)ds_bucket(((uint64_t)key[j] << 32) | (uint64_t)(i + 1), s_spl) : 0u;
        if (i < n) bid[i] = (uint8_t)d;
        const uint64_t peers = match_digit(d, 8, valid);
        if (valid && (peers & lanemask_lt()) == 0) atomicAdd(&s_h[d], (uint32_t)__popcll(peers));
    }
    __syncthreads();
    if (t < kRsBins) {
        const uint32_t c = s_h[t];
        cnt[(int64_t)blockIdx.x * kRsBins + t] = c;
        if (c) atomicAdd(&grp[(int64_t)(blockIdx.x / kRsGroup) * kRsBins + t], c);
    }
}

// The stable radix pass on the bucket id: bkey[o] = (bucket << 32) | depth bits, bval[o] =
// fgidx for the output index o of every non-empty key; tile 0 writes the buckets' starts to
// bstart[0..255], the non-empty count to bstart[256] and *d_kept.
__global__ __launch_bounds__(kRsThreads) __attribute__((amdgpu_waves_per_eu(6))) void k_ds_scatter(
    const uint32_t* __restrict__ keys, int64_t n, const uint8_t* __restrict__ bid, const uint32_t* __restrict__ cnt,
    const uint32_t* __restrict__ grp, uint64_t* __restrict__ bkey, int32_t* __restrict__ bval, uint32_t* err,
    int64_t* d_kept, uint32_t* bstart) {
    constexpr int IT = DsTile::kItems;
    constexpr int TILE = DsTile::kTile;
    __shared__ uint32_t s_raw[rs_stage_words<uint64_t>()];
    __shared__ uint32_t s_part[kRsBins];
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const int64_t tile = blockIdx.x;
    const int64_t wbase = tile * TILE + w * (IT * kWave) + lane;
    uint32_t k32[IT], b8[IT];
#pragma unroll
    for (int j = 0; j < IT; ++j) {
        const int64_t i = wbase + (int64_t)j * kWave;
        k32[j] = i < n ? keys[i] : 0xffffffffu;
        b8[j] = i < n ? bid[i] : 0u;
    }
    uint32_t off_t, total_t;
    rs_group_offsets(cnt, grp, tile, (n + TILE - 1) / TILE, off_t, total_t, s_part);   // (ends with a barrier)
    uint64_t key[IT];
    int32_t val[IT];
    bool valid[IT];
#pragma unroll
    for (int j = 0; j < IT; ++j) {
        const int64_t i = wbase + (int64_t)j * kWave;
        valid[j] = k32[j] != 0xffffffffu;
        key[j] = ((uint64_t)b8[j] << 32) | k32[j];
        val[j] = (int32_t)(i + 1);
    }
    rs_scatter_tile<uint64_t>(key, val, valid, tile, n, 32, 8, off_t, total_t, bkey, bval, err, d_kept, s_raw,
                              RsGather{}, nullptr, nullptr, bstart);
}

// Output indices i0 + 64 (w it + j) + lane, j < it (it 64 <= 2048), valid below n, of the
// sorted Gaussians f[j]: sorted_f[i] = fgidx and the gather of RsGather (rectangle into depth
// order, the packed counts summed per count-scan tile of 2048 outputs). The rectangle loads of
// all items are issued before any store. A wavefront's it 64 outputs span at most two
// count-scan tiles: its sums for both are reduced over the wavefront and added with at most two
// atomics.
template <int IT>
__device__ __forceinline__ void ds_emit(int64_t i0, int it, int n, const int32_t (&f)[IT],
                                        int32_t* __restrict__ sorted_f, const RsGather& g) {
    const int lane = __lane_id(), w = threadIdx.x / kWave;
    if ((w * it) * kWave >= n) return;   // (wave-uniform: no output)
    int4 r[IT];
#pragma unroll
    for (int j = 0; j < IT; ++j) {
        const bool valid = j < it && (w * it + j) * kWave + lane < n;
        r[j] = g.src && valid ? g.src[f[j] - 1] : make_int4(1, 1, 0, 0);
    }
    const int64_t qa = (i0 + (int64_t)(w * it) * kWave) >> kRsSumShift;   // the wavefront's first tile
    int64_t s0 = 0, s1 = 0;
#pragma unroll
    for (int j = 0; j < IT; ++j) {
        if (j >= it) break;
        const int p = (w * it + j) * kWave + lane;
        const int64_t i = i0 + p;
        if (p < n) {
            sorted_f[i] = f[j];
            if (g.src) {
                g.dst[i] = r[j];
                const int32_t blocks = (((r[j].z - 1) >> g.sx) - ((r[j].x - 1) >> g.sx) + 1) *
                                       (((r[j].w - 1) >> g.sy) - ((r[j].y - 1) >> g.sy) + 1);
                const int64_t item =
                    ((int64_t)((r[j].z - r[j].x + 1) * (r[j].w - r[j].y + 1)) << 32) | (int64_t)blocks;
                if ((i >> kRsSumShift) == qa) s0 += item;
                else s1 += item;
            }
        }
    }
    if (g.sums) {
        for (int d = kWave / 2; d >= 1; d >>= 1) {
            s0 += __shfl_xor(s0, d, kWave);
            s1 += __shfl_xor(s1, d, kWave);
        }
        if (lane == 0) {
            if (s0) atomicAdd(reinterpret_cast<unsigned long long*>(g.sums + qa), (unsigned long long)s0);
            if (s1) atomicAdd(reinterpret_cast<unsigned long long*>(g.sums + qa + 1), (unsigned long long)s1);
        }
    }
}

// One workgroup per bucket: its Gaussians sorted by depth bits (stable: the bucket pass kept
// them in fgidx order), then emitted at the bucket's start. (akey, aval): arrays of the slots'
// size that, with (bkey, bval), ping-pong the passes of a bucket past kDsCap (each workgroup
// only touches its bucket's range).
__global__ __launch_bounds__(kDsThreads) void k_ds_buckets(uint64_t* bkey, int32_t* bval, uint64_t* akey,
                                                           int32_t* aval, const uint32_t* __restrict__ bstart,
                                                           int32_t* __restrict__ sorted_f, RsGather g) {
    __shared__ uint64_t s_stage[kDsCap];
    __shared__ uint32_t s_wh[kDsWaves][kDsDigit];
    __shared__ uint32_t s_loc[kDsDigit];
    __shared__ uint32_t s_tmp[kDsWaves];
    __shared__ uint32_t s_mm[2];
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const int64_t start = bstart[blockIdx.x];
    const int nb = (int)((int64_t)bstart[blockIdx.x + 1] - start);
    if (nb <= 0) return;   // (uniform)
    if (t == 0) {
        s_mm[0] = 0xffffffffu;
        s_mm[1] = 0u;
    }
    __syncthreads();
    if (nb <= kDsCap) {
        const int it = (nb + kDsThreads - 1) / kDsThreads;   // items per thread
        uint32_t k[kDsItems];
        int32_t v[kDsItems];
        uint32_t mn = 0xffffffffu, mx = 0u;
#pragma unroll
        for (int j = 0; j < kDsItems; ++j) {
            const int p = (w * it + j) * kWave + lane;
            k[j] = 0u;
            v[j] = 0;
            if (j < it && p < nb) {
                k[j] = (uint32_t)bkey[start + p];
                v[j] = bval[start + p];
                mn = k[j] < mn ? k[j] : mn;
                mx = k[j] > mx ? k[j] : mx;
            }
        }
        for (int d = kWave / 2; d >= 1; d >>= 1) {
            const uint32_t a = __shfl_xor(mn, d, kWave), b = __shfl_xor(mx, d, kWave);
            mn = a < mn ? a : mn;
            mx = b > mx ? b : mx;
        }
        if (lane == 0) {
            atomicMin(&s_mm[0], mn);
            atomicMax(&s_mm[1], mx);
        }
        __syncthreads();
        const uint32_t kmin = s_mm[0], span = s_mm[1] - kmin;
        const int bits = span ? 32 - __clz((int)span) : 0;   // the keys less kmin fit in `bits` bits
#pragma unroll
        for (int j = 0; j < kDsItems; ++j) k[j] -= kmin;    // (invalid items are never read)
        ds_sort_regs<kDsItems, kDsDigit>(k, v, it, nb, bits, s_stage, s_wh, s_loc, s_tmp);
        ds_emit<kDsItems>(start, it, nb, v, sorted_f, g);
        return;
    }
    // A bucket past kDsCap: the same LSD passes over chunks of kDsCap pairs through global
    // memory, ping-ponging between (akey, aval) and (bkey, bval) at the bucket's offsets.
    const uint64_t* sk = bkey + start;
    const int32_t* sv = bval + start;
    uint32_t mn = 0xffffffffu, mx = 0u;
    for (int p = t; p < nb; p += kDsThreads) {
        const uint32_t x = (uint32_t)sk[p];
        mn = x < mn ? x : mn;
        mx = x > mx ? x : mx;
    }
    for (int d = kWave / 2; d >= 1; d >>= 1) {
        const uint32_t a = __shfl_xor(mn, d, kWave), b = __shfl_xor(mx, d, kWave);
        mn = a < mn ? a : mn;
        mx = b > mx ? b : mx;
    }
    if (lane == 0) {
        atomicMin(&s_mm[0], mn);
        atomicMax(&s_mm[1], mx);
    }
    __syncthreads();
    const uint32_t kmin = s_mm[0], span = s_mm[1] - kmin;
    const int bits = span ? 32 - __clz((int)span) : 0;
    const int nchunks = (nb + kDsCap - 1) / kDsCap;
    uint32_t* s_base = s_loc;   // running output start of each digit
    int pass = 0;
    constexpr int W = __builtin_ctz(kDsDigit);
    for (int shift = 0; shift < bits; shift += W, ++pass) {
        const int nbt = bits - shift < W ? bits - shift : W;
        const uint32_t mask = (1u << nbt) - 1u;
        uint64_t* dk = (pass % 2 == 0 ? akey : bkey) + start;
        int32_t* dv = (pass % 2 == 0 ? aval : bval) + start;
        // digit histogram of the whole bucket -> each digit's start
        for (int i = t; i < kDsDigit; i += kDsThreads) s_wh[0][i] = 0;
        __syncthreads();
        for (int p = t; p < nb; p += kDsThreads) atomicAdd(&s_wh[0][(((uint32_t)sk[p] - kmin) >> shift) & mask], 1u);
        __syncthreads();
        const uint32_t h = t < kDsDigit ? s_wh[0][t] : 0u;
        const uint32_t st = ds_block_excl_scan(h, s_tmp);
        if (t < kDsDigit) s_base[t] = st;
        __syncthreads();
        for (int c = 0; c < nchunks; ++c) {
            const int c0 = c * kDsCap;
            const int nc = nb - c0 < kDsCap ? nb - c0 : kDsCap;
            const int it = (nc + kDsThreads - 1) / kDsThreads;
            uint32_t k[kDsItems];
            int32_t v[kDsItems];
#pragma unroll
            for (int j = 0; j < kDsItems; ++j) {
                const int p = (w * it + j) * kWave + lane;
                k[j] = j < it && p < nc ? (uint32_t)sk[c0 + p] - kmin : 0u;
                v[j] = j < it && p < nc ? sv[c0 + p] : 0;
            }
            uint32_t pos[kDsItems], tot;
            ds_rank<kDsItems, kDsDigit>(k, it, nc, shift, nbt, pos, s_wh, tot);
#pragma unroll
            for (int j = 0; j < kDsItems; ++j) {
                if (j < it && (w * it + j) * kWave + lane < nc) {
                    const uint32_t d = (k[j] >> shift) & mask;
                    const uint32_t o = s_base[d] + s_wh[w][d] + pos[j];
                    dk[o] = k[j] + kmin;
                    dv[o] = v[j];
                }
            }
            __syncthreads();
            if (t < kDsDigit) s_base[t] += tot;
            __syncthreads();
        }
        __threadfence();   // this pass's writes are the next pass's reads (other waves)
        __syncthreads();
        sk = dk;
        sv = dv;
    }
    for (int c0 = 0; c0 < nb; c0 += kDsThreads) {
        const int32_t f[1] = {c0 + t < nb ? sv[c0 + t] : 0};
        ds_emit<1>(start + c0, 1, nb - c0, f, sorted_f, g);
    }
}

// Scratch of the bucketed presort: splitters (256), bucket starts (257), the slots' bucket ids,
// and the bucket pass's output and its ping-pong partner (slots each).
struct DsScratch {
    uint32_t* bstart;
    uint32_t* sample;   // kDsSample sampled keys (written by the projection)
    uint8_t* bid;     // bucket id of every slot
    uint64_t* bkey;
    int32_t* bval;
    uint64_t* akey;
    int32_t* aval;
};

// Whether the bucketed presort handles n slots with the grouped count tables (zgrp_words
// zeroed words of group sums).
// Slots up to which the bucket presort is used. Its buckets grow with n (one workgroup each,
// 256 of them) and the radix passes take over above: measured 55 vs 68 us at 1M slots (1920 x
// 1080), 200 vs 142 us at 3M (3840 x 2160); the two lines cross near 1.4M.
constexpr int64_t kDsMaxSlots = 1400000;
inline bool ds_applicable(int64_t n, int64_t zgrp_words) {
    const int64_t tiles = ceil_div(n > 0 ? n : 1, DsTile::kTile);
    return n > 0 && n <= kDsMaxSlots && tiles <= kRsMaxGroupedTiles &&
           zgrp_words >= rs_groups(tiles) * kRsBins;
}

// The presort of n slots of depth keys (fgidx = slot + 1): sorted_f[0..N_b) and the gather;
// *d_kept = N_b. cnt: a count table of ceil(n / 4096) x 256 words; zgrp: zeroed group sums.
inline int depth_sort_buckets(const uint32_t* keys, int64_t n, const DsScratch& d, uint32_t* cnt, uint32_t* zgrp,
                              int32_t* sorted_f, RsGather g, uint32_t* err, int64_t* d_kept, hipStream_t s) {
    const int64_t tiles = ceil_div(n, DsTile::kTile);
    k_ds_count<<<(unsigned)tiles, kRsThreads, 0, s>>>(keys, n, d.sample, d.bid, cnt, zgrp);
    TDGS_LAUNCHED();
    k_ds_scatter<<<(unsigned)tiles, kRsThreads, 0, s>>>(keys, n, d.bid, cnt, zgrp, d.bkey, d.bval, err, d_kept,
                                                         d.bstart);
    TDGS_LAUNCHED();
    k_ds_buckets<<<kDsBuckets, kDsThreads, 0, s>>>(d.bkey, d.bval, d.akey, d.aval, d.bstart, sorted_f, g);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

}  // namespace tdgs
