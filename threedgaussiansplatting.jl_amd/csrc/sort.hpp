// sort.hpp — stable LSD radix sort of (key, int32 value) pairs on a key bit range
// [begin_bit, end_bit), digits of at most 8 bits; replaces CUB DeviceRadixSort::SortPairs
// (deps/cub_sort_pairs/cub_sort_pairs_wrapper.cu:31-43).
//
// Each pass is three launches over tiles of kRsTile consecutive keys:
//   count    per-tile 256-bin digit histogram, written digit-major: counts[d][tile]
//   scan     one workgroup per digit turns its row into exclusive prefixes over the tiles
//            and writes the digit total                                     (k_rs_scan_rows)
//   scatter  each tile ranks its keys stably (wavefront ballot match + per-wave digit
//            counters in LDS), stages the tile in LDS in digit order, and writes it out in
//            contiguous per-digit runs at totals-prefix[d] + counts[d][tile]  (k_rs_scatter)
// Stability: within a tile keys are ranked in index order (wave, item, lane); across tiles
// the row scan orders tiles by index, so equal digits keep their input order.
//
// The count of a pass can come from the kernel that produced the keys (the render pipeline
// fuses it into key emission), so a pass reads its keys once.
//
// Grouped variant (radix_sort_pairs_grouped, up to kRsMaxGroupedTiles tiles): two launches a
// pass. The count writes each tile's histogram as one contiguous row (cnt[tile][digit]) and
// adds it into the sums of its group of kRsGroup tiles (grp[group][digit], 16 atomics per
// word); each scatter workgroup then finds its own offsets by summing the earlier groups'
// sums and the earlier tiles of its group (at most G + 15 loads per digit, all in flight at
// once) instead of waiting for a scan launch. The group sums must be zero on entry.
// Decoupled look-back (Onesweep, Adinets & Merrill 2022) replaces the count and scan
// launches by a chained prefix over tiles; on this part it was measured slower: with
// ~800 tiles in flight the walk back to a published prefix takes several dependent
// round trips of ~2.5 us under load, which halved the scatter's 5.6 TB/s.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace tdgs {

constexpr int kRsThreads = 512;   // scatter / count: threads per workgroup
constexpr int kRsBins = 256;
// Keys per thread and per tile (4096-key tiles). 8192-key tiles for the 64-bit keys (twice
// the keys per digit per tile, so twice-as-long output runs) measured 6% faster on 751M keys
// but 35% slower on 6M keys (half the workgroups, at 151 VGPRs and 74 KB of LDS each).
template <class K>
struct RsTile {
    static constexpr int kItems = 8;
    static constexpr int kTile = kRsThreads * kItems;
};
// 32-bit keys are the depth presort's: ~1M keys of which the later passes sort the few
// hundred thousand non-empty ones. 2048-key tiles spread them over more CUs (72 us vs 81 us
// for the four passes at 1M Gaussians; 1024- and 512-key tiles: 79 us and 102 us).
template <>
struct RsTile<uint32_t> {
    static constexpr int kItems = 4;
    static constexpr int kTile = kRsThreads * kItems;
};
constexpr int kRsMinTile = kRsThreads * 4;   // the smallest tile above (sizes the count table)
static_assert(RsTile<uint16_t>::kTile >= kRsMinTile && RsTile<uint32_t>::kTile >= kRsMinTile &&
                  RsTile<uint64_t>::kTile >= kRsMinTile,
              "count table sized for the smallest tile");
constexpr int kRsWaves = kRsThreads / kWave;
static_assert(kRsThreads >= kRsBins && kRsThreads % kRsBins == 0, "digit owners");

// Column of radix tile `tile` in a row of the digit-major count table. Workgroups are dealt
// round-robin to the kXcds XCDs (each with its own L2), so tile t runs on XCD t % 8; the columns
// are grouped by XCD (tile t at (t % 8) * (pitch / 8) + t / 8) so that the cache lines one
// XCD's count workgroups write, and its scatter workgroups read, are not shared with another
// XCD's L2 (partial lines merged across XCDs cost 7x the table in write traffic). Rows are
// rs_pitch(tiles) words apart.
__host__ __device__ inline int64_t rs_pitch(int64_t tiles) { return (tiles + kXcds - 1) / kXcds * kXcds; }
__host__ __device__ inline int64_t rs_col(int64_t tile, int64_t tiles) {
    return (tile % kXcds) * (rs_pitch(tiles) / kXcds) + tile / kXcds;
}
// Entry of digit d and radix tile `tile` in the count table.
__host__ __device__ inline int64_t rs_entry(int d, int64_t tile, int64_t tiles) {
    return (int64_t)d * rs_pitch(tiles) + rs_col(tile, tiles);
}

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

// Exclusive scan of one value per thread over the first 256 threads of the block (the
// digit owners); every thread of the block must call it.
__device__ __forceinline__ uint32_t digit_excl_scan(uint32_t a, uint32_t* s_tmp) {
    const int lane = __lane_id(), wave = threadIdx.x / kWave;
    uint32_t ia = a;
    for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = __shfl_up(ia, d, kWave);
        if (lane >= d) ia += o;
    }
    if (lane == kWave - 1 && wave < kRsBins / kWave) s_tmp[wave] = ia;
    __syncthreads();
    uint32_t off = 0;
    for (int w = 0; w < wave && w < kRsBins / kWave; ++w) off += s_tmp[w];
    return off + ia - a;
}

// Histogram of one digit over a tile into LDS (wave-aggregated atomics); returns after a
// block barrier with s_h complete.
template <class K>
__device__ __forceinline__ void tile_digit_histogram(const K* __restrict__ keys, int64_t n, int64_t tile, int shift,
                                                     int nbits, uint32_t* s_h, bool drop_max = false) {
    constexpr int kRsItems = RsTile<K>::kItems;
    const int t = threadIdx.x;
    for (int i = t; i < kRsBins; i += kRsThreads) s_h[i] = 0;
    __syncthreads();
    const uint32_t mask = (1u << nbits) - 1u;
    const int64_t base = tile * RsTile<K>::kTile + t;
    K key[kRsItems];
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        const int64_t i = base + (int64_t)k * kRsThreads;
        key[k] = i < n ? keys[i] : (K)0;
    }
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        const bool valid = base + (int64_t)k * kRsThreads < n && !(drop_max && key[k] == (K)~(K)0);
        const uint32_t d = (uint32_t)(key[k] >> shift) & mask;
        const uint64_t peers = match_digit(d, nbits, valid);
        if (valid && (peers & lanemask_lt()) == 0) atomicAdd(&s_h[d], (uint32_t)__popcll(peers));
    }
    __syncthreads();
}

// d_n, when not null, replaces n by a count computed on the device, min(*d_n, n) (the grid
// still covers n);
// drop_max leaves keys equal to the all-ones key out of the count (and of the sort).
template <class K>
__global__ __launch_bounds__(kRsThreads) void k_rs_count(const K* __restrict__ keys, int64_t n, int shift,
                                                         int nbits, uint32_t* __restrict__ counts, int64_t tiles,
                                                         const int64_t* d_n, int drop_max) {
    __shared__ uint32_t s_h[kRsBins];
    // (tiles past a device count hold no keys; the row scan skips their columns)
    if (d_n && (int64_t)blockIdx.x * RsTile<K>::kTile >= *d_n) return;
    tile_digit_histogram(keys, d_n ? (*d_n < n ? *d_n : n) : n, blockIdx.x, shift, nbits, s_h, drop_max != 0);
    if (threadIdx.x < kRsBins) counts[rs_entry(threadIdx.x, blockIdx.x, tiles)] = s_h[threadIdx.x];
}

// Workgroup d: exclusive prefix of digit d's counts over the tiles (in tile order), in place,
// total to totals[d]. With d_n (device count, may be null), only the tiles holding the first
// *d_n keys (tile_keys per tile) are scanned: the table's other columns are neither written
// by the counts nor read by the scatter.
static __global__ __launch_bounds__(256) void k_rs_scan_rows(uint32_t* __restrict__ counts, int64_t tiles_all,
                                                             uint32_t* __restrict__ totals,
                                                             const int64_t* d_n = nullptr, int tile_keys = 1) {
    __shared__ uint32_t s_tmp[4];
    uint32_t* const row0 = counts + (int64_t)blockIdx.x * rs_pitch(tiles_all);
    const int64_t per = rs_pitch(tiles_all) / kXcds;
    int64_t tiles = tiles_all;
    if (d_n) {
        const int64_t used = (*d_n + tile_keys - 1) / tile_keys;
        if (used < tiles) tiles = used > 0 ? used : 0;
    }
    // entry of tile i in the row
    auto at = [&](int64_t i) -> uint32_t& { return row0[(i % kXcds) * per + i / kXcds]; };
    const int t = threadIdx.x, lane = __lane_id(), wave = t / kWave;
    constexpr int IT = 8;
    uint32_t carry = 0;
    for (int64_t start = 0; start < tiles; start += 256 * IT) {
        const int64_t b = start + (int64_t)t * IT;
        uint32_t v[IT];
        uint32_t acc = 0;
#pragma unroll
        for (int k = 0; k < IT; ++k) {
            v[k] = b + k < tiles ? at(b + k) : 0u;
            acc += v[k];
        }
        uint32_t incl = acc;
        for (int d = 1; d < kWave; d <<= 1) {
            const uint32_t o = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += o;
        }
        if (lane == kWave - 1) s_tmp[wave] = incl;
        __syncthreads();
        uint32_t off = carry, blk = 0;
        for (int w = 0; w < 4; ++w) {
            if (w < wave) off += s_tmp[w];
            blk += s_tmp[w];
        }
        __syncthreads();
        off += incl - acc;
#pragma unroll
        for (int k = 0; k < IT; ++k) {
            if (b + k < tiles) at(b + k) = off;
            off += v[k];
        }
        carry += blk;
    }
    if (t == 0) totals[blockIdx.x] = carry;
}

// The scatter of one radix tile (tile index `tile`, kRsThreads threads) whose keys and values
// are in registers: thread t = (wave w, lane l) holds in item k the key of tile index
// w kItems 64 + k 64 + l, valid[k] false for keys that are not sorted (past n, or dropped).
// Ranks the keys stably (per-wavefront ballot match with per-wave digit counters in LDS,
// items in index order), stages the tile in digit order in s_raw (kTile 32-bit words, or
// 64-bit for 64-bit keys), and writes keys and values out as contiguous per-digit runs at
// totals-prefix[d] + offsets[d][tile] + rank. `n` bounds the output index (an inconsistent
// count sets *err instead of writing out of bounds). When d_kept is not null, tile 0 writes
// the number of keys sorted in all. When gather.src is not null, each written value v (a
// 1-based index) also moves gather.src[v - 1] to gather.dst at the value's output index.
// With sums not null, every gathered rectangle r = (x0, y0, x1, y1) (1-based, inclusive) also
// adds (its tile count << 32) | (the count of 2^sx x 2^sy tile blocks it touches) to
// sums[i >> kRsSumShift] for its output index i (the tile sums of a scan of these packed counts
// in output order, which then needs no reduce launch; sums zero on entry).
struct RsGather {
    const int4* src;
    int4* dst;
    int64_t* sums;
    int sx, sy;
};
constexpr int kRsSumShift = 11;   // 2048 outputs per tile sum

// Adds v of every lane whose key is >= 0 to dst[key]: one atomic per run of equal keys in
// consecutive lanes (the run's sum from an inclusive scan over the wavefront).
__device__ __forceinline__ void wave_run_add(int64_t key, int64_t v, int64_t* dst) {
    const int lane = __lane_id();
    const int64_t prev = __shfl_up(key, 1, kWave);
    const bool head = lane == 0 || prev != key;
    const uint64_t heads = __ballot(head);
    int64_t incl = v;
    for (int d = 1; d < kWave; d <<= 1) {
        const int64_t o = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += o;
    }
    const uint64_t upto = heads & ((2ull << lane) - 1ull);   // heads at or below this lane (lane 0 is one)
    const int start = 63 - __clzll((long long)upto);
    const int64_t before = __shfl(incl, start > 0 ? start - 1 : 0, kWave);
    const bool tail = lane == kWave - 1 || ((heads >> (lane + 1)) & 1ull);
    if (tail && key >= 0) {
        const int64_t sum = incl - (start > 0 ? before : 0);
        if (sum != 0) atomicAdd(reinterpret_cast<unsigned long long*>(dst + key), (unsigned long long)sum);
    }
}

// off_t and total_t (read by the digit owners, threads t < kRsBins): the tile's offset inside
// digit t's output (digit t's keys in earlier tiles) and digit t's total. With V2 a second
// 32-bit payload (val2, one per key) is moved along to vout2. bin_out (may be null): tile 0
// writes each digit's start in the output there, and the keys sorted in all at kRsBins.
template <class K, bool V2 = false>
__device__ __forceinline__ void rs_scatter_tile(const K (&key)[RsTile<K>::kItems], const int32_t (&val)[RsTile<K>::kItems],
                                                const bool (&valid)[RsTile<K>::kItems], int64_t tile, int64_t n,
                                                int shift, int nbits, uint32_t off_t, uint32_t total_t,
                                                K* __restrict__ kout, int32_t* __restrict__ vout, uint32_t* err,
                                                int64_t* d_kept, uint32_t* s_raw, RsGather gather = {},
                                                const uint32_t* val2 = nullptr, uint32_t* __restrict__ vout2 = nullptr,
                                                uint32_t* bin_out = nullptr) {
    constexpr int kRsItems = RsTile<K>::kItems;
    constexpr int kRsTile = RsTile<K>::kTile;
    // Keys narrower than 32 bits are staged as 32-bit words: lanes storing 16-bit keys to
    // neighbouring positions would share LDS words, which the hardware serialises.
    using Stage = typename std::conditional<(sizeof(K) < 4), uint32_t, K>::type;
    Stage* s_buf = reinterpret_cast<Stage*>(s_raw);
    __shared__ uint32_t s_wh[kRsWaves][kRsBins];  // per-wave digit counts -> offsets
    __shared__ uint32_t s_local[kRsBins];         // start of each digit inside the tile
    __shared__ int32_t s_delta[kRsBins];          // output index - tile-local index
    __shared__ uint32_t s_tmp[kRsWaves];
    __shared__ uint32_t s_tile_n;                 // keys of the tile that are sorted
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const bool owner = t < kRsBins;
    for (int i = t; i < kRsWaves * kRsBins; i += kRsThreads) (&s_wh[0][0])[i] = 0;
    __syncthreads();
    const uint32_t mask = (1u << nbits) - 1u;
    const int32_t nn = (int32_t)n;
    uint32_t pos[kRsItems];
    // Rank inside the wavefront, items in index order: the first lane of each group of equal
    // digits advances the wave's counter for that digit after every lane has read it.
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        const uint32_t d = (uint32_t)(key[k] >> shift) & mask;
        const uint64_t peers = match_digit(d, nbits, valid[k]);
        const uint64_t below = peers & lanemask_lt();
        const uint32_t cnt = s_wh[w][d];
        pos[k] = cnt + (uint32_t)__popcll(below);
        if (valid[k] && below == 0) s_wh[w][d] = cnt + (uint32_t)__popcll(peers);
    }
    __syncthreads();

    // Digit owners: wave offsets and the tile's count of the digit.
    uint32_t tot = 0;
    if (owner) {
#pragma unroll
        for (int i = 0; i < kRsWaves; ++i) {
            const uint32_t c = s_wh[i][t];
            s_wh[i][t] = tot;
            tot += c;
        }
    }
    const uint32_t local = digit_excl_scan(tot, s_tmp);
    __syncthreads();
    const uint32_t bin = digit_excl_scan(total_t, s_tmp);
    if (owner) {
        s_local[t] = local;
        s_delta[t] = (int32_t)(bin + off_t) - (int32_t)local;
        if (t == kRsBins - 1) {
            s_tile_n = local + tot;
            if (d_kept && tile == 0) *d_kept = (int64_t)bin + total_t;   // keys sorted in all
        }
        // the digits' starts in the output (and, at kRsBins, the keys sorted in all)
        if (bin_out && tile == 0) {
            bin_out[t] = bin;
            if (t == kRsBins - 1) bin_out[kRsBins] = bin + total_t;
        }
    }
    __syncthreads();

    // Stage keys in digit order, then write contiguous runs per digit.
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        if (valid[k]) {
            const uint32_t d = (uint32_t)(key[k] >> shift) & mask;
            pos[k] += s_local[d] + s_wh[w][d];
            if (pos[k] < (uint32_t)kRsTile) s_buf[pos[k]] = (Stage)key[k];
        }
    }
    __syncthreads();
    const int tile_n = (int)s_tile_n;
    int32_t opos[kRsItems];
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        const int i = k * kRsThreads + t;
        opos[k] = -1;
        if (i < tile_n) {
            const K kk = (K)s_buf[i];
            const uint32_t d = (uint32_t)(kk >> shift) & mask;
            const int32_t o = s_delta[d] + i;
            if (o >= 0 && o < nn) {
                if (kout) kout[o] = kk;   // (null: a last pass whose sorted keys nothing reads)
                opos[k] = o;
            } else {
                atomicOr(err, 1u);   // inconsistent counts: never write out of bounds
            }
        }
    }
    __syncthreads();
    int32_t* s_val = reinterpret_cast<int32_t*>(s_raw);
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        if (valid[k] && pos[k] < (uint32_t)kRsTile) s_val[pos[k]] = val[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        const int i = k * kRsThreads + t;
        int64_t item = 0;
        if (opos[k] >= 0) {
            const int32_t v = s_val[i];
            vout[opos[k]] = v;
            if (gather.src) {
                const int4 r = gather.src[v - 1];
                gather.dst[opos[k]] = r;
                const int32_t blocks = (((r.z - 1) >> gather.sx) - ((r.x - 1) >> gather.sx) + 1) *
                                       (((r.w - 1) >> gather.sy) - ((r.y - 1) >> gather.sy) + 1);
                item = ((int64_t)((r.z - r.x + 1) * (r.w - r.y + 1)) << 32) | (int64_t)blocks;
            }
        }
        // (consecutive lanes hold consecutive outputs of a digit's run: few runs per wavefront)
        if (gather.sums) wave_run_add(opos[k] >= 0 ? (int64_t)(opos[k] >> kRsSumShift) : -1, item, gather.sums);
    }
    if constexpr (V2) {
        __syncthreads();   // every value is read: s_val takes the second payload
#pragma unroll
        for (int k = 0; k < kRsItems; ++k) {
            if (valid[k] && pos[k] < (uint32_t)kRsTile) s_val[pos[k]] = (int32_t)val2[k];
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kRsItems; ++k) {
            if (opos[k] >= 0) vout2[opos[k]] = (uint32_t)s_val[k * kRsThreads + t];
        }
    }
}

// Words of LDS rs_scatter_tile stages a tile of K keys in.
template <class K>
constexpr int rs_stage_words() {
    return RsTile<K>::kTile * (sizeof(K) > 4 ? (int)sizeof(K) : 4) / 4;
}

template <class K>
__global__ __launch_bounds__(kRsThreads) __attribute__((amdgpu_waves_per_eu(6))) void k_rs_scatter(
    const K* __restrict__ kin, const int32_t* __restrict__ vin, K* __restrict__ kout,
    int32_t* __restrict__ vout, int64_t n, int shift, int nbits, const uint32_t* __restrict__ offsets,
    const uint32_t* __restrict__ totals, int64_t tiles, uint32_t* err, const int64_t* d_n, int drop_max,
    int64_t* d_kept, RsGather gather) {
    constexpr int kRsItems = RsTile<K>::kItems;
    constexpr int kRsTile = RsTile<K>::kTile;
    __shared__ uint32_t s_raw[rs_stage_words<K>()];
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const int64_t tile = blockIdx.x;
    if (d_n && *d_n < n) n = *d_n;
    const int32_t base = (int32_t)(tile * kRsTile);
    const int32_t wbase = base + w * (kRsItems * kWave) + lane;
    const int32_t nn = (int32_t)n;
    K key[kRsItems];
    int32_t val[kRsItems];
    bool valid[kRsItems];
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        const int32_t i = wbase + k * kWave;
        key[k] = i < nn ? kin[i] : (K)0;
        val[k] = i < nn ? vin[i] : 0;
    }
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) valid[k] = wbase + k * kWave < nn && !(drop_max && key[k] == (K)~(K)0);
    const bool owner = t < kRsBins;
    rs_scatter_tile<K>(key, val, valid, tile, n, shift, nbits, owner ? offsets[rs_entry(t, tile, tiles)] : 0u,
                       owner ? totals[t] : 0u, kout, vout, err, drop_max ? d_kept : nullptr, s_raw, gather);
}

// ---- grouped count tables ----------------------------------------------------------------
constexpr int kRsGroup = 16;                    // radix tiles per group
constexpr int64_t kRsMaxGroupedTiles = 4096;    // at most 256 groups: 256 + 15 loads per digit
__host__ __device__ inline int64_t rs_groups(int64_t tiles) { return (tiles + kRsGroup - 1) / kRsGroup; }

// Digit owners (t < kRsBins) get the offset of radix tile `tile` inside digit t's output (the
// digit's keys in earlier tiles) and digit t's total over the first tiles_used tiles, from the
// per-tile rows cnt[tile][digit] and the group sums grp[group][digit]; threads kRsBins..2
// kRsBins-1 load the earlier tiles of the tile's own group. Ends with a block barrier.
__device__ __forceinline__ void rs_group_offsets(const uint32_t* __restrict__ cnt, const uint32_t* __restrict__ grp,
                                                 int64_t tile, int64_t tiles_used, uint32_t& off, uint32_t& tot,
                                                 uint32_t* s_part) {
    static_assert(kRsThreads == 2 * kRsBins, "one owner and one helper thread per digit");
    const int t = threadIdx.x;
    const int64_t g = tile / kRsGroup;
    const int64_t groups = rs_groups(tiles_used);
    constexpr int U = 8;
    off = 0;
    tot = 0;
    if (t < kRsBins) {
        for (int64_t q0 = 0; q0 < groups; q0 += U) {
            uint32_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = q0 + u < groups ? grp[(q0 + u) * kRsBins + t] : 0u;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                tot += v[u];
                if (q0 + u < g) off += v[u];
            }
        }
    } else {
        const int d = t - kRsBins;
        uint32_t v[kRsGroup - 1];
#pragma unroll
        for (int u = 0; u < kRsGroup - 1; ++u) {
            const int64_t q = g * kRsGroup + u;
            v[u] = q < tile ? cnt[q * kRsBins + d] : 0u;
        }
        uint32_t in = 0;
#pragma unroll
        for (int u = 0; u < kRsGroup - 1; ++u) in += v[u];
        s_part[d] = in;
    }
    __syncthreads();
    if (t < kRsBins) off += s_part[t];
}

// Per-tile histogram as a row of cnt, added into its group's sums (d_n, drop_max: as k_rs_count).
template <class K>
__global__ __launch_bounds__(kRsThreads) void k_rs_count_grouped(const K* __restrict__ keys, int64_t n, int shift,
                                                                 int nbits, uint32_t* __restrict__ cnt,
                                                                 uint32_t* __restrict__ grp, const int64_t* d_n,
                                                                 int drop_max) {
    __shared__ uint32_t s_h[kRsBins];
    if (d_n && (int64_t)blockIdx.x * RsTile<K>::kTile >= *d_n) return;
    tile_digit_histogram(keys, d_n ? (*d_n < n ? *d_n : n) : n, blockIdx.x, shift, nbits, s_h, drop_max != 0);
    if (threadIdx.x < kRsBins) {
        const uint32_t c = s_h[threadIdx.x];
        cnt[(int64_t)blockIdx.x * kRsBins + threadIdx.x] = c;
        if (c) atomicAdd(&grp[(int64_t)(blockIdx.x / kRsGroup) * kRsBins + threadIdx.x], c);
    }
}

// The scatter with offsets from the grouped tables (arguments as k_rs_scatter's).
template <class K>
__global__ __launch_bounds__(kRsThreads) __attribute__((amdgpu_waves_per_eu(6))) void k_rs_scatter_grouped(
    const K* __restrict__ kin, const int32_t* __restrict__ vin, K* __restrict__ kout,
    int32_t* __restrict__ vout, int64_t n, int shift, int nbits, const uint32_t* __restrict__ cnt,
    const uint32_t* __restrict__ grp, uint32_t* err, const int64_t* d_n, int drop_max, int64_t* d_kept,
    RsGather gather) {
    constexpr int kRsItems = RsTile<K>::kItems;
    constexpr int kRsTile = RsTile<K>::kTile;
    __shared__ uint32_t s_raw[rs_stage_words<K>()];
    __shared__ uint32_t s_part[kRsBins];
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const int64_t tile = blockIdx.x;
    if (d_n && *d_n < n) n = *d_n;
    if (tile * kRsTile >= n) return;   // (uniform: past the keys)
    const int32_t base = (int32_t)(tile * kRsTile);
    const int32_t wbase = base + w * (kRsItems * kWave) + lane;
    const int32_t nn = (int32_t)n;
    K key[kRsItems];
    int32_t val[kRsItems];
    bool valid[kRsItems];
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) {
        const int32_t i = wbase + k * kWave;
        key[k] = i < nn ? kin[i] : (K)0;
        val[k] = i < nn ? vin[i] : 0;
    }
#pragma unroll
    for (int k = 0; k < kRsItems; ++k) valid[k] = wbase + k * kWave < nn && !(drop_max && key[k] == (K)~(K)0);
    uint32_t off_t, total_t;
    rs_group_offsets(cnt, grp, tile, (n + kRsTile - 1) / kRsTile, off_t, total_t, s_part);
    rs_scatter_tile<K>(key, val, valid, tile, n, shift, nbits, off_t, total_t, kout, vout, err,
                       drop_max ? d_kept : nullptr, s_raw, gather);
}

inline int radix_passes(int begin_bit, int end_bit) {
    return end_bit > begin_bit ? (end_bit - begin_bit + 7) / 8 : 0;
}

// Digit width of every pass but possibly the last: the bits spread evenly over the passes
// (14 bits sort as 7 + 7, not 8 + 6), so no pass scatters into more bins than it needs; more
// keys per bin per tile means longer contiguous output runs.
inline int radix_digit_bits(int begin_bit, int end_bit) {
    const int passes = radix_passes(begin_bit, end_bit);
    return passes > 0 ? (end_bit - begin_bit + passes - 1) / passes : 0;
}

template <class K>
inline int64_t radix_tiles(int64_t n) { return ceil_div(n > 0 ? n : 1, RsTile<K>::kTile); }

// The count table inside radix_sort_pairs' scratch, for producers that fill the first
// pass's counts themselves.
inline uint32_t* radix_count_table(void* temp) { return (uint32_t*)temp; }

// The digit totals inside radix_sort_pairs' scratch for n keys (after the count table).
inline uint32_t* radix_totals(void* temp, int64_t n) {
    return (uint32_t*)((char*)temp +
                       align_up((size_t)rs_pitch(ceil_div(n > 0 ? n : 1, kRsMinTile)) * kRsBins * sizeof(uint32_t)));
}

// Scratch for radix_sort_pairs, excluding the ping-pong buffers: the digit-major count
// table (rows padded to a multiple of kXcds tiles), the digit totals and an error word.
// (Sized for the smallest tile, so it serves every key width.)
inline size_t radix_temp_bytes(int64_t n) {
    return align_up((size_t)rs_pitch(ceil_div(n > 0 ? n : 1, kRsMinTile)) * kRsBins * sizeof(uint32_t)) +
           align_up((kRsBins + 64) * 4);
}

// Sort n pairs from (kin, vin) into (kout, vout) on key bits [begin_bit, end_bit).
// (alt_k, alt_v) is the ping-pong buffer. The first pass writes (kout) when the pass count is
// odd and (alt) when it is even, so kin may alias whichever of the two the first pass does
// not write (and it is never written otherwise). first_counts, when not null, is the count
// table of the first pass (256 rows of radix_tiles<K>(n) tiles at rs_entry, from the producer of the
// keys); it is consumed (scanned in place). `err` (device word, may be null) is set nonzero
// if the counts disagree with the keys (the affected keys are not written).
//
// kept_out (device word, may be null) asks for the pairs whose key is all ones to be left
// out: they are not counted or written by the first pass, the later passes sort only the
// kept pairs (their count read on the device, so the host needs no synchronisation), and the
// count of kept pairs is written to *kept_out. The output then holds the kept pairs, stably
// sorted, in its first *kept_out entries.
//
// d_count (device word, may be null; not with kept_out) holds the number of pairs to sort,
// min(*d_count, n): n only sizes the launches, so the host needs no synchronisation.
//
// gather (src may be null): the last pass also writes gather.dst[i] = gather.src[vout[i] - 1]
// for every output i (the values are 1-based indices into src), so per-value data comes out
// in sorted order from one gather instead of one per later reader.
template <class K>
int radix_sort_pairs(const K* kin, K* kout, const int32_t* vin, int32_t* vout, K* alt_k,
                     int32_t* alt_v, int64_t n, int begin_bit, int end_bit, void* temp,
                     size_t temp_bytes, hipStream_t stream, uint32_t* first_counts = nullptr,
                     uint32_t* err = nullptr, int64_t* kept_out = nullptr, const int64_t* d_count = nullptr,
                     RsGather gather = {}) {
    const int passes = radix_passes(begin_bit, end_bit);
    const int width = radix_digit_bits(begin_bit, end_bit);
    if (n <= 0) return TDGS_OK;
    if (n > (int64_t)INT32_MAX) {
        set_error("radix sort of %lld keys exceeds the int32 index range", (long long)n);
        return TDGS_ERR_INVALID;
    }
    if (passes == 0) {
        if (kept_out || d_count || gather.src) {
            set_error("radix sort: dropping keys, a device count or a gather needs at least one pass");
            return TDGS_ERR_INVALID;
        }
        if (kout != kin) TDGS_HIP(hipMemcpyAsync(kout, kin, n * sizeof(K), hipMemcpyDeviceToDevice, stream));
        if (vout != vin) TDGS_HIP(hipMemcpyAsync(vout, vin, n * sizeof(int32_t), hipMemcpyDeviceToDevice, stream));
        return TDGS_OK;
    }
    if (temp_bytes < radix_temp_bytes(n) || temp == nullptr) {
        set_error("radix sort scratch too small (%zu bytes for %lld keys)", temp_bytes, (long long)n);
        return TDGS_ERR_CAPACITY;
    }
    const int64_t tiles = radix_tiles<K>(n);
    uint32_t* counts = (uint32_t*)temp;
    uint32_t* totals = radix_totals(temp, n);
    if (!err) err = totals + kRsBins;
    const K* src_k = kin;
    const int32_t* src_v = vin;
    for (int p = 0; p < passes; ++p) {
        const int shift = begin_bit + width * p;
        const int nbits = end_bit - shift < width ? end_bit - shift : width;
        const bool to_out = ((passes - 1 - p) % 2) == 0;
        K* dk = to_out ? kout : alt_k;
        int32_t* dv = to_out ? vout : alt_v;
        uint32_t* table = counts;
        const int64_t* d_n = kept_out ? (p > 0 ? kept_out : nullptr) : d_count;
        const int drop = (kept_out && p == 0) ? 1 : 0;
        if (p == 0 && first_counts) {
            if (kept_out) {
                set_error("radix sort: dropping keys with producer counts is not supported");
                return TDGS_ERR_INVALID;
            }
            table = first_counts;
        } else {
            k_rs_count<K><<<(unsigned)tiles, kRsThreads, 0, stream>>>(src_k, n, shift, nbits, table, tiles, d_n, drop);
            TDGS_LAUNCHED();
        }
        k_rs_scan_rows<<<kRsBins, 256, 0, stream>>>(table, tiles, totals, d_n, RsTile<K>::kTile);
        TDGS_LAUNCHED();
        k_rs_scatter<K><<<(unsigned)tiles, kRsThreads, 0, stream>>>(src_k, src_v, dk, dv, n, shift, nbits, table,
                                                                     totals, tiles, err, d_n, drop,
                                                                     drop ? kept_out : nullptr,
                                                                     p == passes - 1 ? gather : RsGather{});
        TDGS_LAUNCHED();
        src_k = dk;
        src_v = dv;
    }
    return TDGS_OK;
}

// Words of group sums radix_sort_pairs_grouped needs for n keys sorted on [begin_bit, end_bit).
template <class K>
inline int64_t radix_group_words(int64_t n, int begin_bit, int end_bit) {
    return (int64_t)radix_passes(begin_bit, end_bit) * rs_groups(radix_tiles<K>(n)) * kRsBins;
}

// radix_sort_pairs (same arguments, without first_counts) with the grouped count tables: a
// count and a scatter launch per pass. zgrp holds radix_group_words<K>(n, ...) words that are
// zero on entry (an earlier launch on the stream clears them); they hold the group sums after.
// Sorts of more than kRsMaxGroupedTiles tiles, or with too few words in zgrp, take
// radix_sort_pairs' path (zgrp unused).
template <class K>
int radix_sort_pairs_grouped(const K* kin, K* kout, const int32_t* vin, int32_t* vout, K* alt_k, int32_t* alt_v,
                             int64_t n, int begin_bit, int end_bit, void* temp, size_t temp_bytes, uint32_t* zgrp,
                             int64_t zgrp_words, hipStream_t stream, uint32_t* err = nullptr,
                             int64_t* kept_out = nullptr, const int64_t* d_count = nullptr, RsGather gather = {}) {
    const int passes = radix_passes(begin_bit, end_bit);
    const int width = radix_digit_bits(begin_bit, end_bit);
    const int64_t tiles = radix_tiles<K>(n);
    const int64_t gwords = rs_groups(tiles) * kRsBins;
    if (n <= 0) return TDGS_OK;
    if (passes == 0 || n > (int64_t)INT32_MAX || tiles > kRsMaxGroupedTiles || zgrp == nullptr ||
        zgrp_words < passes * gwords)
        return radix_sort_pairs<K>(kin, kout, vin, vout, alt_k, alt_v, n, begin_bit, end_bit, temp, temp_bytes,
                                   stream, nullptr, err, kept_out, d_count, gather);
    if (temp_bytes < radix_temp_bytes(n) || temp == nullptr) {
        set_error("radix sort scratch too small (%zu bytes for %lld keys)", temp_bytes, (long long)n);
        return TDGS_ERR_CAPACITY;
    }
    uint32_t* cnt = (uint32_t*)temp;   // tiles x kRsBins <= the count table's size
    if (!err) err = radix_totals(temp, n) + kRsBins;
    const K* src_k = kin;
    const int32_t* src_v = vin;
    for (int p = 0; p < passes; ++p) {
        const int shift = begin_bit + width * p;
        const int nbits = end_bit - shift < width ? end_bit - shift : width;
        const bool to_out = ((passes - 1 - p) % 2) == 0;
        K* dk = to_out ? kout : alt_k;
        int32_t* dv = to_out ? vout : alt_v;
        uint32_t* grp = zgrp + p * gwords;
        const int64_t* d_n = kept_out ? (p > 0 ? kept_out : nullptr) : d_count;
        const int drop = (kept_out && p == 0) ? 1 : 0;
        k_rs_count_grouped<K><<<(unsigned)tiles, kRsThreads, 0, stream>>>(src_k, n, shift, nbits, cnt, grp, d_n, drop);
        TDGS_LAUNCHED();
        k_rs_scatter_grouped<K><<<(unsigned)tiles, kRsThreads, 0, stream>>>(
            src_k, src_v, dk, dv, n, shift, nbits, cnt, grp, err, d_n, drop, drop ? kept_out : nullptr,
            p == passes - 1 ? gather : RsGather{});
        TDGS_LAUNCHED();
        src_k = dk;
        src_v = dv;
    }
    return TDGS_OK;
}

}  // namespace tdgs
