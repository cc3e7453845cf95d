// forward.hip — render! on gfx950: cull + compact, projection, key duplication, sort,
// tile ranges and per-tile front-to-back blending.
//
// Reference: src/forward_core.jl:196-993, src/forward_structs.jl:743-757.
//
// Pipeline of tdgs_render with at most 65535 tiles (host counts: one synchronisation, after
// step 5, to learn N_f and M; with TDGS_FLAG_DEVICE_COUNTS none):
//   1. keep flags + kept counts per 256 and 1024 k_keep_counts (also clears the frame's
//                                                 zeroed scratch: group sums, scan tile sums)
//   2-3. compaction + projection, gidx order      k_project (each kept Gaussian's fgidx from
//                                                 its block's offset, summed from the counts,
//                                                 and its rank), also writes N_f and a 32-bit
//                                                 depth key (all ones when its box is empty)
//   4. depth presort: stable sort of (depth bits, k_rs_count_grouped + k_rs_scatter_grouped,
//      fgidx) of the non-empty Gaussians          4 passes; the last gathers the tile
//                                                 rectangles into depth order and sums the
//                                                 count scan's tiles
//   5. tiles and coarse blocks per Gaussian in    k_scan_apply -> M and the coarse offsets
//      depth order, scanned
//   6. coarse emission: one entry per (Gaussian,  k_emit_count (block-id histograms)
//      block of 8 x 8 .. 16 x 16 tiles touched)
//   7. coarse sort: the entries generated again   k_emit_scatter (one radix pass; each entry's
//      and scattered by block id                  tile masks of its block go along)
//   8. tile lists                                 k_bin_tiles<COUNT>, k_bin_scan,
//                                                 k_bin_tiles<WRITE>
//   9. blending                                   k_render_tiles
// With more than 65535 tiles, steps 6-8 are the reference's 64-bit keys emitted in depth order
// (k_emit_depth_order), sorted stably on their tile bits and ranged.
// Why the lists equal CUB's result on the reference's emission order: a Gaussian emits at most
// one key per tile, so the reference's stable sort by (tile, depth bits) orders the keys by
// (tile, depth bits, fgidx). Distributing the Gaussians, sorted by (depth bits, fgidx), to
// coarse blocks and then to tiles, each step keeping their order, yields the same lists
// without sorting the M keys; the 64-bit keys are assembled only on request
// (tdgs_render_sorted_keys).
#include <mutex>

#include "dsort.hpp"
#include "internal.hpp"
#include "scan.hpp"
#include "sort.hpp"

namespace tdgs {

// Scratch of tdgs_scan_counts_noalloc: the per-tile sums of the scan, in a fixed device array
// (one copy per GPU). Host code uses the address hipGetSymbolAddress gives for the current
// device, never the array's name.
constexpr int64_t kNoAllocScanTiles = TDGS_SCAN_NOALLOC_MAX_ITEMS / kScanTile;
static_assert(kNoAllocScanTiles * kScanTile == TDGS_SCAN_NOALLOC_MAX_ITEMS, "whole tiles");
static __device__ __align__(256) int64_t scratch[kNoAllocScanTiles];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static int64_t* g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the current device, looked up once per device.
static int noalloc_scratch(int64_t** out) {
    int dev = -1;
    TDGS_HIP(hipGetDevice(&dev));
    TDGS_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d beyond the %d supported", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        TDGS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        TDGS_REQUIRE(p != nullptr, "no device address for the scan scratch");
        g_scratch_ptr[dev] = static_cast<int64_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    return TDGS_OK;
}

// ------------------------------------------------------------------------------------
// Culling + compaction
// ------------------------------------------------------------------------------------

struct KeepEval {
    const float* mo;
    int kind;
    tdgs_camera cam;
    tdgs_render_options opt;
    uint8_t* keep;             // optional keep flags
    __device__ bool test(int64_t i, float4 m) const {
        const bool k = keep_gaussian(cam, opt, m.x, m.y, m.z, opacity_of(kind, m.w));
        if (keep) keep[i] = k ? 1 : 0;
        return k;
    }
    __device__ int32_t operator()(int64_t i) const {
        return test(i, reinterpret_cast<const float4*>(mo)[i]) ? 1 : 0;
    }
};

struct CompactOut {
    int32_t* fgidx_to_gidx;
    int32_t* keep_cs;
    __device__ void operator()(int64_t i, int64_t incl, int32_t item) const {
        if (keep_cs) keep_cs[i] = (int32_t)incl;
        if (item) fgidx_to_gidx[incl - 1] = (int32_t)(i + 1);
    }
};

__global__ void k_fill_i32(int32_t* p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_fill_keep(KeepEval ev, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) ev(i);
}

// ------------------------------------------------------------------------------------
// Projection (project_fgaussians_kernel!, forward_core.jl:411-517)
// ------------------------------------------------------------------------------------

struct ProjectArgs {
    tdgs_gaussians g;
    tdgs_camera cam;
    tdgs_tiling tiling;
    tdgs_render_options opt;
    const int32_t* block_counts;    // kept Gaussians per 256-Gaussian block
    const int32_t* group_counts;    // kept Gaussians per kKeepSub blocks
    int64_t ngroups;
    int64_t* d_nbf;                 // written by workgroup 0: N_f
    int32_t* fgidx_to_gidx;         // written: the order-preserving compaction
    float* depths;
    float* f2d;
    int32_t* ranges;
    int32_t* counts;
    uint32_t* depth_keys;     // depth bits by fgidx (0xffffffff when empty); culled: slots past N_f
    int32_t* depth_vals;      // fgidx (1-based); 0 for the slots past N_f
    uint32_t* depth_sample;   // or null: the depth presort's sample of the depth keys (ds_sample_store)
};

// Tile ranges from tile rectangles (used when Gaussians cover many tiles, where reading the
// M sorted keys costs more than 4 atomics per Gaussian): each non-empty Gaussian adds its
// rectangle to a 2D difference array, +1 at (x0, y0), -1 at (x1+1, y0) and (x0, y1+1), +1 at
// (x1+1, y1+1) (0-based corners). Workgroup b adds into copy b % kRectCopies, which spreads
// the atomics on popular corners (and, with round-robin dispatch over the 8 XCDs, keeps each
// copy on one XCD); k_merge_rect_diff sums the copies.
constexpr int kRectCopies = 32;
constexpr int64_t kRectKeysPerGaussian = 32;   // use rectangles when M > this x N_f

__global__ __launch_bounds__(256) void k_rect_diff(int64_t nbf, const int32_t* __restrict__ counts,
                                                   const int32_t* __restrict__ ranges, int ntx,
                                                   int32_t* __restrict__ diff, int64_t ndiff) {
    const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= nbf || counts[f] == 0) return;
    const int4 r = reinterpret_cast<const int4*>(ranges)[f];
    const int64_t w = ntx + 1;
    const int x0 = r.x - 1, y0 = r.y - 1, x1 = r.z, y1 = r.w;
    int32_t* d = diff + (int64_t)(blockIdx.x % kRectCopies) * ndiff;
    atomicAdd(d + y0 * w + x0, 1);
    atomicAdd(d + y0 * w + x1, -1);
    atomicAdd(d + y1 * w + x0, -1);
    atomicAdd(d + y1 * w + x1, 1);
}

// Keep counts (fill_keep_gaussians_kernel! and the count half of the compaction scan,
// forward_core.jl:231-244, 326-355): workgroup g evaluates the keep test of Gaussians
// [1024 g, 1024 g + 1024) with coalesced loads and writes the counts of its 4 blocks of 256
// (block_counts) and their sum (group_counts). The projection derives each block's offset
// from these directly, so no scan pass runs in between. (A single pass with a decoupled
// look-back over per-workgroup counts measured slower: the cross-workgroup status round
// trips cost more than this pass.)
constexpr int kKeepSub = 4;
// It also clears zero[0, nzero) (16-byte aligned, nzero a multiple of 4: the frame's zeroed
// scratch) for the sorts and scans that accumulate into it.
__global__ __launch_bounds__(256) void k_keep_counts(KeepEval ev, int64_t n, int32_t* __restrict__ block_counts,
                                                     int32_t* __restrict__ group_counts, int64_t nblocks,
                                                     uint32_t* __restrict__ zero, int64_t nzero) {
    __shared__ int32_t s_cnt[kKeepSub][256 / kWave];
    const int t = threadIdx.x, lane = __lane_id(), wave = t / kWave;
    for (int64_t k = (int64_t)blockIdx.x * 256 + t; k < nzero / 4; k += (int64_t)gridDim.x * 256)
        reinterpret_cast<uint4*>(zero)[k] = make_uint4(0u, 0u, 0u, 0u);
    float4 mv[kKeepSub];   // all loads in flight before any test
#pragma unroll
    for (int k = 0; k < kKeepSub; ++k) {
        const int64_t i = ((int64_t)blockIdx.x * kKeepSub + k) * 256 + t;
        mv[k] = i < n ? reinterpret_cast<const float4*>(ev.mo)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    bool kp[kKeepSub];
#pragma unroll
    for (int k = 0; k < kKeepSub; ++k) {
        const int64_t i = ((int64_t)blockIdx.x * kKeepSub + k) * 256 + t;
        kp[k] = i < n && ev.test(i, mv[k]);
    }
#pragma unroll
    for (int k = 0; k < kKeepSub; ++k) {
        const uint64_t bal = __ballot(kp[k]);
        if (lane == 0) s_cnt[k][wave] = __popcll(bal);
    }
    __syncthreads();
    if (t < kKeepSub) {
        const int64_t sb = (int64_t)blockIdx.x * kKeepSub + t;
        int32_t c = 0;
        for (int w = 0; w < 256 / kWave; ++w) c += s_cnt[t][w];
        if (sb < nblocks) block_counts[sb] = c;
    }
    if (t == 0) {
        int32_t c = 0;
        for (int k = 0; k < kKeepSub; ++k)
            for (int w = 0; w < 256 / kWave; ++w) c += s_cnt[k][w];
        group_counts[blockIdx.x] = c;
    }
}

// Compaction + projection (fill_fgidx_to_gidx_kernel! and project_fgaussians_kernel!,
// forward_core.jl:371-386, 411-517), one thread per Gaussian in gidx order: the keep test is
// repeated, and a kept Gaussian's fgidx is its block's offset plus its rank among the block's
// kept Gaussians (wave ballots), so parameter reads are coalesced and the compaction costs no
// pass of its own. All parameter loads issue at once; a non-empty Gaussian's 48 SH
// coefficients (12 float4 for 16-coefficient storage) are loaded by its own thread and its
// colour evaluated before the workgroup barrier that resolves the ranks. (Staging the SH
// blocks through LDS for coalescing measured slower once the loads overlap like this.)
constexpr int kProjThreads = 256;
constexpr int kGroupLoads = 4;   // group counts per thread per round

template <int KIND>
__global__ __launch_bounds__(kProjThreads) void k_project(ProjectArgs a) {
    __shared__ int32_t s_wave[kProjThreads / kWave];
    __shared__ int64_t s_red[2][kProjThreads / kWave];
    __shared__ float s_rec[kProjThreads * 9];   // the block's f2d records, by rank
    const int t = threadIdx.x, lane = __lane_id(), wave = t / kWave;
    const int64_t gi = (int64_t)blockIdx.x * kProjThreads + t;
    const int64_t n = a.g.n;
    // all parameter loads issue together, without branches (the culled few percent are read
    // for nothing; threads past n read the last Gaussian and are not kept)
    const int64_t gl = gi < n ? gi : n - 1;
    const float4 m = reinterpret_cast<const float4*>(a.g.means_opacity)[gl];
    float params[7];
    if constexpr (KIND == TDGS_TRAINABLE) {
        params[0] = a.g.scaling[3 * gl];
        params[1] = a.g.scaling[3 * gl + 1];
        params[2] = a.g.scaling[3 * gl + 2];
        const float4 q = reinterpret_cast<const float4*>(a.g.rotation)[gl];
        params[3] = q.x; params[4] = q.y; params[5] = q.z; params[6] = q.w;
    } else {
#pragma unroll
        for (int k = 0; k < 6; ++k) params[k] = a.g.covariances[6 * gl + k];
    }
    // this block's offset (kept Gaussians in earlier groups, then in earlier blocks of its
    // group) and N_f, summed from the group counts (a few KB, read from L2 by every block;
    // the loads of one round are all in flight together)
    {
        const int64_t grp = blockIdx.x / kKeepSub;
        int64_t before = 0, total = 0;
        for (int64_t k0 = 0; k0 < a.ngroups; k0 += kGroupLoads * kProjThreads) {
            int32_t c[kGroupLoads];
#pragma unroll
            for (int u = 0; u < kGroupLoads; ++u) {
                const int64_t k = k0 + u * kProjThreads + t;
                c[u] = a.group_counts[k < a.ngroups ? k : a.ngroups - 1];   // clamped: no branch
            }
#pragma unroll
            for (int u = 0; u < kGroupLoads; ++u) {
                const int64_t k = k0 + u * kProjThreads + t;
                const int32_t cu = k < a.ngroups ? c[u] : 0;
                total += cu;
                if (k < grp) before += cu;
            }
        }
        const int32_t bc = a.block_counts[grp * kKeepSub + (t & (kKeepSub - 1))];
        if (t < (int)(blockIdx.x - grp * kKeepSub)) before += bc;
#pragma unroll
        for (int d = kWave / 2; d > 0; d >>= 1) {
            before += __shfl_xor(before, d, kWave);
            total += __shfl_xor(total, d, kWave);
        }
        if (lane == 0) { s_red[0][wave] = before; s_red[1][wave] = total; }
    }
    const float op = opacity_of(KIND, m.w);
    const bool keep = gi < n && keep_gaussian(a.cam, a.opt, m.x, m.y, m.z, op);
    const uint64_t bal = __ballot(keep);
    if (lane == 0) s_wave[wave] = __popcll(bal);
    Projected pr;
    pr.count = 0;
    if (keep) pr = project_geometry(a.cam, a.opt, a.tiling, KIND, m.x, m.y, m.z, op, params);
    float rgb[3];
    if (pr.count > 0) {
        const int hs = (a.g.sh_degree + 1) * (a.g.sh_degree + 1);
        float bs[16];
        if (hs == 16) {
            const float4* p = reinterpret_cast<const float4*>(a.g.sh) + (int64_t)12 * gi;
            float cc[48];
#pragma unroll
            for (int r = 0; r < 12; ++r) {
                const float4 v = p[r];
                cc[4 * r] = v.x; cc[4 * r + 1] = v.y; cc[4 * r + 2] = v.z; cc[4 * r + 3] = v.w;
            }
            view_sh_basis(a.cam, a.opt.sh_degree, m.x, m.y, m.z, bs);
#pragma unroll
            for (int c = 0; c < 3; ++c) rgb[c] = sh_channel_to_color(a.opt.sh_degree, cc + 16 * c, bs);
        } else {
            view_sh_basis(a.cam, a.opt.sh_degree, m.x, m.y, m.z, bs);
            sh_to_color(a.opt.sh_degree, a.g.sh + 3 * (int64_t)hs * gi, hs, bs, rgb);
        }
    }
    __syncthreads();
    int before = 0, kept = 0;
#pragma unroll
    for (int w = 0; w < kProjThreads / kWave; ++w) {
        if (w < wave) before += s_wave[w];
        kept += s_wave[w];
    }
    const int local = before + __popcll(bal & lanemask_lt());
    int64_t off = 0, nbf = 0;
#pragma unroll
    for (int w = 0; w < kProjThreads / kWave; ++w) {
        off += s_red[0][w];
        nbf += s_red[1][w];
    }
    if (blockIdx.x == 0 && t == 0) *a.d_nbf = nbf;
    const int64_t f = off + local;   // 0-based fgidx if kept
    if (keep) {
        a.fgidx_to_gidx[f] = (int32_t)(gi + 1);
        a.counts[f] = pr.count;
        uint32_t dk = 0xffffffffu;
        float* r = s_rec + 9 * local;   // empty Gaussians get a zero record
        if (pr.count > 0) {
            a.depths[f] = pr.depth;
            reinterpret_cast<int4*>(a.ranges)[f] = make_int4(pr.rect[0], pr.rect[1], pr.rect[2], pr.rect[3]);
            r[0] = pr.mux; r[1] = pr.muy; r[2] = pr.a;
            r[3] = pr.m11; r[4] = pr.m21; r[5] = pr.m22;
            r[6] = rgb[0]; r[7] = rgb[1]; r[8] = rgb[2];
            dk = float_bits(pr.depth);
        } else {
#pragma unroll
            for (int k = 0; k < 9; ++k) r[k] = 0.0f;
        }
        if (a.depth_keys) {
            a.depth_keys[f] = dk;
            a.depth_vals[f] = (int32_t)(f + 1);
            if (a.depth_sample) ds_sample_store(a.depth_sample, n, f, dk);
        }
    } else if (gi < n && a.depth_keys) {
        const int64_t slot = nbf + (gi - f);   // culled Gaussians fill the slots past N_f
        a.depth_keys[slot] = 0xffffffffu;
        a.depth_vals[slot] = 0;
        if (a.depth_sample) ds_sample_store(a.depth_sample, n, slot, 0xffffffffu);
    }
    // the block's records are one contiguous run of f2d: write it with consecutive lanes on
    // consecutive floats (36-byte strided stores from each thread split into many partial
    // requests)
    __syncthreads();
    float* dst = a.f2d + 9 * off;
    const int total = 9 * kept;
    const int head = (int)((4 - ((9 * off) & 3)) & 3);   // floats before the first 16-byte boundary
    if (t < head && t < total) dst[t] = s_rec[t];
    const int quads = total > head ? (total - head) >> 2 : 0;
    for (int q = t; q < quads; q += kProjThreads) {
        const int e = head + 4 * q;
        *reinterpret_cast<float4*>(dst + e) = make_float4(s_rec[e], s_rec[e + 1], s_rec[e + 2], s_rec[e + 3]);
    }
    const int tail = head + 4 * quads;
    if (tail + t < total) dst[tail + t] = s_rec[tail + t];
}

// ------------------------------------------------------------------------------------
// Key duplication
// ------------------------------------------------------------------------------------

// Overlap counts of the non-empty Gaussians in depth order (entries past N_b count 0): the
// areas of their tile rectangles, which the depth sort's last pass gathered into depth order
// (srect: contiguous reads here instead of a gather per reader).
__device__ __forceinline__ int32_t rect_area(const int4 r) { return (r.z - r.x + 1) * (r.w - r.y + 1); }
struct SortedCounts {
    const int4* srect;
    const int64_t* d_nb;
    __device__ int32_t operator()(int64_t j) const { return j < *d_nb ? rect_area(srect[j]) : 0; }
};

// The inclusive scan of the tile counts in depth order, and for every emission block (keys
// [b kEmitTile, (b + 1) kEmitTile)) the Gaussian that owns its first key: the one whose keys
// [incl - count, incl) contain b kEmitTile.
struct WriteScanAndBlocks {
    int32_t* cs;
    int32_t* blk_first;
    int64_t nblk;   // entries of blk_first (blocks past it, for keys beyond the key capacity, are not recorded)
    __device__ void operator()(int64_t j, int64_t incl, int32_t count) const;
};

// Key emission in depth order. Each workgroup owns kEmitTile consecutive keys; the count scan
// recorded the Gaussian (depth order) that owns the first key of every block, which bounds
// the span of Gaussians producing them, and the workgroup stages their scan values in LDS.
// Thread t then produces the kEmitItems consecutive keys d0 + kEmitItems t, ...: one binary
// search in LDS for the first, then a walk that moves to the next Gaussian when the key
// passes its end and steps the tile (x fastest) without a division. Within a Gaussian, key
// number `local` is tile (x0 + local % wx, y0 + local / wx): tiles row-major, x fastest, as
// the reference emits them (forward_core.jl:577-597). The keys go through LDS (a rotated
// layout without bank conflicts) to fully coalesced stores.
constexpr int kEmitThreads = 256;
constexpr int kEmitItems = 16;
constexpr int kEmitTile = kEmitThreads * kEmitItems;
static_assert((kKeepSub & (kKeepSub - 1)) == 0, "power of two");
static_assert(kEmitTile == RsTile<uint64_t>::kTile && kEmitTile == RsTile<uint16_t>::kTile,
              "one emission workgroup fills one radix count tile");

__device__ void WriteScanAndBlocks::operator()(int64_t j, int64_t incl, int32_t count) const {
    cs[j] = (int32_t)incl;
    for (int64_t b = (incl - count + kEmitTile - 1) / kEmitTile; b * kEmitTile < incl && b < nblk; ++b)
        blk_first[b] = (int32_t)j;
}

// sorted_f holds the nb non-empty Gaussians in depth order and cs the inclusive scan of
// their tile counts. The kernel also counts the digit of the first tile-sort pass (the low
// nbits0 bits of the tile id) of its keys, which form one radix count tile:
// counts0[d][blockIdx.x]. TILE16 writes only the tile id of each key (uint16_t): the keys
// already are in depth order, so the stable sort by tile needs no depth bits, and the full
// keys are assembled on request (k_assemble_keys).
//
// When the block's keys come from at most kEmitStage Gaussians, their fgidx, first tile id
// and rectangle width are staged in LDS too (in the part of the scan buffer that a span of
// that size leaves free); otherwise the walk reads them from global memory.
constexpr int kEmitStage = 1024;

// The grid the emission walks: the tiles (sx = sy = 0), or the coarse blocks of 2^sx x 2^sy
// tiles (ntx blocks per row); a Gaussian's rectangle of tiles covers the rectangle of blocks
// from the block of its first tile to the block of its last.
struct EmitGrid {
    int32_t ntx, sx, sy;
    __device__ __forceinline__ void rect(const int4 r, int32_t* t0, int32_t* wx) const {
        const int32_t x0 = (r.x - 1) >> sx, y0 = (r.y - 1) >> sy, x1 = (r.z - 1) >> sx;
        *t0 = x0 + 1 + y0 * ntx;
        *wx = x1 - x0 + 1;
    }
    // rect() with, for the blocks' tile masks (at most 255 blocks, blocks of at most 16 x 16
    // tiles), the rectangle's first and last tile column inside its first and last block
    // column, the same for rows, and its block rows less one, packed with the width:
    // wx | ox0 << 8 | ox1 << 12 | oy0 << 16 | oy1 << 20 | (rows - 1) << 24
    __device__ __forceinline__ void rect_packed(const int4 r, int32_t* t0, int32_t* pk) const {
        const int32_t x0 = (r.x - 1) >> sx, y0 = (r.y - 1) >> sy, x1 = (r.z - 1) >> sx, y1 = (r.w - 1) >> sy;
        const int32_t bwm = (1 << sx) - 1, bhm = (1 << sy) - 1;
        *t0 = x0 + 1 + y0 * ntx;
        *pk = (x1 - x0 + 1) | (((r.x - 1) & bwm) << 8) | (((r.z - 1) & bwm) << 12) | (((r.y - 1) & bhm) << 16) |
              (((r.w - 1) & bhm) << 20) | ((y1 - y0) << 24);
    }
    // The tiles of block (column rx, row q of the rectangle's blocks) that the rectangle
    // covers, as bit masks relative to the block: columns in bits 0-15, rows in bits 16-31.
    __device__ __forceinline__ uint32_t block_mask(int32_t pk, int32_t q, int32_t rx) const {
        const int32_t bwm = (1 << sx) - 1, bhm = (1 << sy) - 1;
        const int32_t cx0 = rx == 0 ? (pk >> 8) & 15 : 0;
        const int32_t cx1 = rx == (pk & 0xff) - 1 ? (pk >> 12) & 15 : bwm;
        const int32_t cy0 = q == 0 ? (pk >> 16) & 15 : 0;
        const int32_t cy1 = q == ((pk >> 24) & 0xff) ? (pk >> 20) & 15 : bhm;
        return ((2u << cx1) - (1u << cx0)) | (((2u << cy1) - (1u << cy0)) << 16);
    }
};
static_assert(kEmitStage + 1 + 3 * kEmitStage <= kEmitTile + 1, "staging fits the scan buffer");

// Slot of key k (0 <= k < kEmitTile) of the block in the LDS transpose: thread k / kEmitItems
// writes its item k % kEmitItems rotated by the thread index, so that the 64 lanes of a
// wavefront writing item i, and the 64 lanes reading consecutive keys, spread over the banks.
__device__ __forceinline__ int emit_slot(int k) {
    const int t = k / kEmitItems, i = k % kEmitItems;
    return t * kEmitItems + ((i + t) & (kEmitItems - 1));
}

// The tile ids and values of keys d0 + ITEMS t + i (i < ITEMS) of emission block `block`
// (d0 = block THREADS ITEMS), computed by thread t of a THREADS-thread workgroup into
// tile[] and val[] (zeros past m); with MASK (a coarse grid of at most 255 blocks) also
// mask[]: the tiles of the entry's block that its rectangle covers (EmitGrid::block_mask).
// s_buf holds THREADS ITEMS + 1 ints of LDS; ends with a workgroup barrier after its last use
// of s_buf and s_range.
template <int THREADS, int ITEMS, bool MASK = false>
__device__ __forceinline__ void emit_generate(int64_t nb, int64_t m, int64_t block, const int32_t* __restrict__ sorted_f,
                                              const int32_t* __restrict__ cs, const int32_t* __restrict__ blk_first,
                                              const int4* __restrict__ srect, EmitGrid grid, int32_t* s_buf,
                                              int64_t* s_range, int32_t (&tile)[ITEMS], int32_t (&val)[ITEMS],
                                              uint32_t* mask = nullptr) {
    constexpr int kBlock = THREADS * ITEMS;
    static_assert(kBlock == kEmitTile, "emission blocks of kEmitTile keys");
    int32_t* const s_cs = s_buf;                      // [0, cnt]: scan values of the span
    int32_t* const s_f = s_buf + kEmitStage + 1;      // staged Gaussians: fgidx,
    int32_t* const s_t0 = s_f + kEmitStage;           // tile id of the rectangle's first tile,
    int32_t* const s_wx = s_t0 + kEmitStage;          // rectangle width in tiles (MASK: packed)
    const int t = threadIdx.x;
    const int64_t d0 = block * kBlock;
    // Gaussians owning the block's first and last keys: from the block table of the count scan
    // (the next block's first Gaussian, or the one before it when that one starts exactly at
    // the next block), clamped to [0, nb)
    if (t == 0) s_range[0] = blk_first[block];
    if (t == 1) {
        const int64_t dn = d0 + kBlock;
        int64_t jh = nb - 1;
        if (dn < m) {
            const int64_t jn = blk_first[block + 1];
            const int64_t sn = jn <= 0 ? 0 : cs[jn - 1];
            jh = sn < dn ? jn : jn - 1;
        }
        s_range[1] = jh;
    }
    __syncthreads();
    int64_t j_lo = s_range[0];
    int64_t j_hi = s_range[1];
    if (j_hi > nb - 1) j_hi = nb - 1;
    if (j_lo < 0) j_lo = 0;
    if (j_lo > j_hi) j_lo = j_hi;
    const int64_t cnt = j_hi - j_lo + 1;  // Gaussians spanned (each owns >= 1 key here)
    const bool staged = cnt <= kBlock;    // always, with consistent counts
    const bool full = cnt <= kEmitStage;
    if (staged) {
        for (int64_t k = t; k <= cnt; k += THREADS) {
            const int64_t j = j_lo + k - 1;
            s_cs[k] = j < 0 ? 0 : cs[j];
            if (full && k < cnt) {
                s_f[k] = sorted_f[j + 1];
                if (MASK)
                    grid.rect_packed(srect[j + 1], &s_t0[k], &s_wx[k]);
                else
                    grid.rect(srect[j + 1], &s_t0[k], &s_wx[k]);
            }
        }
    }
    __syncthreads();
    // scan value before span entry k (k <= cnt): the first key of Gaussian j_lo + k
    auto start_of = [&](int64_t k) -> int64_t {
        if (staged) return s_cs[k];
        const int64_t j = j_lo + k - 1;
        return j < 0 ? 0 : cs[j];
    };
    const int64_t first = d0 + (int64_t)t * ITEMS;
    if (first < m) {
        int64_t lo = 0, hi = cnt;   // largest k in [0, cnt) with start_of(k) <= first
        while (hi - lo > 1) {
            const int64_t mid = (lo + hi) >> 1;
            if (start_of(mid) <= first) lo = mid; else hi = mid;
        }
        int64_t nxt = start_of(lo + 1);
        int32_t f, t0, wx, pk = 0;
        auto load = [&](int64_t k) {
            if (full) {
                f = s_f[k]; t0 = s_t0[k]; wx = s_wx[k];
            } else {
                f = sorted_f[j_lo + k];
                if (MASK)
                    grid.rect_packed(srect[j_lo + k], &t0, &wx);
                else
                    grid.rect(srect[j_lo + k], &t0, &wx);
            }
            if (MASK) {
                pk = wx;
                wx &= 0xff;
            }
        };
        load(lo);
        const int32_t local = (int32_t)(first - start_of(lo));
        int32_t q = local / wx, rx = local - q * wx;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            const int64_t d = first + i;
            if (d >= nxt && lo + 1 < cnt) {   // next Gaussian (each owns >= 1 key)
                ++lo;
                nxt = start_of(lo + 1);
                load(lo);
                q = 0;
                rx = 0;
            }
            tile[i] = t0 + q * grid.ntx + rx;
            val[i] = f;
            if (MASK) mask[i] = grid.block_mask(pk, q, rx);
            if (++rx == wx) {
                rx = 0;
                ++q;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            tile[i] = val[i] = 0;
            if (MASK) mask[i] = 0;
        }
    }
    __syncthreads();   // s_buf is free again
}

template <bool TILE16>
__global__ __launch_bounds__(kEmitThreads) void k_emit_depth_order(
    int64_t nb, int64_t m, const int32_t* __restrict__ sorted_f, const int32_t* __restrict__ cs,
    const int32_t* __restrict__ blk_first, const float* __restrict__ depths, const int4* __restrict__ srect,
    EmitGrid grid, void* __restrict__ keys_out, int32_t* __restrict__ vals, int nbits0,
    uint32_t* __restrict__ counts0, int64_t count_tiles) {
    __shared__ int32_t s_buf[kEmitTile + 1];
    __shared__ int64_t s_range[2];
    __shared__ uint32_t s_h[kRsBins];
    const int t = threadIdx.x;
    s_h[t] = 0;
    const int64_t d0 = (int64_t)blockIdx.x * kEmitTile;
    int32_t tile[kEmitItems], val[kEmitItems];
    emit_generate<kEmitThreads, kEmitItems>(nb, m, blockIdx.x, sorted_f, cs, blk_first, srect, grid, s_buf, s_range,
                                            tile, val);
    // values, then tile ids (or keys), through LDS to coalesced stores
    const int64_t nk = m - d0 < kEmitTile ? m - d0 : kEmitTile;
    const uint32_t mask0 = (1u << nbits0) - 1u;
#pragma unroll
    for (int i = 0; i < kEmitItems; ++i) s_buf[t * kEmitItems + ((i + t) & (kEmitItems - 1))] = val[i];
    __syncthreads();
    int32_t fv[kEmitItems];   // the value of key t + kEmitThreads i (the 64-bit keys need it)
#pragma unroll
    for (int i = 0; i < kEmitItems; ++i) {
        const int k = t + kEmitThreads * i;
        fv[i] = s_buf[emit_slot(k)];
        if (k < nk) vals[d0 + k] = fv[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kEmitItems; ++i) s_buf[t * kEmitItems + ((i + t) & (kEmitItems - 1))] = tile[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kEmitItems; ++i) {
        const int k = t + kEmitThreads * i;
        if (k < nk) {
            const int32_t tl = s_buf[emit_slot(k)];
            if (TILE16)
                static_cast<uint16_t*>(keys_out)[d0 + k] = (uint16_t)tl;
            else
                static_cast<int64_t*>(keys_out)[d0 + k] = ((int64_t)tl << 32) |
                                                          (int64_t)float_bits(depths[fv[i] - 1]);
            atomicAdd(&s_h[(uint32_t)tl & mask0], 1u);
        }
    }
    __syncthreads();
    counts0[rs_entry(t, blockIdx.x, count_tiles)] = s_h[t];
}

// The 16-bit tile sort's first pass fused with key emission: emission blocks are radix tiles
// (kEmitTile keys), generated twice instead of written and read back.
//   k_emit_count:   the first-pass digit (low nbits0 bits of the block id) histogram of each
//                   block's keys: with group sums (grp), one row counts0[block][d] added into
//                   its group's sums, from which every scatter workgroup takes its offsets;
//                   else counts0[d][block] for k_rs_scan_rows;
//   k_emit_scatter: the keys again, moved through LDS into the radix tile layout (wavefront
//                   w, item k, lane l <-> key w 512 + k 64 + l), then rs_scatter_tile writes
//                   tile ids and values straight to their first-pass sorted positions.
constexpr int kEmitSortThreads = kRsThreads;
constexpr int kEmitSortItems = kEmitTile / kEmitSortThreads;
static_assert(kEmitSortItems == RsTile<uint16_t>::kItems, "radix tile layout");

template <bool LOOP>
__global__ __launch_bounds__(kEmitSortThreads) void k_emit_count(int64_t nb, int64_t m,
                                                                 const int32_t* __restrict__ sorted_f,
                                                                 const int32_t* __restrict__ cs,
                                                                 const int32_t* __restrict__ blk_first,
                                                                 const int4* __restrict__ srect, EmitGrid grid,
                                                                 int nbits0, uint32_t* __restrict__ counts0,
                                                                 int64_t count_tiles, uint32_t* __restrict__ grp,
                                                                 int64_t* dc, int64_t key_cap, int32_t* zero,
                                                                 int64_t nzero) {
    __shared__ int32_t s_buf[kEmitTile + 1];
    __shared__ int64_t s_range[2];
    __shared__ uint32_t s_h[kRsBins];
    const int t = threadIdx.x;
    // (also clears zero[0, nzero) for the binning that follows)
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + t; k < nzero; k += (int64_t)gridDim.x * blockDim.x) zero[k] = 0;
    if (dc) {
        // device counts: the grid covers key_cap entries; when the M keys fit the key arrays the
        // passes emit the blocks' entries (at most M), else none (the status says why)
        nb = dc[4];
        const int64_t packed = dc[kCntCoarse];   // (M << 32) | coarse entries, from the scan
        const int64_t keys = packed >> 32;
        const int64_t st = keys > key_cap ? kFrameKeyCapacity : keys >= (int64_t)INT32_MAX ? kFrameKeyRange : kFrameOk;
        m = st == kFrameOk ? (packed & kLow32) : 0;
        if (blockIdx.x == 0 && t == 0) {
            dc[1] = keys;
            dc[kCntKeysUsed] = st == kFrameOk ? keys : 0;
            dc[kCntCoarseUsed] = m;
            dc[kCntStatus] = st;
        }
    }
    // emission blocks blockIdx.x, + gridDim.x, ... (LOOP: a grid capped below the
    // capacity-sized block count of a device-count render; else one block per workgroup); the
    // count columns of the blocks past the entries are left alone (the row scan reads the used
    // ones only)
    const uint32_t mask0 = (1u << nbits0) - 1u;
    for (int64_t blk = blockIdx.x; blk * kEmitTile < m; blk += LOOP ? gridDim.x : m) {
        if (t < kRsBins) s_h[t] = 0;
        int32_t tile[kEmitSortItems], val[kEmitSortItems];
        emit_generate<kEmitSortThreads, kEmitSortItems>(nb, m, blk, sorted_f, cs, blk_first, srect, grid, s_buf,
                                                        s_range, tile, val);
        const int64_t first = blk * kEmitTile + (int64_t)t * kEmitSortItems;
#pragma unroll
        for (int i = 0; i < kEmitSortItems; ++i)
            if (first + i < m) atomicAdd(&s_h[(uint32_t)tile[i] & mask0], 1u);
        __syncthreads();
        if (t < kRsBins) {
            const uint32_t c = s_h[t];
            if (grp) {   // grouped tables: the block's row, added into its group's sums
                counts0[blk * kRsBins + t] = c;
                if (c) atomicAdd(&grp[(blk / kRsGroup) * kRsBins + t], c);
            } else {
                counts0[rs_entry(t, blk, count_tiles)] = c;
            }
        }
        __syncthreads();   // s_h and s_buf are reused by the next block
    }
}

// Slot of key k of the block in k_emit_scatter's transpose (thread k / 8 writes item k % 8,
// rotated by the thread index so that neither the writes nor the radix-layout reads of a
// wavefront meet in one bank).
__device__ __forceinline__ int emit_sort_slot(int k) {
    const int t = k / kEmitSortItems, i = k % kEmitSortItems;
    return t * kEmitSortItems + ((i + t) & (kEmitSortItems - 1));
}

// One emission block of k_emit_scatter (MASK: each entry's block mask goes along to mout).
template <bool MASK>
__device__ __forceinline__ void emit_scatter_block(int64_t blk, int64_t nb, int64_t m, const int32_t* __restrict__ sorted_f,
                                                   const int32_t* __restrict__ cs, const int32_t* __restrict__ blk_first,
                                                   const int4* __restrict__ srect, EmitGrid grid, int nbits0,
                                                   const uint32_t* __restrict__ offsets,
                                                   uint32_t* __restrict__ totals, int64_t count_tiles,
                                                   const uint32_t* __restrict__ grp, uint16_t* __restrict__ kout,
                                                   int32_t* __restrict__ vout, uint32_t* __restrict__ mout,
                                                   uint32_t* err, int32_t* s_buf, int64_t* s_range, uint32_t* s_part) {
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const int64_t d0 = blk * kEmitTile;
    int32_t tile[kEmitSortItems], val[kEmitSortItems];
    uint32_t msk[kEmitSortItems];
    emit_generate<kEmitSortThreads, kEmitSortItems, MASK>(nb, m, blk, sorted_f, cs, blk_first, srect, grid, s_buf,
                                                          s_range, tile, val, MASK ? msk : nullptr);
    uint16_t key[kEmitSortItems];
    int32_t v[kEmitSortItems];
    uint32_t mv[kEmitSortItems];
    bool valid[kEmitSortItems];
#pragma unroll
    for (int i = 0; i < kEmitSortItems; ++i) s_buf[t * kEmitSortItems + ((i + t) & (kEmitSortItems - 1))] = tile[i];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kEmitSortItems; ++k) {
        const int q = w * (kEmitSortItems * kWave) + k * kWave + lane;
        key[k] = (uint16_t)s_buf[emit_sort_slot(q)];
        valid[k] = d0 + q < m;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kEmitSortItems; ++i) s_buf[t * kEmitSortItems + ((i + t) & (kEmitSortItems - 1))] = val[i];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kEmitSortItems; ++k) v[k] = s_buf[emit_sort_slot(w * (kEmitSortItems * kWave) + k * kWave + lane)];
    if (MASK) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kEmitSortItems; ++i)
            s_buf[t * kEmitSortItems + ((i + t) & (kEmitSortItems - 1))] = (int32_t)msk[i];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kEmitSortItems; ++k)
            mv[k] = (uint32_t)s_buf[emit_sort_slot(w * (kEmitSortItems * kWave) + k * kWave + lane)];
    }
    uint32_t off_t = 0, total_t = 0;
    if (grp) {
        rs_group_offsets(offsets, grp, blk, (m + kEmitTile - 1) / kEmitTile, off_t, total_t, s_part);
        if (blk == 0 && t < kRsBins) totals[t] = total_t;   // (the binning's block ends)
    } else if (t < kRsBins) {
        off_t = offsets[rs_entry(t, blk, count_tiles)];
        total_t = totals[t];
    }
    // (rs_scatter_tile reuses s_buf for its staging after its first barrier)
    rs_scatter_tile<uint16_t, MASK>(key, v, valid, blk, m, 0, nbits0, off_t, total_t, kout, vout, err, nullptr,
                                    reinterpret_cast<uint32_t*>(s_buf), RsGather{}, MASK ? mv : nullptr, mout);
}

// LOOP: a capped grid walks the emission blocks blockIdx.x, + gridDim.x, ... (a device-count
// render whose capacity-sized block count exceeds the cap; the loop costs registers: 134
// VGPRs against 73, so the grid is one block per workgroup otherwise).
// MASK: the entries' block masks are sorted along into mout (one radix pass only).
template <bool LOOP, bool MASK>
__global__ __launch_bounds__(kEmitSortThreads) void k_emit_scatter(
    int64_t nb, int64_t m, const int32_t* __restrict__ sorted_f, const int32_t* __restrict__ cs,
    const int32_t* __restrict__ blk_first, const int4* __restrict__ srect, EmitGrid grid, int nbits0,
    const uint32_t* __restrict__ offsets, uint32_t* __restrict__ totals, int64_t count_tiles,
    const uint32_t* __restrict__ grp, uint16_t* __restrict__ kout, int32_t* __restrict__ vout,
    uint32_t* __restrict__ mout, uint32_t* err, const int64_t* dc) {
    __shared__ int32_t s_buf[kEmitTile + 1];
    __shared__ int64_t s_range[2];
    __shared__ uint32_t s_part[kRsBins];
    if (dc) {   // device counts (k_emit_count set the entry count used)
        nb = dc[4];
        m = dc[kCntCoarseUsed];
    }
    // no entries: the digit totals are zero (with group sums nothing else writes them)
    if (grp && m == 0 && blockIdx.x == 0 && threadIdx.x < kRsBins) totals[threadIdx.x] = 0;
    if (!LOOP) {
        if ((int64_t)blockIdx.x * kEmitTile < m)
            emit_scatter_block<MASK>(blockIdx.x, nb, m, sorted_f, cs, blk_first, srect, grid, nbits0, offsets, totals,
                                     count_tiles, grp, kout, vout, mout, err, s_buf, s_range, s_part);
        return;
    }
    for (int64_t blk = blockIdx.x; blk * kEmitTile < m; blk += gridDim.x) {
        emit_scatter_block<MASK>(blk, nb, m, sorted_f, cs, blk_first, srect, grid, nbits0, offsets, totals, count_tiles,
                                 grp, kout, vout, mout, err, s_buf, s_range, s_part);
        __syncthreads();   // s_buf is reused by the next block
    }
}

// fill_df2dgs_codes_and_dfgidx_to_fgidx_kernel! (forward_core.jl:531-603): reference
// emission order (ascending fgidx).
__global__ __launch_bounds__(256) void k_emit_keys(int64_t nbf, const float* __restrict__ depths,
                                                   const int32_t* __restrict__ ranges,
                                                   const int32_t* __restrict__ cs, int32_t ntx,
                                                   int64_t* __restrict__ keys,
                                                   int32_t* __restrict__ vals) {
    const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= nbf) return;
    const int64_t end = cs[f];
    int64_t d = f == 0 ? 0 : cs[f - 1];
    if (d >= end) return;
    const int4 r = reinterpret_cast<const int4*>(ranges)[f];
    const float depth = depths[f];
    for (int32_t ty = r.y; ty <= r.w; ++ty) {
        for (int32_t tx = r.x; tx <= r.z; ++tx) {
            if (d >= end) return;
            keys[d] = make_key(tx + (ty - 1) * ntx, depth);
            vals[d] = (int32_t)(f + 1);
            ++d;
        }
    }
}

// Tile id of sorted entry i: the high word of a 64-bit key, or a 16-bit tile id.
__device__ __forceinline__ int32_t tile_of(const int64_t* sk, int64_t i) { return (int32_t)(sk[i] >> 32); }
__device__ __forceinline__ int32_t tile_of(const uint16_t* st, int64_t i) { return st[i]; }

// fill_tiles_end_sdfgidx_kernel! (forward_core.jl:676-734). Tile ids are clamped to
// [1, nb_tiles] so that a malformed key cannot write out of bounds.
template <class K>
__global__ __launch_bounds__(256) void k_tile_ranges(int64_t m, const K* __restrict__ sk, int32_t nb_tiles,
                                                     int32_t* __restrict__ te, const int64_t* dm = nullptr) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (dm) {   // device key count (the grid covers the key capacity); no keys: empty tiles
        m = *dm;
        if (m == 0)
            for (int64_t k = i; k < nb_tiles; k += (int64_t)gridDim.x * blockDim.x) te[k] = 0;
    }
    if (i >= m) return;
    const int32_t cur = tile_of(sk, i);
    if (i == 0) {
        const int32_t stop = cur < nb_tiles + 1 ? cur : nb_tiles + 1;
        for (int32_t t = 1; t < stop; ++t) te[t - 1] = 0;
    }
    int32_t lo = cur < 1 ? 1 : cur;
    if (i + 1 < m) {
        int32_t nxt = tile_of(sk, i + 1);
        if (nxt > nb_tiles + 1) nxt = nb_tiles + 1;
        for (int32_t t = lo; t < nxt; ++t) te[t - 1] = (int32_t)(i + 1);
    } else {
        for (int32_t t = lo; t <= nb_tiles; ++t) te[t - 1] = (int32_t)m;
    }
}

// The same on 16-bit tile ids, eight sorted entries per thread (one 16-byte load, plus the id
// that follows them).
__global__ __launch_bounds__(256) void k_tile_ranges16(int64_t m, const uint16_t* __restrict__ st, int32_t nb_tiles,
                                                       int32_t* __restrict__ te, const int64_t* dm = nullptr,
                                                       int32_t* zero = nullptr, int64_t nzero = 0) {
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    // (also clears zero[0, nzero) for the next kernel)
    for (int64_t k = i0 / 8; k < nzero; k += (int64_t)gridDim.x * blockDim.x) zero[k] = 0;
    if (dm) {   // device key count (the grid covers the key capacity); no keys: empty tiles
        m = *dm;
        if (m == 0)
            for (int64_t k = i0 / 8; k < nb_tiles; k += (int64_t)gridDim.x * blockDim.x) te[k] = 0;
    }
    if (i0 >= m) return;
    int32_t id[9];
    if (i0 + 8 < m) {
        const uint4 q = *reinterpret_cast<const uint4*>(st + i0);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            id[2 * k] = (int32_t)(w[k] & 0xffffu);
            id[2 * k + 1] = (int32_t)(w[k] >> 16);
        }
        id[8] = st[i0 + 8];
    } else {
#pragma unroll
        for (int k = 0; k < 9; ++k) id[k] = i0 + k < m ? (int32_t)st[i0 + k] : 0;
    }
    if (i0 == 0) {
        const int32_t stop = id[0] < nb_tiles + 1 ? id[0] : nb_tiles + 1;
        for (int32_t t = 1; t < stop; ++t) te[t - 1] = 0;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int64_t i = i0 + k;
        if (i >= m) break;
        const int32_t lo = id[k] < 1 ? 1 : id[k];
        if (i + 1 < m) {
            const int32_t nxt = id[k + 1] > nb_tiles + 1 ? nb_tiles + 1 : id[k + 1];
            for (int32_t t = lo; t < nxt; ++t) te[t - 1] = (int32_t)(i + 1);
        } else {
            for (int32_t t = lo; t <= nb_tiles; ++t) te[t - 1] = (int32_t)m;
        }
    }
}

// ------------------------------------------------------------------------------------
// Tile lists by coarse binning (at most 65535 tiles)
// ------------------------------------------------------------------------------------
// The reference sorts the M (tile, depth) keys (forward_core.jl:605-660); its result is, for
// every tile in id order, the Gaussians covering the tile in depth order. Here the non-empty
// Gaussians, already in depth order, are binned to coarse blocks of 2^sx x 2^sy tiles: one
// 16-bit block id per (Gaussian, block its tile rectangle touches), stably sorted by the radix
// passes (emission fused with the first), far fewer entries than keys. Then one workgroup
// per block walks the block's Gaussians in depth order and, for each of its tiles, keeps
// those whose rectangle covers the tile: k_bin_tiles<COUNT> counts them, a scan turns the
// counts into tiles_end (a scan), and k_bin_tiles<WRITE> writes each tile's Gaussians (wavefront
// compaction, consecutive addresses) at the tile's place. Same lists as the sort, bit for
// bit, with the M keys never written or moved.

// Block geometry: the smallest of 8 x 8, 16 x 8, 16 x 16 tiles that leaves at most 255 blocks
// (8-bit ids: one radix pass), else 16 x 16.
struct BinGeom {
    int sx, sy;
    int32_t nbx, nby;
    int32_t nblocks() const { return nbx * nby; }
    int tpb() const { return 1 << (sx + sy); }   // tiles per block
};
static BinGeom bin_geom(const tdgs_tiling* t) {
    const int shapes[3][2] = {{3, 3}, {4, 3}, {4, 4}};
    BinGeom g{4, 4, 0, 0};
    for (int k = 0; k < 3; ++k) {
        g.sx = shapes[k][0];
        g.sy = shapes[k][1];
        g.nbx = (int32_t)ceil_div(t->nb_tiles_x, 1 << g.sx);
        g.nby = (int32_t)ceil_div(t->nb_tiles_y, 1 << g.sy);
        if (g.nblocks() <= 255) break;   // 1-based ids of at most 8 bits
    }
    return g;
}

// Tiles and blocks touched by each non-empty Gaussian in depth order, packed as
// (tiles << 32) | blocks (entries past N_b count 0): one scan gives the blocks' emission
// offsets in the low half and, in its total, the key count M in the high half (both below
// 2^31, so the halves never carry into each other).
struct SortedTileBlockCounts {
    const int4* srect;   // rectangles in depth order
    int sx, sy;
    const int64_t* d_nb;
    __device__ int64_t operator()(int64_t j) const {
        if (j >= *d_nb) return 0;
        const int4 r = srect[j];
        const int32_t blocks =
            (((r.z - 1) >> sx) - ((r.x - 1) >> sx) + 1) * (((r.w - 1) >> sy) - ((r.y - 1) >> sy) + 1);
        return ((int64_t)rect_area(r) << 32) | (int64_t)blocks;
    }
};
// WriteScanAndBlocks on the blocks' half of the packed scan.
struct WriteBlockScan {
    WriteScanAndBlocks w;
    __device__ void operator()(int64_t j, int64_t incl, int64_t item) const {
        w(j, incl & kLow32, (int32_t)(item & kLow32));
    }
};

// Work is dealt in chunks of the coarse list, not per block, so that every workgroup gets the
// same number of entries however unevenly the Gaussians spread over the blocks: chunk k is
// entries [k E, (k + 1) E) of the lists of all blocks one after the other (E = the
// workgroup's threads x bin_per). A chunk that straddles block boundaries is processed as one
// segment per block; segment (k, b) has the unique index k + b (both grow along the list), and
// its per-tile counts are table[(k + b) tpb + local tile] (tpb = tiles per block).
// Candidates each thread stages per chunk (their loads in flight together): 4 for blocks 16
// tiles wide, where the write pass runs one tile at a time and longer runs per segment pay
// (3840 x 2160, 3M Gaussians: 0.97 -> 0.91 ms for the lists), 2 for blocks 8 wide (1920 x 1080,
// 1M Gaussians: 4 measured 45 -> 55 us).
constexpr int bin_per(int sx) { return sx >= 4 ? 4 : 2; }
// Workgroups of a launch (a grid-stride loop covers the rest): one per chunk up to 8192 chunks
// (3840 x 2160, 3M Gaussians: 5.3k chunks; lists 0.866 -> 0.82 ms against a cap of 2048, and
// 0.90 ms with 1024 or 512).
constexpr int kBinMaxGrid = 8192;

// Entries of the segment count table for key capacity kc (the coarse entries never exceed
// the keys: each Gaussian touches at least one tile of every block it is listed in): at most
// 4 / (4 bin_per) bytes per key. (Chunks of 2 entries per thread measured 70 -> 66 us for the
// tile lists at 1M Gaussians, 1080p; 1 per thread 63 us, but twice the table.)
inline int64_t bin_table_entries(int64_t kc, const BinGeom& g) {
    return (ceil_div(kc > 0 ? kc : 1, (int64_t)g.tpb() * 4 * bin_per(g.sx)) + g.nblocks() + 1) * g.tpb();
}

struct BinArgs {
    int32_t ntx, nty, nbx, sy, nblocks;
    const int32_t* cvals;      // the blocks' lists: fgidx (1-based), block by block, depth order within
    const int32_t* cend;       // end (exclusive) of each block's run in cvals, or null:
    const uint32_t* totals;    // the coarse radix pass's digit totals (block b has id b + 1)
    int64_t mc;                // entries of cvals (launch bound)
    const int64_t* dmc;        // entries used (device counts), or null
    const int32_t* ranges;     // tile rectangles [x0, y0, x1, y1] (1-based, inclusive) by fgidx
    const uint32_t* cmask;     // or null: each entry's tiles of its block (EmitGrid::block_mask)
    int32_t* table;            // COUNT writes the Gaussians of each segment covering each tile
    int32_t* tile_totals;      // COUNT adds them up per tile (zeroed beforehand)
    const int32_t* tiles_end;  // WRITE: inclusive ends of the tiles' lists
    int32_t* out;              // WRITE: sdfgidx_to_fgidx
    int32_t cap;               // WRITE: entries of out
    uint32_t* err;
};

// Workgroup: 4 threads per tile of a block of 2^SX x 2^sy tiles; wavefront w takes the
// block's tiles 16 w .. 16 w + 15 (row-major, 2^SX per row). A segment's Gaussians go
// through LDS, bin_per(SX) per thread, as the tile rectangle clipped to the block in two bit
// masks (columns, rows). COUNT counts the hits of each (segment, tile), each lane in byte
// counters over its own candidates, summed over the wavefront; WRITE tests 64 candidates at a
// time against a tile with one ballot and writes each hit at the tile's list start + the
// earlier segments' hits + the hits before it.
// (Staging the writes in LDS rings and storing 64 entries at a time measured no faster.)
// LDS (dynamic): the chunk's candidates, 2 bin_per(SX) words per thread.
template <int SX, bool WRITE>
__global__ __launch_bounds__(1024) void k_bin_tiles(BinArgs a) {
    extern __shared__ uint32_t s_dyn[];
    __shared__ int32_t s_cend[1024];   // the blocks' ends, when there are at most 1024 blocks
    __shared__ int32_t s_b[2];
    constexpr int PER = bin_per(SX);
    int32_t* const s_f = reinterpret_cast<int32_t*>(s_dyn);   // the candidates' fgidx
    uint32_t* const s_m = s_dyn + blockDim.x * PER;           // and tile masks
    constexpr int BW = 1 << SX;
    const int BH = 1 << a.sy;
    const int tpb = BW * BH;
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    const int nt = (int)blockDim.x * PER;   // entries per chunk
    int64_t mc = a.mc;
    if (a.dmc && *a.dmc < mc) mc = *a.dmc;
    const int64_t nchunks = (mc + nt - 1) / nt;
    if ((int64_t)blockIdx.x >= nchunks) return;
    const bool lds_ends = a.nblocks <= 1024;
    if (a.totals) {
        // one radix pass sorted the 8-bit block ids (at most 255 blocks, at least 256
        // threads): the ends are the inclusive prefix sums of the digit totals 1..255
        const int lane = __lane_id();
        int32_t c = t < kRsBins && t > 0 ? (int32_t)a.totals[t] : 0;
        for (int d = 1; d < kWave; d <<= 1) {
            const int32_t o = __shfl_up(c, d, kWave);
            if (lane >= d) c += o;
        }
        if (t < kRsBins && lane == kWave - 1) s_cend[1020 + t / kWave] = c;   // wave totals (t < 256)
        __syncthreads();
        if (t < kRsBins) {
            for (int q = 0; q < t / kWave; ++q) c += s_cend[1020 + q];
        }
        __syncthreads();
        if (t > 0 && t <= a.nblocks) s_cend[t - 1] = c;
    } else if (lds_ends) {
        for (int i = t; i < a.nblocks; i += blockDim.x) s_cend[i] = a.cend[i];
    }
    auto end_of = [&](int i) -> int64_t {
        const int64_t e = lds_ends ? s_cend[i] : a.cend[i];
        return e < mc ? e : mc;
    };
    const int li = 16 * w + lane;     // lanes < 16: the tile this lane reports (local index)
    const int ly0 = (16 * w) >> SX;   // the wavefront's first local row
    for (int64_t k = blockIdx.x; k < nchunks; k += gridDim.x) {
        const int64_t lo = k * nt, hi = lo + nt < mc ? lo + nt : mc;
        // the blocks holding entries lo and hi - 1 (the ends never decrease): counts of the
        // blocks ending at or before lo, and before hi
        if (t == 0) s_b[0] = s_b[1] = 0;
        __syncthreads();
        int c0 = 0, c1 = 0;
        for (int i = t; i < a.nblocks; i += blockDim.x) {
            const int64_t e = end_of(i);
            c0 += e <= lo;
            c1 += e < hi;
        }
        for (int d = kWave / 2; d >= 1; d >>= 1) {
            c0 += __shfl_xor(c0, d);
            c1 += __shfl_xor(c1, d);
        }
        if (lane == 0 && (c0 | c1) != 0) {
            atomicAdd(&s_b[0], c0);
            atomicAdd(&s_b[1], c1);
        }
        __syncthreads();
        const int b0 = s_b[0], b1 = s_b[1];
        __syncthreads();   // (s_b is reset by the next chunk)
        for (int b = b0; b <= b1 && b < a.nblocks; ++b) {
            const int64_t bb = b == 0 ? 0 : end_of(b - 1), be = end_of(b);
            const int64_t cb = lo > bb ? lo : bb, ce = hi < be ? hi : be;
            if (cb >= ce) continue;
            const int bx = b % a.nbx, by = b / a.nbx;
            const int x0b = bx * BW, y0b = by * BH;   // 0-based first tile of the block
            const int x = x0b + (li & (BW - 1)), y = y0b + (li >> SX);
            const bool in_image = lane < 16 && x < a.ntx && y < a.nty;
            int32_t* const row = a.table + (k + b) * (int64_t)tpb;
            int32_t cnt[16];   // WRITE: the next output index of each tile
            int32_t start = 0;
            int32_t seg_hits = 0;   // WRITE, lane i < 16: this segment's hits of tile i (COUNT's row)
            if (WRITE) {
                // tile i (i < 16) of the wavefront: its list start plus the block's earlier
                // segments' hits, summed by lanes i, i + 16, i + 32, i + 48 over every fourth
                // segment (independent loads), then across the four
                const int tl = 16 * w + (lane & 15), part = lane >> 4;
                const int xs = x0b + (tl & (BW - 1)), ys = y0b + (tl >> SX);
                if (xs < a.ntx && ys < a.nty) {
                    const int tile = xs + ys * a.ntx;
                    if (part == 0) seg_hits = row[tl];
                    if (part == 0 && tile > 0) start = a.tiles_end[tile - 1];
#pragma unroll 4
                    for (int64_t k2 = bb / nt + part; k2 < k; k2 += 4) start += a.table[(k2 + b) * (int64_t)tpb + tl];
                }
                start += __shfl_xor(start, 16);
                start += __shfl_xor(start, 32);
            }
            // candidates cb + t + blockDim q (q < PER): the loads issue together. Their
            // masks come sorted along with them (cmask), else from the rectangles.
            int32_t f[PER];
            uint32_t mk[PER];
            if (a.cmask) {
#pragma unroll
                for (int q = 0; q < PER; ++q) {
                    const int64_t e = cb + t + (int64_t)blockDim.x * q;
                    f[q] = WRITE && e < ce ? a.cvals[e] : 0;
                    mk[q] = e < ce ? a.cmask[e] : 0u;
                }
            } else {
#pragma unroll
                for (int q = 0; q < PER; ++q) {
                    const int64_t e = cb + t + (int64_t)blockDim.x * q;
                    f[q] = e < ce ? a.cvals[e] : 0;
                }
                int4 r[PER];
#pragma unroll
                for (int q = 0; q < PER; ++q)
                    r[q] = f[q] > 0 ? reinterpret_cast<const int4*>(a.ranges)[f[q] - 1] : make_int4(1, 1, 0, 0);
#pragma unroll
                for (int q = 0; q < PER; ++q) {
                    // columns in bits 0-15, rows in bits 16-31 (of the block); none for an empty slot
                    const int cx0 = max(r[q].x - 1 - x0b, 0), cx1 = min(r[q].z - 1 - x0b, BW - 1);
                    const int cy0 = max(r[q].y - 1 - y0b, 0), cy1 = min(r[q].w - 1 - y0b, BH - 1);
                    const uint32_t cm = cx1 >= cx0 ? (2u << cx1) - (1u << cx0) : 0u;
                    const uint32_t rm = cy1 >= cy0 ? (2u << cy1) - (1u << cy0) : 0u;
                    mk[q] = cm | (rm << 16);
                }
            }
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                s_f[t + blockDim.x * q] = f[q];
                s_m[t + blockDim.x * q] = mk[q];
            }
            __syncthreads();
            const int nk = __builtin_amdgcn_readfirstlane((int)(ce - cb));
            int32_t wave_hits = seg_hits;
            if (WRITE) {
                for (int d = 16; d >= 1; d >>= 1) wave_hits += __shfl_xor(wave_hits, d);
                wave_hits = __builtin_amdgcn_readfirstlane(wave_hits);
            }
            // WRITE with long runs (per tile and segment, on average 16 or more hits per 64
            // candidates and 256 or more in all): one tile at a time, so that the wavefront's
            // stores to a tile's list follow each other (one contiguous run of the list per
            // segment) instead of interleaving sixteen lists; the segment's hits of each tile
            // (counted by k_bin_tiles<COUNT>) skip the tiles without any and end a tile's walk
            // at its last hit. Shorter runs take the candidate-major loop below (one LDS read
            // per 64 candidates for all 16 tiles). (At 3840 x 2160, 3M Gaussians, runs average
            // ~1100 entries: lists 1.31 -> 0.92 ms; at 1920 x 1080, 1M Gaussians, ~70, and the
            // tile-major walk from 16 hits per 64 candidates alone measured 45 -> 49 us.)
            if (WRITE && wave_hits >= 4 * nk && wave_hits >= 16 * 256) {
                const int row0 = 16 + __builtin_amdgcn_readfirstlane(ly0);
#pragma unroll 1
                for (int i = 0; i < 16; ++i) {
                    const int32_t nh = __builtin_amdgcn_readlane(seg_hits, i);
                    if (nh <= 0) continue;
                    const uint32_t need = (1u << (i & (BW - 1))) | (1u << (row0 + (i >> SX)));
                    int32_t c = __builtin_amdgcn_readlane(start, i);
                    const int32_t c_end = c + nh;
                    // (entries past nk are zero: no hits)
                    int32_t nf = s_f[lane];
                    uint32_t nm = s_m[lane];
                    for (int j0 = 0; j0 < nk && c < c_end; j0 += kWave) {
                        const int32_t fv = nf;
                        const uint32_t p = nm;
                        if (j0 + kWave < nk) {   // read ahead, both words
                            nf = s_f[j0 + kWave + lane];
                            nm = s_m[j0 + kWave + lane];
                        }
                        asm volatile("" ::"v"(fv));   // not sunk into the branch below
                        const bool hit = (p & need) == need;
                        const uint64_t bal = __ballot(hit);
                        if (hit) {
                            const int32_t o = (int32_t)__builtin_amdgcn_mbcnt_hi(
                                (uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, (uint32_t)c));
                            a.out[o < a.cap ? o : a.cap - 1] = fv;
                        }
                        c += __popcll(bal);
                    }
                }
                __syncthreads();   // s_f, s_m are free again
                continue;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) cnt[i] = WRITE ? __builtin_amdgcn_readlane(start, i) : 0;
            // the wavefront's 16 tiles as bits of candidate mask p: 8 x 2 (SX = 3) or 16 x 1 (SX = 4)
            auto tile_bits = [&](uint32_t p) -> uint32_t {
                if (SX == 3)
                    return (((p >> (16 + ly0)) & 1u) ? (p & 0xffu) : 0u) |
                           (((p >> (17 + ly0)) & 1u) ? (p & 0xffu) << 8 : 0u);
                return ((p >> (16 + ly0)) & 1u) ? (p & 0xffffu) : 0u;
            };
            if (!WRITE) {
                // Each lane counts its own candidates' hits of tile i in byte i of acc (at most
                // nk / 64 <= 32 per byte): every 4 bits of the hit mask become 4 bytes of 0 / 1
                // by one multiply (n 0x204081 puts bit k of n at bit 8 k, the four copies not
                // overlapping). The bytes are then summed over the wavefront as 16-bit fields.
                // (A ballot and a population count per tile cost ~36 vector and ~34 scalar
                // instructions per 64 candidates, against 16 vector ones here.)
                uint32_t acc[4] = {0u, 0u, 0u, 0u};
                for (int j0 = 0; j0 < nk; j0 += kWave) {
                    const uint32_t h = tile_bits(s_m[j0 + lane]);   // (entries past nk are zero: no hits)
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[q] += (((h >> (4 * q)) & 15u) * 0x204081u) & 0x01010101u;
                }
                // s[2q] holds bytes 0 and 2 of acc[q] (tiles 4q, 4q + 2) as 16-bit fields, s[2q + 1]
                // bytes 1 and 3 (tiles 4q + 1, 4q + 3): wavefront sums stay below 64 x 32
                uint32_t sm[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    sm[2 * q] = acc[q] & 0x00ff00ffu;
                    sm[2 * q + 1] = (acc[q] >> 8) & 0x00ff00ffu;
                }
#pragma unroll
                for (int d = kWave / 2; d >= 1; d >>= 1) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) sm[k] += (uint32_t)__shfl_xor((int)sm[k], d, kWave);
                }
                int32_t mine = 0;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t word = sm[2 * (i >> 2) + (i & 1)];
                    const int32_t c = (int32_t)((word >> (16 * ((i >> 1) & 1))) & 0xffffu);
                    mine = lane == i ? c : mine;
                }
                if (lane < 16) row[li] = mine;
                if (in_image && mine != 0) atomicAdd(&a.tile_totals[x + y * a.ntx], mine);
                __syncthreads();   // s_f, s_m are free again
                continue;
            }
            for (int j0 = 0; j0 < nk; j0 += kWave) {
                const uint32_t h = tile_bits(s_m[j0 + lane]);   // (entries past nk are zero: no hits)
                const int32_t fv = s_f[j0 + lane];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const bool hit = (h >> i) & 1u;
                    const uint64_t bal = __ballot(hit);
                    if (hit) {
                        // the tile's next index plus the hits in lower lanes (v_mbcnt); the
                        // counts come from the same walk, the index is clamped all the same
                        const int32_t o = (int32_t)__builtin_amdgcn_mbcnt_hi(
                            (uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, (uint32_t)cnt[i]));
                        a.out[o < a.cap ? o : a.cap - 1] = fv;
                    }
                    cnt[i] += __popcll(bal);
                }
            }
            __syncthreads();   // s_f, s_m are free again
        }
    }
}

// One workgroup: tiles_end = inclusive scan of the tiles' totals, 4096 tiles per step (four
// per thread, read as int4 from the array padded to 4k and written as int4 where all four are
// tiles and tiles_end is 16-byte aligned), with a running carry. The total must equal the key count M (*expect, or
// expect_value; else *err is set: the lists would be incomplete).
__global__ __launch_bounds__(1024) void k_bin_scan(const int32_t* __restrict__ totals, int32_t nt,
                                                   int32_t* __restrict__ tiles_end, const int64_t* expect,
                                                   int64_t expect_value, uint32_t* err) {
    __shared__ int64_t s_w[2][1024 / kWave];
    const int t = threadIdx.x, lane = __lane_id(), w = t / kWave;
    int64_t carry = 0;
    int step = 0;
    for (int base = 0; base < nt; base += 4096, step ^= 1) {
        const int i = base + 4 * t;
        int4 v = make_int4(0, 0, 0, 0);
        if (i < nt) {
            v = *reinterpret_cast<const int4*>(totals + i);
            if (i + 1 >= nt) v.y = 0;
            if (i + 2 >= nt) v.z = 0;
            if (i + 3 >= nt) v.w = 0;
        }
        const int64_t sum = (int64_t)v.x + v.y + v.z + v.w;
        int64_t incl = sum;
        for (int d = 1; d < kWave; d <<= 1) {
            const int64_t o = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += o;
        }
        if (lane == kWave - 1) s_w[step][w] = incl;   // (alternate buffers: one barrier a step)
        __syncthreads();
        int64_t off = carry, total = 0;
        for (int k = 0; k < 1024 / kWave; ++k) {
            const int64_t x = s_w[step][k];
            if (k < w) off += x;
            total += x;
        }
        carry += total;
        if (i < nt) {
            int4 e;
            e.x = (int32_t)(off + incl - sum + v.x);
            e.y = e.x + v.y;
            e.z = e.y + v.z;
            e.w = e.z + v.w;
            if (i + 3 < nt && (reinterpret_cast<uintptr_t>(tiles_end) & 15) == 0) {
                *reinterpret_cast<int4*>(tiles_end + i) = e;
            } else {
                tiles_end[i] = e.x;
                if (i + 1 < nt) tiles_end[i + 1] = e.y;
                if (i + 2 < nt) tiles_end[i + 2] = e.z;
                if (i + 3 < nt) tiles_end[i + 3] = e.w;
            }
        }
    }
    if (t == 0 && carry != (expect ? *expect : expect_value)) atomicOr(err, 1u);
}

// The sorted keys (tile << 32 | depth bits) of the tile lists: the tile of list entry i is the
// first with tiles_end > i.
__global__ __launch_bounds__(256) void k_assemble_keys_te(int64_t m, const int32_t* __restrict__ te, int32_t nt,
                                                          const int32_t* __restrict__ sv,
                                                          const float* __restrict__ depths,
                                                          int64_t* __restrict__ sk) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m) return;
    int lo = 0, hi = nt - 1;   // smallest tile index with te > i
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((int64_t)te[mid] > i) hi = mid; else lo = mid + 1;
    }
    sk[i] = ((int64_t)(lo + 1) << 32) | (int64_t)float_bits(depths[sv[i] - 1]);
}

// The 64-bit sorted keys (tile << 32 | depth bits of the Gaussian) from the 16-bit sorted
// tile ids and the sorted values.
__global__ __launch_bounds__(256) void k_assemble_keys(int64_t m, const uint16_t* __restrict__ st,
                                                       const int32_t* __restrict__ sv,
                                                       const float* __restrict__ depths,
                                                       int64_t* __restrict__ sk) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m) return;
    sk[i] = ((int64_t)st[i] << 32) | (int64_t)float_bits(depths[sv[i] - 1]);
}

// tiles_end from the tile-coverage difference array D ((ntx+1) x (nty+1), 0-based corners).
// With col_y(x) = sum_{y' <= y} D[y'][x], the keys of tile (x, y) number
// count(x, y) = sum_{x' <= x} col_y(x'), tiles_end(x, y) = sum_{x' <= x} count(x', y) plus the
// keys of all rows above, sum_{y' < y, x' < ntx} (y - y') (ntx - x') D[y'][x']. Workgroup y
// reads rows 0..y (L2-resident) and scans its row twice, so tiles_end needs no pass over the M
// sorted keys and equals fill_tiles_end_sdfgidx_kernel!'s (forward_core.jl:676-734) exactly.
constexpr int kTeThreads = 256;

// copy 0 <- sum of the kRectCopies copies
__global__ __launch_bounds__(256) void k_merge_rect_diff(int32_t* __restrict__ diff, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int32_t s = diff[i];
#pragma unroll 8
    for (int k = 1; k < kRectCopies; ++k) s += diff[(int64_t)k * n + i];
    diff[i] = s;
}

// Inclusive block scan of one int64 per thread (kTeThreads threads); *total gets the sum.
__device__ __forceinline__ int64_t te_block_scan(int64_t v, int64_t* s_red, int64_t* total) {
    const int lane = __lane_id(), wave = threadIdx.x / kWave;
    int64_t incl = v;
    for (int d = 1; d < kWave; d <<= 1) {
        const int64_t o = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) s_red[wave] = incl;
    __syncthreads();
    int64_t off = 0, tot = 0;
    for (int k = 0; k < kTeThreads / kWave; ++k) {
        if (k < wave) off += s_red[k];
        tot += s_red[k];
    }
    __syncthreads();
    *total = tot;
    return off + incl;
}

__global__ __launch_bounds__(kTeThreads) void k_tiles_end_from_rects(const int32_t* __restrict__ diff, int ntx,
                                                                    int32_t* __restrict__ te) {
    __shared__ int64_t s_red[kTeThreads / kWave];
    const int y = blockIdx.x, t = threadIdx.x, lane = __lane_id(), wave = t / kWave;
    const int w = ntx + 1;
    int64_t above = 0;   // this thread's share of the keys in rows < y
    int64_t carry_col = 0, carry_cnt = 0;
    for (int x0 = 0; x0 < ntx; x0 += kTeThreads) {
        const int x = x0 + t;
        int64_t col = 0;
        if (x < ntx) {
            const int64_t wx = ntx - x;
            int yy = 0;
            for (; yy + 4 <= y; yy += 4) {
                const int32_t d0 = diff[(int64_t)yy * w + x], d1 = diff[(int64_t)(yy + 1) * w + x];
                const int32_t d2 = diff[(int64_t)(yy + 2) * w + x], d3 = diff[(int64_t)(yy + 3) * w + x];
                col += (int64_t)d0 + d1 + d2 + d3;
                above += wx * ((int64_t)(y - yy) * d0 + (int64_t)(y - yy - 1) * d1 + (int64_t)(y - yy - 2) * d2 +
                               (int64_t)(y - yy - 3) * d3);
            }
            for (; yy < y; ++yy) {
                const int32_t d = diff[(int64_t)yy * w + x];
                col += d;
                above += wx * (int64_t)(y - yy) * d;
            }
            col += diff[(int64_t)y * w + x];
        }
        int64_t tot;
        const int64_t count = te_block_scan(col, s_red, &tot) + carry_col;   // keys of tile (x, y)
        carry_col += tot;
        const int64_t incl = te_block_scan(x < ntx ? count : 0, s_red, &tot) + carry_cnt;
        carry_cnt += tot;
        if (x < ntx) te[(int64_t)y * ntx + x] = (int32_t)incl;   // rows above added below
    }
    for (int d = 32; d >= 1; d >>= 1) above += __shfl_xor(above, d, kWave);
    if (lane == 0) s_red[wave] = above;
    __syncthreads();
    int64_t rows_above = 0;
    for (int k = 0; k < kTeThreads / kWave; ++k) rows_above += s_red[k];
    for (int x = t; x < ntx; x += kTeThreads) te[(int64_t)y * ntx + x] += (int32_t)rows_above;
}

// ------------------------------------------------------------------------------------
// Blending (render_tiles_kernel!, forward_core.jl:756-993)
// ------------------------------------------------------------------------------------

struct __align__(16) BlendRec {
    float4 a;  // p0 p1 p2 p3
    float4 b;  // p4 p5 r g
    float4 c;  // b depth - -
};

struct BlendArgs {
    int32_t W, H, TW, TH, ntx;
    float bg0, bg1, bg2, min_alpha, max_alpha, min_T;
    float e_cut;   // exp_f(e) < min_alpha for every exponent e < e_cut
    int cut_low;   // e_cut < -87: live exponents may leave exp_f's polynomial range
    int64_t m;
    const int32_t* tiles_end;
    const int32_t* sorted_f;
    const float* f2d;
    const float* depths;
    float* rgb;
    float* T;
    float* depth;
    int32_t* last;
    unsigned long long* evaluations;  // COUNT variant: [evaluations, live, contributing]
    // device-count render: the context's counters (key count used, N_f), and the frame counts
    // of the render buffers, which workgroup (0, 0) fills in
    const int64_t* dcount;
    int64_t* frame;
    int64_t* mon;        // frame monitor state (device) and its host copy
    int64_t* mon_host;
};

// The blending steps of one batch of nb staged records, written out instruction by instruction.
// Per record it performs exactly the single-precision operations of the C++ loop in
// k_render_tiles below (same operands, same order: the exponent's five fused multiply-adds,
// exp_f_core's sequence, min with max_alpha, 1 - alpha, the products and the colour fused
// multiply-adds; exp_f_core's final product with 2^n is one v_ldexp_f32, which rounds exactly
// as that product does, subnormal results included), so every result is bit for bit the
// compiled loop's. What differs is the bookkeeping. Inside the loop exec holds the lanes still
// blending (act), so every compare yields its mask restricted to them: the live lanes are the
// compare with e_cut (the exponential is skipped, by a branch on VCC, when none is live), the
// contributing lanes the compare with min_alpha under exec = live, the stopping lanes the
// compare with min_T under exec = contributing, and the state update runs under exec =
// contributing and not stopping; exec is restored on exit. That is 7 scalar and 31 vector
// instructions per live record (the compiled loop needed about 30 and 39) and 1 scalar
// instruction per skipped one. The next record (all ten floats) is read from LDS
// into a second register set while the current one is processed, so no step waits on LDS.
// Records run in groups of four with one bound check per group (a scalar instruction costs a
// step about as much as a vector one): after a batch of nb records the LDS array holds three
// records of padding that no pixel is live for, and one more for the read past the last group.
// Valid only when every live exponent lies in [-87, 88] (the batch is not `checked`). v39-v63
// are its scratch registers (the kernel stays within 64 VGPRs, 8 wavefronts per SIMD). Returns
// the mask of the lanes that did not stop.
// the literals of blend_batch's exponential are exp_poly's coefficients
static_assert(__builtin_bit_cast(uint32_t, kExpC6) == 0x3ab51223u && __builtin_bit_cast(uint32_t, kExpC4) == 0x3d2aac79u &&
                  __builtin_bit_cast(uint32_t, kExpC3) == 0x3e2aaa49u && __builtin_bit_cast(uint32_t, kExpC2) == 0x3efffffeu &&
                  __builtin_bit_cast(uint32_t, -kLn2Hi) == 0xbf317200u && __builtin_bit_cast(uint32_t, -kLn2Lo) == 0xb5bfbe8eu &&
                  __builtin_bit_cast(uint32_t, kLog2e) == 0x3fb8aa3bu,
              "blend_batch constants");
// A record no pixel is live for: every exponent coefficient 0 but the constant term, -inf
// (colour and depth unused). The constants are made at the store (an asm the compiler does not
// hoist), so that they hold no registers across the blending loop.
__device__ __forceinline__ void blend_pad(BlendRec* r) {
    float z, ninf;
    asm volatile("v_mov_b32 %0, 0\n v_mov_b32 %1, 0xff800000" : "=v"(z), "=v"(ninf));
    r->a = make_float4(z, z, z, z);
    *reinterpret_cast<float2*>(&r->b) = make_float2(z, ninf);
}

template <bool DEPTH, bool LAST>
__device__ __forceinline__ uint64_t blend_batch(uint32_t lds_addr, int32_t idx0, int32_t idx_end, float uu,
                                                float vv, float uv, float cu, float cv, float e_cut,
                                                float max_alpha, float min_alpha, float min_T, float& T,
                                                float& C0, float& C1, float& C2, float& D, int32_t& last) {
    const float c5 = kExpC5;   // exp_poly's coefficient of r^5 (a VGPR operand)
    uint64_t act, ent, stp;
    int32_t idx;
#define TDGS_BLEND_ASM(DEPTH_FMA, READ_C, LAST_MOV)                                                         \
    asm volatile(                                                                                           \
        "s_mov_b64 %[ent], exec\n"                                                                          \
        "s_and_b64 %[act], exec, exec\n"                                                                    \
        "s_cbranch_scc0 .Lend_%=\n"                                                                         \
        "s_mov_b32 %[idx], %[i0]\n"                                                                         \
        "v_mov_b32 v39, %[addr]\n"                                                                          \
        "ds_read_b128 v[40:43], v39\n"                                                                      \
        "ds_read_b128 v[44:47], v39 offset:16\n"                                                            \
        READ_C("v[48:49]", "v48", "32")                                                                     \
        ".Lstep_%=:\n"                                                                                      \
        "s_waitcnt lgkmcnt(0)\n"                                                                            \
        "ds_read_b128 v[50:53], v39 offset:48\n"                                                            \
        "ds_read_b128 v[54:57], v39 offset:64\n"                                                            \
        READ_C("v[58:59]", "v58", "80")                                                                     \
        "v_fma_f32 v60, v44, %[cv], v45\n"                                                                  \
        "v_fmac_f32 v60, v43, %[cu]\n"                                                                      \
        "v_fmac_f32 v60, v42, %[uv]\n"                                                                      \
        "v_fmac_f32 v60, v41, %[vv]\n"                                                                      \
        "v_fmac_f32 v60, v40, %[uu]\n"                                                                      \
        "v_cmp_ngt_f32 vcc, %[cut], v60\n"                                                                  \
        "s_cbranch_vccz .Ls0_%=\n"                                                                          \
        "s_mov_b64 exec, vcc\n"                                                                             \
        "v_mul_f32 v61, 0x3fb8aa3b, v60\n"                                                                  \
        "v_rndne_f32 v61, v61\n"                                                                            \
        "v_fmac_f32 v60, 0xbf317200, v61\n"                                                                 \
        "v_fmac_f32 v60, 0xb5bfbe8e, v61\n"                                                                 \
        "v_fmamk_f32 v62, v60, 0x3ab51223, %[c5]\n"                                                         \
        "v_fmaak_f32 v62, v62, v60, 0x3d2aac79\n"                                                           \
        "v_fmaak_f32 v62, v62, v60, 0x3e2aaa49\n"                                                           \
        "v_fmaak_f32 v62, v62, v60, 0x3efffffe\n"                                                           \
        "v_fma_f32 v62, v62, v60, 1.0\n"                                                                    \
        "v_fma_f32 v62, v62, v60, 1.0\n"                                                                    \
        "v_cvt_i32_f32 v61, v61\n"                                                                          \
        "v_ldexp_f32 v62, v62, v61\n"                                                                       \
        "v_min_f32 v62, %[maxa], v62\n"                                                                     \
        "v_cmp_ngt_f32 vcc, %[mina], v62\n"                                                                 \
        "v_sub_f32 v63, 1.0, v62\n"                                                                         \
        "v_mul_f32 v63, %[T], v63\n"                                                                        \
        "s_mov_b64 exec, vcc\n"                                                                             \
        "v_cmp_gt_f32 %[stp], %[minT], v63\n"                                                               \
        "s_andn2_b64 exec, exec, %[stp]\n"                                                                  \
        "v_mul_f32 v61, %[T], v62\n"                                                                        \
        "v_fmac_f32 %[C0], v61, v46\n"                                                                      \
        "v_fmac_f32 %[C1], v61, v47\n"                                                                      \
        "v_fmac_f32 %[C2], v61, v48\n"                                                                      \
        DEPTH_FMA("v49")                                                                                    \
        "v_mov_b32 %[T], v63\n"                                                                             \
        LAST_MOV("0")                                                                                       \
        "s_andn2_b64 %[act], %[act], %[stp]\n"                                                              \
        "s_mov_b64 exec, %[act]\n"                                                                          \
        "s_cbranch_scc0 .Lend_%=\n"                                                                         \
        ".Ls0_%=:\n"                                                                                        \
        "s_waitcnt lgkmcnt(0)\n"                                                                            \
        "ds_read_b128 v[40:43], v39 offset:96\n"                                                            \
        "ds_read_b128 v[44:47], v39 offset:112\n"                                                           \
        READ_C("v[48:49]", "v48", "128")                                                                    \
        "v_fma_f32 v60, v54, %[cv], v55\n"                                                                  \
        "v_fmac_f32 v60, v53, %[cu]\n"                                                                      \
        "v_fmac_f32 v60, v52, %[uv]\n"                                                                      \
        "v_fmac_f32 v60, v51, %[vv]\n"                                                                      \
        "v_fmac_f32 v60, v50, %[uu]\n"                                                                      \
        "v_cmp_ngt_f32 vcc, %[cut], v60\n"                                                                  \
        "s_cbranch_vccz .Ls1_%=\n"                                                                          \
        "s_mov_b64 exec, vcc\n"                                                                             \
        "v_mul_f32 v61, 0x3fb8aa3b, v60\n"                                                                  \
        "v_rndne_f32 v61, v61\n"                                                                            \
        "v_fmac_f32 v60, 0xbf317200, v61\n"                                                                 \
        "v_fmac_f32 v60, 0xb5bfbe8e, v61\n"                                                                 \
        "v_fmamk_f32 v62, v60, 0x3ab51223, %[c5]\n"                                                         \
        "v_fmaak_f32 v62, v62, v60, 0x3d2aac79\n"                                                           \
        "v_fmaak_f32 v62, v62, v60, 0x3e2aaa49\n"                                                           \
        "v_fmaak_f32 v62, v62, v60, 0x3efffffe\n"                                                           \
        "v_fma_f32 v62, v62, v60, 1.0\n"                                                                    \
        "v_fma_f32 v62, v62, v60, 1.0\n"                                                                    \
        "v_cvt_i32_f32 v61, v61\n"                                                                          \
        "v_ldexp_f32 v62, v62, v61\n"                                                                       \
        "v_min_f32 v62, %[maxa], v62\n"                                                                     \
        "v_cmp_ngt_f32 vcc, %[mina], v62\n"                                                                 \
        "v_sub_f32 v63, 1.0, v62\n"                                                                         \
        "v_mul_f32 v63, %[T], v63\n"                                                                        \
        "s_mov_b64 exec, vcc\n"                                                                             \
        "v_cmp_gt_f32 %[stp], %[minT], v63\n"                                                               \
        "s_andn2_b64 exec, exec, %[stp]\n"                                                                  \
        "v_mul_f32 v61, %[T], v62\n"                                                                        \
        "v_fmac_f32 %[C0], v61, v56\n"                                                                      \
        "v_fmac_f32 %[C1], v61, v57\n"                                                                      \
        "v_fmac_f32 %[C2], v61, v58\n"                                                                      \
        DEPTH_FMA("v59")                                                                                    \
        "v_mov_b32 %[T], v63\n"                                                                             \
        LAST_MOV("1")                                                                                       \
        "s_andn2_b64 %[act], %[act], %[stp]\n"                                                              \
        "s_mov_b64 exec, %[act]\n"                                                                          \
        "s_cbranch_scc0 .Lend_%=\n"                                                                         \
        ".Ls1_%=:\n"                                                                                        \
        "s_waitcnt lgkmcnt(0)\n"                                                                            \
        "ds_read_b128 v[50:53], v39 offset:144\n"                                                           \
        "ds_read_b128 v[54:57], v39 offset:160\n"                                                           \
        READ_C("v[58:59]", "v58", "176")                                                                    \
        "v_fma_f32 v60, v44, %[cv], v45\n"                                                                  \
        "v_fmac_f32 v60, v43, %[cu]\n"                                                                      \
        "v_fmac_f32 v60, v42, %[uv]\n"                                                                      \
        "v_fmac_f32 v60, v41, %[vv]\n"                                                                      \
        "v_fmac_f32 v60, v40, %[uu]\n"                                                                      \
        "v_cmp_ngt_f32 vcc, %[cut], v60\n"                                                                  \
        "s_cbranch_vccz .Ls2_%=\n"                                                                          \
        "s_mov_b64 exec, vcc\n"                                                                             \
        "v_mul_f32 v61, 0x3fb8aa3b, v60\n"                                                                  \
        "v_rndne_f32 v61, v61\n"                                                                            \
        "v_fmac_f32 v60, 0xbf317200, v61\n"                                                                 \
        "v_fmac_f32 v60, 0xb5bfbe8e, v61\n"                                                                 \
        "v_fmamk_f32 v62, v60, 0x3ab51223, %[c5]\n"                                                         \
        "v_fmaak_f32 v62, v62, v60, 0x3d2aac79\n"                                                           \
        "v_fmaak_f32 v62, v62, v60, 0x3e2aaa49\n"                                                           \
        "v_fmaak_f32 v62, v62, v60, 0x3efffffe\n"                                                           \
        "v_fma_f32 v62, v62, v60, 1.0\n"                                                                    \
        "v_fma_f32 v62, v62, v60, 1.0\n"                                                                    \
        "v_cvt_i32_f32 v61, v61\n"                                                                          \
        "v_ldexp_f32 v62, v62, v61\n"                                                                       \
        "v_min_f32 v62, %[maxa], v62\n"                                                                     \
        "v_cmp_ngt_f32 vcc, %[mina], v62\n"                                                                 \
        "v_sub_f32 v63, 1.0, v62\n"                                                                         \
        "v_mul_f32 v63, %[T], v63\n"                                                                        \
        "s_mov_b64 exec, vcc\n"                                                                             \
        "v_cmp_gt_f32 %[stp], %[minT], v63\n"                                                               \
        "s_andn2_b64 exec, exec, %[stp]\n"                                                                  \
        "v_mul_f32 v61, %[T], v62\n"                                                                        \
        "v_fmac_f32 %[C0], v61, v46\n"                                                                      \
        "v_fmac_f32 %[C1], v61, v47\n"                                                                      \
        "v_fmac_f32 %[C2], v61, v48\n"                                                                      \
        DEPTH_FMA("v49")                                                                                    \
        "v_mov_b32 %[T], v63\n"                                                                             \
        LAST_MOV("2")                                                                                       \
        "s_andn2_b64 %[act], %[act], %[stp]\n"                                                              \
        "s_mov_b64 exec, %[act]\n"                                                                          \
        "s_cbranch_scc0 .Lend_%=\n"                                                                         \
        ".Ls2_%=:\n"                                                                                        \
        "s_waitcnt lgkmcnt(0)\n"                                                                            \
        "ds_read_b128 v[40:43], v39 offset:192\n"                                                           \
        "ds_read_b128 v[44:47], v39 offset:208\n"                                                           \
        READ_C("v[48:49]", "v48", "224")                                                                    \
        "v_fma_f32 v60, v54, %[cv], v55\n"                                                                  \
        "v_fmac_f32 v60, v53, %[cu]\n"                                                                      \
        "v_fmac_f32 v60, v52, %[uv]\n"                                                                      \
        "v_fmac_f32 v60, v51, %[vv]\n"                                                                      \
        "v_fmac_f32 v60, v50, %[uu]\n"                                                                      \
        "v_cmp_ngt_f32 vcc, %[cut], v60\n"                                                                  \
        "s_cbranch_vccz .Ls3_%=\n"                                                                          \
        "s_mov_b64 exec, vcc\n"                                                                             \
        "v_mul_f32 v61, 0x3fb8aa3b, v60\n"                                                                  \
        "v_rndne_f32 v61, v61\n"                                                                            \
        "v_fmac_f32 v60, 0xbf317200, v61\n"                                                                 \
        "v_fmac_f32 v60, 0xb5bfbe8e, v61\n"                                                                 \
        "v_fmamk_f32 v62, v60, 0x3ab51223, %[c5]\n"                                                         \
        "v_fmaak_f32 v62, v62, v60, 0x3d2aac79\n"                                                           \
        "v_fmaak_f32 v62, v62, v60, 0x3e2aaa49\n"                                                           \
        "v_fmaak_f32 v62, v62, v60, 0x3efffffe\n"                                                           \
        "v_fma_f32 v62, v62, v60, 1.0\n"                                                                    \
        "v_fma_f32 v62, v62, v60, 1.0\n"                                                                    \
        "v_cvt_i32_f32 v61, v61\n"                                                                          \
        "v_ldexp_f32 v62, v62, v61\n"                                                                       \
        "v_min_f32 v62, %[maxa], v62\n"                                                                     \
        "v_cmp_ngt_f32 vcc, %[mina], v62\n"                                                                 \
        "v_sub_f32 v63, 1.0, v62\n"                                                                         \
        "v_mul_f32 v63, %[T], v63\n"                                                                        \
        "s_mov_b64 exec, vcc\n"                                                                             \
        "v_cmp_gt_f32 %[stp], %[minT], v63\n"                                                               \
        "s_andn2_b64 exec, exec, %[stp]\n"                                                                  \
        "v_mul_f32 v61, %[T], v62\n"                                                                        \
        "v_fmac_f32 %[C0], v61, v56\n"                                                                      \
        "v_fmac_f32 %[C1], v61, v57\n"                                                                      \
        "v_fmac_f32 %[C2], v61, v58\n"                                                                      \
        DEPTH_FMA("v59")                                                                                    \
        "v_mov_b32 %[T], v63\n"                                                                             \
        LAST_MOV("3")                                                                                       \
        "s_andn2_b64 %[act], %[act], %[stp]\n"                                                              \
        "s_mov_b64 exec, %[act]\n"                                                                          \
        "s_cbranch_scc0 .Lend_%=\n"                                                                         \
        ".Ls3_%=:\n"                                                                                        \
        "v_add_u32 v39, 0xc0, v39\n"                                                                        \
        "s_add_u32 %[idx], %[idx], 4\n"                                                                     \
        "s_cmp_lt_u32 %[idx], %[iend]\n"                                                                    \
        "s_cbranch_scc1 .Lstep_%=\n"                                                                        \
        ".Lend_%=:\n"                                                                                       \
        "s_waitcnt lgkmcnt(0)\n"                                                                            \
        "s_mov_b64 exec, %[ent]\n"                                                                          \
        : [act] "=&s"(act), [ent] "=&s"(ent), [stp] "=&s"(stp),                                       \
          [idx] "=&s"(idx), [T] "+v"(T), [C0] "+v"(C0), [C1] "+v"(C1), [C2] "+v"(C2), [D] "+v"(D),   \
          [last] "+v"(last)                                                                         \
        : [addr] "v"(lds_addr), [i0] "s"(idx0), [iend] "s"(idx_end), [uu] "v"(uu), [vv] "v"(vv),     \
          [uv] "v"(uv), [cu] "v"(cu), [cv] "v"(cv), [c5] "v"(c5), [cut] "s"(e_cut),                  \
          [maxa] "s"(max_alpha), [mina] "s"(min_alpha), [minT] "s"(min_T)                           \
        : "v39", "v40", "v41", "v42", "v43", "v44", "v45", "v46", "v47", "v48", "v49", "v50", "v51",  \
          "v52", "v53", "v54", "v55", "v56", "v57", "v58", "v59", "v60", "v61", "v62", "v63", "vcc",    \
          "scc", "memory")
#define TDGS_DEPTH_ON(R) "v_fmac_f32 %[D], v61, " R "\n"
#define TDGS_DEPTH_OFF(R) ""
// the record's last floats: blue and depth (b64), or blue alone (b32) without depth
#define TDGS_READ_BD(PAIR, ONE, OFF) "ds_read_b64 " PAIR ", v39 offset:" OFF "\n"
#define TDGS_READ_B(PAIR, ONE, OFF) "ds_read_b32 " ONE ", v39 offset:" OFF "\n"
// the last contributing index is tracked only when it is an output
#define TDGS_LAST_ON(K) "v_add_u32_e64 %[last], %[idx], " K "\n"
#define TDGS_LAST_OFF(K) ""
    if constexpr (DEPTH && LAST)
        TDGS_BLEND_ASM(TDGS_DEPTH_ON, TDGS_READ_BD, TDGS_LAST_ON);
    else if constexpr (DEPTH)
        TDGS_BLEND_ASM(TDGS_DEPTH_ON, TDGS_READ_BD, TDGS_LAST_OFF);
    else if constexpr (LAST)
        TDGS_BLEND_ASM(TDGS_DEPTH_OFF, TDGS_READ_B, TDGS_LAST_ON);
    else
        TDGS_BLEND_ASM(TDGS_DEPTH_OFF, TDGS_READ_B, TDGS_LAST_OFF);
#undef TDGS_BLEND_ASM
#undef TDGS_DEPTH_ON
#undef TDGS_DEPTH_OFF
#undef TDGS_READ_BD
#undef TDGS_READ_B
#undef TDGS_LAST_ON
#undef TDGS_LAST_OFF
    return act;
}

// One workgroup per tile, one thread per pixel (tile_pixel). Each batch of TW*TH sorted
// entries is converted to blending parameters once per tile and staged in LDS, where every
// lane reads the same record (broadcast). A wavefront skips an entry when no pixel it still
// blends can reach min_alpha (exponent below e_cut), leaves the batch when all its pixels
// are done, and the tile stops loading batches once every pixel is done. The steps of a batch
// run in blend_batch, except for the counting replay (COUNT) and for batches whose live
// exponents may leave [-87, 88] (`checked`), which take the loop below with exp_f's range
// handling.
template <bool RGB, bool DEPTH, bool COUNT = false, bool LAST = true>
__global__ __launch_bounds__(1024) void k_render_tiles(BlendArgs a) {
    extern __shared__ BlendRec s_rec[];
    const int NT = a.TW * a.TH;
    const int t = threadIdx.x;
    const int tx = blockIdx.x + 1, ty = blockIdx.y + 1;
    const int tile = tx + (ty - 1) * a.ntx;
    int u_in, v_in;
    tile_pixel(t, a.TW, a.TH, &u_in, &v_in);
    const int U = u_in + (tx - 1) * a.TW, V = v_in + (ty - 1) * a.TH;
    const bool on = U <= a.W && V <= a.H;
    const float cu = (float)u_in - 0.5f, cv = (float)v_in - 0.5f;
    const float uu = cu * cu, uv = cu * cv, vv = cv * cv;
    const float u0 = (float)((tx - 1) * a.TW), v0 = (float)((ty - 1) * a.TH);
    int64_t m = a.m;
    bool nothing = false;   // render_void!'s outputs (a device-count render with no keys)
    if (!COUNT && a.dcount) {
        m = a.dcount[kCntKeysUsed];
        nothing = m == 0 || a.dcount[0] == 0;
        if (tile == 1 && t == 0) {
            const int64_t keys = a.dcount[1], status = a.dcount[kCntStatus];
            a.frame[0] = a.dcount[0];
            a.frame[1] = keys;
            a.frame[2] = a.dcount[4];
            a.frame[3] = status;
            const int64_t mon[kMonitor] = {a.mon[0] + 1, a.mon[1] > keys ? a.mon[1] : keys,
                                           a.mon[2] + (status != kFrameOk ? 1 : 0), keys,
                                           a.dcount[kErrSlot] & 0xffffffffll};
#pragma unroll
            for (int k = 0; k < kMonitor; ++k) {
                a.mon[k] = mon[k];
                __hip_atomic_store(a.mon_host + k, mon[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
    }
    int64_t end = a.tiles_end[tile - 1];
    int64_t beg = tile == 1 ? 0 : a.tiles_end[tile - 2];
    if (end > m) end = m;
    if (beg < 0) beg = 0;
    if (beg > end) beg = end;

    float T = 1.0f, C0 = 0.0f, C1 = 0.0f, C2 = 0.0f, D = 0.0f;
    int32_t last = 0;
    bool done = !on;
    unsigned long long evals = 0, live_n = 0, contrib_n = 0;
    // blend_batch runs records in groups of four: up to three records after a batch are padding
    // that no pixel is live for (exponent -inf), written where a batch ends
    for (int k = t; k < 3; k += NT) blend_pad(s_rec + NT + k);   // (tiles of fewer than 3 pixels too)
    for (int64_t base = beg; base < end; base += NT) {
        if (__syncthreads_count(done ? 0 : 1) == 0) break;
        const int64_t s = base + t;
        bool big = false;   // opacity above 1e38: exponents may pass 88
        if (s >= end && s < end + 3) blend_pad(s_rec + t);
        if (s < end) {
            const int64_t f = (int64_t)a.sorted_f[s] - 1;
            const float* r = a.f2d + 9 * f;
            float p[6];
            blend_params(r[0], r[1], r[2], r[3], r[4], r[5], u0, v0, p);
            BlendRec rec;
            rec.a = make_float4(p[0], p[1], p[2], p[3]);
            rec.b = make_float4(p[4], p[5], RGB ? r[6] : 0.0f, RGB ? r[7] : 0.0f);
            rec.c = make_float4(RGB ? r[8] : 0.0f, DEPTH ? a.depths[f] : 0.0f, 0.0f, 0.0f);
            s_rec[t] = rec;
            big = !(r[2] <= 1e38f);
        }
        // A live exponent lies in [e_cut, log a]; unless e_cut < -87 or an opacity in the
        // batch is huge (or NaN), that is inside [-87, 88], where exp_f is its polynomial core.
        const bool checked = __syncthreads_or(big) || a.cut_low;
        const int nb = (int)((end - base) < NT ? (end - base) : NT);
        if (!COUNT && !checked) {
            if (!done) {
                const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) BlendRec*)s_rec;
                const uint64_t act = blend_batch<DEPTH, LAST>(lds, (int32_t)(base + 1), (int32_t)(base + nb + 1), uu,
                                                        vv, uv, cu, cv, a.e_cut, a.max_alpha, a.min_alpha,
                                                        a.min_T, T, C0, C1, C2, D, last);
                done = ((act >> __lane_id()) & 1ull) == 0;
            }
        } else if (!done) {
            for (int j = 0; j < nb; ++j) {
                if (COUNT && !done) ++evals;
                const float4 ra = s_rec[j].a;
                const float4 rb = s_rec[j].b;
                const float e = fmaf(ra.x, uu, fmaf(ra.y, vv, fmaf(ra.z, uv, fmaf(ra.w, cu, fmaf(rb.x, cv, rb.y)))));
                const bool live = !done && !(e < a.e_cut);
                if (!wave_any(live)) continue;
                // exp_f(e) for the live lanes: the polynomial core unless a live lane is outside
                // [-87, 88] or NaN (the other lanes' values are not used)
                const float ex = (checked && wave_any(live && !(e >= -87.0f && e <= 88.0f))) ? exp_f_sel(e)
                                                                                            : exp_f_core(e);
                // min(ex, max_alpha); equal to the select ex < max_alpha ? ex : max_alpha for a
                // non-NaN max_alpha, NaN ex included
                const float alpha = __builtin_fminf(ex, a.max_alpha);
                const bool contrib = live && !(alpha < a.min_alpha);
                if (COUNT) {
                    live_n += live ? 1 : 0;
                    contrib_n += contrib ? 1 : 0;
                }
                const float Tn = T * (1.0f - alpha);
                const bool stop = contrib && Tn < a.min_T;
                if (contrib && !stop) {
                    const float w = T * alpha;
                    if (RGB || DEPTH) {
                        const float4 rc = s_rec[j].c;
                        if (RGB) {
                            C0 = fmaf(w, rb.z, C0);
                            C1 = fmaf(w, rb.w, C1);
                            C2 = fmaf(w, rc.x, C2);
                        }
                        if (DEPTH) D = fmaf(w, rc.y, D);
                    }
                    T = Tn;
                    last = (int32_t)(base + j + 1);
                }
                if (wave_any(stop)) {
                    done = done || stop;
                    if (!wave_any(!done)) break;
                }
            }
        }
    }
    if (COUNT) {
        for (int d = 32; d >= 1; d >>= 1) {
            evals += __shfl_xor(evals, d, kWave);
            live_n += __shfl_xor(live_n, d, kWave);
            contrib_n += __shfl_xor(contrib_n, d, kWave);
        }
        if (__lane_id() == 0) {
            atomicAdd(a.evaluations, evals);
            atomicAdd(a.evaluations + 1, live_n);
            atomicAdd(a.evaluations + 2, contrib_n);
        }
        return;
    }
    if (!on) return;
    const int64_t px = (int64_t)(V - 1) + (int64_t)a.H * (U - 1);
    if (RGB && a.rgb) {
        a.rgb[3 * px] = fmaf(T, a.bg0, C0);
        a.rgb[3 * px + 1] = fmaf(T, a.bg1, C1);
        a.rgb[3 * px + 2] = fmaf(T, a.bg2, C2);
    }
    if (a.T) a.T[px] = T;
    if (DEPTH && a.depth) a.depth[px] = nothing ? kInf : D;
    if (a.last) a.last[px] = last;
}

// render_void! (forward_structs.jl:743-757).
__global__ void k_render_void(int64_t npx, float bg0, float bg1, float bg2, float* rgb, float* T,
                              float* depth, int32_t* last) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npx) return;
    if (rgb) {
        rgb[3 * i] = bg0;
        rgb[3 * i + 1] = bg1;
        rgb[3 * i + 2] = bg2;
    }
    if (T) T[i] = 1.0f;
    if (depth) depth[i] = kInf;
    if (last) last[i] = 0;
}

static int launch_render_void(hipStream_t s, const tdgs_camera* cam, const tdgs_render_options* o,
                              const tdgs_render_outputs* out) {
    const int64_t npx = (int64_t)cam->width * cam->height;
    k_render_void<<<(unsigned)ceil_div(npx, 256), 256, 0, s>>>(npx, o->background[0], o->background[1],
                                                               o->background[2], out->rgb, out->T,
                                                               out->depth, out->last);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

static int launch_render_tiles(hipStream_t s, const tdgs_camera* cam, const tdgs_tiling* t,
                               const tdgs_render_options* o, int64_t m, const int32_t* tiles_end,
                               const int32_t* sorted_f, const float* f2d, const float* depths,
                               const tdgs_render_outputs* out, unsigned long long* evaluations = nullptr,
                               const int64_t* dcount = nullptr, int64_t* frame = nullptr,
                               int64_t* mon = nullptr, int64_t* mon_host = nullptr) {
    BlendArgs a;
    a.W = cam->width; a.H = cam->height; a.TW = t->tile_width; a.TH = t->tile_height;
    a.ntx = t->nb_tiles_x;
    a.bg0 = o->background[0]; a.bg1 = o->background[1]; a.bg2 = o->background[2];
    a.min_alpha = o->min_alpha; a.max_alpha = o->max_alpha; a.min_T = o->min_transmittance;
    a.e_cut = exponent_cut(o->min_alpha);
    a.cut_low = !(a.e_cut >= -87.0f);
    a.m = m; a.tiles_end = tiles_end; a.sorted_f = sorted_f; a.f2d = f2d; a.depths = depths;
    a.rgb = out->rgb; a.T = out->T; a.depth = out->depth; a.last = out->last;
    a.evaluations = evaluations;
    a.dcount = dcount;
    a.frame = frame;
    a.mon = mon;
    a.mon_host = mon_host;
    const int nt = t->tile_width * t->tile_height;
    const dim3 grid(t->nb_tiles_x, t->nb_tiles_y);
    // + the padding after a batch and the record blend_batch reads past its last group of four
    const size_t lds = (size_t)(nt + 4) * sizeof(BlendRec);
    if (evaluations) {
        k_render_tiles<false, false, true><<<grid, nt, lds, s>>>(a);
        TDGS_LAUNCHED();
        return TDGS_OK;
    }
    const bool rgb = out->rgb != nullptr, dep = out->depth != nullptr;
    const bool last = out->last != nullptr;
    if (rgb && dep) {
        if (last) k_render_tiles<true, true, false, true><<<grid, nt, lds, s>>>(a);
        else k_render_tiles<true, true, false, false><<<grid, nt, lds, s>>>(a);
    } else if (rgb) {
        if (last) k_render_tiles<true, false, false, true><<<grid, nt, lds, s>>>(a);
        else k_render_tiles<true, false, false, false><<<grid, nt, lds, s>>>(a);
    } else if (dep) {
        if (last) k_render_tiles<false, true, false, true><<<grid, nt, lds, s>>>(a);
        else k_render_tiles<false, true, false, false><<<grid, nt, lds, s>>>(a);
    } else {
        if (last) k_render_tiles<false, false, false, true><<<grid, nt, lds, s>>>(a);
        else k_render_tiles<false, false, false, false><<<grid, nt, lds, s>>>(a);
    }
    TDGS_LAUNCHED();
    return TDGS_OK;
}

static int end_bit_of(const tdgs_tiling* t) {
    const int64_t nt = (int64_t)t->nb_tiles_x * t->nb_tiles_y;
    int fl = 0;
    while ((2ll << fl) <= nt) ++fl;  // floor(log2(nt))
    return 33 + fl;
}

// Scratch layout of tdgs_render.
// Items of the largest scan: the Gaussians, or the tiles (tile lists).
static int64_t scan_items(int64_t cap, const tdgs_tiling* t) {
    const int64_t nt = t ? (int64_t)t->nb_tiles_x * t->nb_tiles_y : 0;
    return cap > nt ? cap : nt;
}
// The frame's zeroed scratch (cleared by k_keep_counts): the depth sort's group sums (when
// grouped), the emission pass's group sums (when grouped: decided by the key capacity) and
// the count scan's tile sums (int64, accumulated by the depth sort's last pass).
static int64_t depth_group_words(int64_t cap) {
    return radix_tiles<uint32_t>(cap) <= kRsMaxGroupedTiles ? radix_group_words<uint32_t>(cap, 0, 32) : 0;
}
static int64_t emit_group_words(int64_t key_cap) {
    const int64_t tiles = radix_tiles<uint16_t>(key_cap);
    return tiles <= kRsMaxGroupedTiles ? rs_groups(tiles) * kRsBins : 0;
}
static_assert(kScanTile == (1 << kRsSumShift), "the depth sort sums the count scan's tiles");
static int64_t zero_words(int64_t cap, int64_t key_cap) {
    return (depth_group_words(cap) + emit_group_words(key_cap) + 2 * ceil_div(cap > 0 ? cap : 1, kScanTile) + 3) /
           4 * 4;
}
static int64_t rect_diff_size(const tdgs_tiling* t) {
    return t ? (int64_t)(t->nb_tiles_x + 1) * (t->nb_tiles_y + 1) : 0;
}

template <class A>
static void render_layout(A& ar, int64_t cap, int64_t key_cap, const tdgs_tiling* t) {
    ar.template take<int64_t>(kCounters);                 // unused slot (alignment)
    ar.template take<uint32_t>(cap);                      // depth keys
    ar.template take<uint32_t>(cap);                      // depth keys, ping-pong
    ar.template take<uint32_t>(cap);                      // depth keys, sorted
    ar.template take<int32_t>(cap);                       // depth values
    ar.template take<int32_t>(cap);                       // depth values, ping-pong
    ar.template take<int32_t>(cap);                       // depth values, sorted (fgidx)
    ar.template take<int32_t>(cap);                       // counts scan in depth order
    ar.template take<char>((int64_t)scan_temp_bytes_for(scan_items(cap, t)));
    ar.template take<int32_t>(ceil_div(cap, kProjThreads * kKeepSub) * kKeepSub);   // keep counts per block
    ar.template take<int32_t>(ceil_div(cap, kProjThreads * kKeepSub));   // and per kKeepSub blocks
    const int64_t big = cap > key_cap ? cap : key_cap;
    ar.template take<char>((int64_t)radix_temp_bytes(big));
    ar.template take<int32_t>(kRectCopies * rect_diff_size(t));   // tile-coverage difference arrays
    ar.template take<int32_t>(ceil_div(key_cap, kEmitTile) + 2);  // first Gaussian of each emission block
    ar.template take<int32_t>(t ? bin_table_entries(key_cap, bin_geom(t)) : 0);   // per (segment, tile)
    ar.template take<int32_t>(t ? bin_geom(t).nblocks() : 0);                    // ends of the blocks' lists
    ar.template take<int32_t>(t ? ((int64_t)t->nb_tiles_x * t->nb_tiles_y + 3) / 4 * 4 : 0);   // tiles' totals
    ar.template take<int4>(cap);                                                  // rectangles in depth order
    ar.template take<uint32_t>(zero_words(cap, key_cap));                         // zeroed each frame
    ar.template take<uint32_t>(kDsBuckets + 1);                                   // bucket starts
    ar.template take<uint32_t>(kDsSample);                                        // sampled keys
    ar.template take<uint8_t>(cap);                                               // bucket ids
    ar.template take<uint64_t>(cap);                                              // bucket pass output
    ar.template take<int32_t>(cap);
    ar.template take<uint64_t>(cap);                                              // and its ping-pong partner
    ar.template take<int32_t>(cap);
}

// The scratch arrays of tdgs_render / tdgs_project inside buf->temp (render_layout's order).
struct RenderScratch {
    uint32_t *dkey, *dkey_alt, *dkey_sorted;
    int32_t *dval, *dval_alt, *sorted_f, *cs;
    void* stemp;
    size_t sbytes;
    int32_t *block_counts, *group_counts;
    void* rtemp;
    size_t rbytes;
    int32_t* rect_diff;
    int64_t ndiff;
    int32_t* blk_first;
    int64_t nblk;
    int32_t* tile_counts;
    int32_t* block_end;
    int32_t* tile_totals;
    int64_t ntt;   // entries of tile_totals (tiles, padded to 4)
    int4* srect;   // tile rectangles of the non-empty Gaussians in depth order
    uint32_t* zero;   // the frame's zeroed scratch: dgrp, egrp, scan_sums
    int64_t nzero;
    uint32_t* dgrp;   // depth sort group sums (ndgrp words; 0: the sort is not grouped)
    int64_t ndgrp;
    uint32_t* egrp;   // emission pass group sums (negrp words; 0: not grouped)
    int64_t negrp;
    int64_t* scan_sums;   // count scan tile sums (kScanTile items each)
    DsScratch ds;         // the bucketed depth presort
};

static RenderScratch carve_render_scratch(const tdgs_render_buffers* buf, const tdgs_tiling* tiling) {
    RenderScratch r;
    const int64_t cap = buf->capacity;
    Arena ar(buf->temp, buf->temp_bytes);
    ar.take<int64_t>(kCounters);
    r.dkey = ar.take<uint32_t>(cap);
    r.dkey_alt = ar.take<uint32_t>(cap);
    r.dkey_sorted = ar.take<uint32_t>(cap);
    r.dval = ar.take<int32_t>(cap);
    r.dval_alt = ar.take<int32_t>(cap);
    r.sorted_f = ar.take<int32_t>(cap);
    r.cs = ar.take<int32_t>(cap);
    r.sbytes = scan_temp_bytes_for(scan_items(cap, tiling));
    r.stemp = ar.take<char>((int64_t)r.sbytes);
    r.block_counts = ar.take<int32_t>(ceil_div(cap, kProjThreads * kKeepSub) * kKeepSub);
    r.group_counts = ar.take<int32_t>(ceil_div(cap, kProjThreads * kKeepSub));
    const int64_t big = cap > buf->key_capacity ? cap : buf->key_capacity;
    r.rbytes = radix_temp_bytes(big);
    r.rtemp = ar.take<char>((int64_t)r.rbytes);
    r.ndiff = rect_diff_size(tiling);
    r.rect_diff = ar.take<int32_t>(kRectCopies * r.ndiff);
    r.nblk = ceil_div(buf->key_capacity, kEmitTile) + 2;
    r.blk_first = ar.take<int32_t>(r.nblk);
    r.tile_counts = ar.take<int32_t>(
        tiling ? bin_table_entries(buf->key_capacity, bin_geom(tiling)) : 0);
    r.block_end = ar.take<int32_t>(tiling ? bin_geom(tiling).nblocks() : 0);
    r.ntt = tiling ? ((int64_t)tiling->nb_tiles_x * tiling->nb_tiles_y + 3) / 4 * 4 : 0;
    r.tile_totals = ar.take<int32_t>(r.ntt);
    r.srect = ar.take<int4>(cap);
    r.nzero = zero_words(cap, buf->key_capacity);
    r.zero = ar.take<uint32_t>(r.nzero);
    r.dgrp = r.zero;
    r.ndgrp = depth_group_words(cap);
    r.egrp = r.dgrp + r.ndgrp;
    r.negrp = emit_group_words(buf->key_capacity);
    r.scan_sums = reinterpret_cast<int64_t*>(r.egrp + r.negrp);
    r.ds.bstart = ar.take<uint32_t>(kDsBuckets + 1);
    r.ds.sample = ar.take<uint32_t>(kDsSample);
    r.ds.bid = ar.take<uint8_t>(cap);
    r.ds.bkey = ar.take<uint64_t>(cap);
    r.ds.bval = ar.take<int32_t>(cap);
    r.ds.akey = ar.take<uint64_t>(cap);
    r.ds.aval = ar.take<int32_t>(cap);
    return r;
}

// Arguments shared by tdgs_render and tdgs_project.
static int check_render_args(const tdgs_gaussians* g, const tdgs_camera* cam, const tdgs_tiling* tiling,
                             const tdgs_render_options* opt, const tdgs_render_buffers* buf) {
    TDGS_TRY(check_gaussians(g, false));
    TDGS_TRY(check_tiling(tiling, cam));
    TDGS_TRY(check_options(opt, g->sh_degree));
    TDGS_REQUIRE(cam->near_z >= 0.0f, "near clipping plane must be >= 0 (got %g)", (double)cam->near_z);
    TDGS_REQUIRE(buf->capacity >= g->n, "render buffers hold %d Gaussians, need %d", buf->capacity, g->n);
    if (g->n == 0) return TDGS_OK;
    TDGS_REQUIRE(buf->fgidx_to_gidx && buf->depths && buf->f2d && buf->tile_ranges && buf->counts &&
                     buf->tiles_end && buf->temp,
                 "null render buffers");
    TDGS_REQUIRE(((uintptr_t)buf->f2d & 15) == 0 && ((uintptr_t)buf->tile_ranges & 15) == 0,
                 "render buffers: f2d and tile_ranges must be 16-byte aligned");
    const size_t need = tdgs_render_temp_bytes(buf->capacity, buf->key_capacity, tiling);
    if (buf->temp_bytes < need) {
        set_error("render scratch too small: need %zu bytes, have %zu", need, buf->temp_bytes);
        return TDGS_ERR_CAPACITY;
    }
    return TDGS_OK;
}

// Steps 1-3 of the pipeline: keep counts, then compaction + projection (N_f into d_nbf).
// depth_keys / depth_vals (may be null) receive the depth presort's input.
static int launch_keep_and_project(hipStream_t s, const tdgs_gaussians* g, const tdgs_camera* cam,
                                   const tdgs_tiling* tiling, const tdgs_render_options* opt,
                                   const tdgs_render_buffers* buf, const RenderScratch& r, int64_t* d_nbf,
                                   uint32_t* depth_keys, int32_t* depth_vals) {
    const int64_t n = g->n;
    const int64_t nblocks = ceil_div(n, kProjThreads);
    const int64_t ngroups = ceil_div(nblocks, kKeepSub);
    {
        StageScope sc(TDGS_STAGE_CULL_COMPACT, s);
        KeepEval ev{g->means_opacity, g->kind, *cam, *opt, buf->keep};
        k_keep_counts<<<(unsigned)ngroups, 256, 0, s>>>(ev, n, r.block_counts, r.group_counts, nblocks, r.zero,
                                                         r.nzero);
        TDGS_LAUNCHED();
    }
    ProjectArgs pa;
    pa.g = *g; pa.cam = *cam; pa.tiling = *tiling; pa.opt = *opt;
    pa.block_counts = r.block_counts; pa.group_counts = r.group_counts; pa.ngroups = ngroups; pa.d_nbf = d_nbf;
    pa.fgidx_to_gidx = buf->fgidx_to_gidx; pa.depths = buf->depths; pa.f2d = buf->f2d;
    pa.ranges = buf->tile_ranges; pa.counts = buf->counts;
    pa.depth_keys = depth_keys; pa.depth_vals = depth_vals;
    pa.depth_sample = depth_keys && ds_applicable(n, r.ndgrp) ? r.ds.sample : nullptr;
    StageScope sc(TDGS_STAGE_PROJECT, s);
    if (g->kind == TDGS_TRAINABLE)
        k_project<TDGS_TRAINABLE><<<(unsigned)nblocks, kProjThreads, 0, s>>>(pa);
    else
        k_project<TDGS_RENDER_ONLY><<<(unsigned)nblocks, kProjThreads, 0, s>>>(pa);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

}  // namespace tdgs

using namespace tdgs;

// Steps 6-8 for at most 65535 tiles: the coarse blocks' lists (emission of one block id per
// (Gaussian, block touched) in depth order, fused with the first stable radix pass on the
// ids; usually the only pass), their ends, then the tile lists (count, scan, write).
// Synchronous: nb, mc (entries) and m (keys) are the host's counts. With device counts
// (dc not null) the launches are sized by the key capacity, k_emit_count decides on the device
// whether the keys fit, and every kernel reads the entry count it uses from dc.
static int bin_tile_lists(hipStream_t s, const tdgs_tiling* tiling, tdgs_render_buffers* buf,
                          const RenderScratch& r, int64_t nb, int64_t mc, int64_t m, int64_t* dc,
                          uint32_t* d_err) {
    const BinGeom bg = bin_geom(tiling);
    const int32_t nblocks = bg.nblocks();
    int cbits = 0;   // bits of the 1-based block ids
    while ((1ll << cbits) <= nblocks) ++cbits;
    const int passes = radix_passes(0, cbits);
    const int nbits0 = radix_digit_bits(0, cbits);
    const bool one_pass = passes == 1;
    const int64_t kc = buf->key_capacity;
    const int64_t mb = dc ? kc : mc;   // launch bound of the entries
    uint16_t* c16 = reinterpret_cast<uint16_t*>(buf->keys);
    uint16_t* c16_alt = c16 + kc;
    // with one pass the entries' block masks are sorted along, into the keys array's second
    // half (the 16-bit ids take its first): the binning then reads no rectangles
    uint32_t* cmask = one_pass ? reinterpret_cast<uint32_t*>(buf->keys) + kc : nullptr;
    const EmitGrid cg{bg.nbx, bg.sx, bg.sy};
    // (with device counts the blocks are bounded by the key capacity; a capped grid walks them)
    constexpr int64_t kEmitMaxGrid = 4096;
    const int64_t eblocks = ceil_div(mb, kEmitTile);
    const unsigned egrid = (unsigned)(dc && eblocks > kEmitMaxGrid ? kEmitMaxGrid : eblocks);
    const int64_t count_tiles = radix_tiles<uint16_t>(mb);
    uint32_t* table = radix_count_table(r.rtemp);
    uint32_t* totals = radix_totals(r.rtemp, mb);
    const int64_t* d_used = dc ? dc + kCntCoarseUsed : nullptr;
    // group sums (cleared at frame start) replace the row scan when the capacity allows
    uint32_t* grp = r.negrp > 0 && count_tiles <= kRsMaxGroupedTiles ? r.egrp : nullptr;
    {
        StageScope sc(TDGS_STAGE_EMIT, s);
        if ((int64_t)egrid < eblocks)
            k_emit_count<true><<<egrid, kEmitSortThreads, 0, s>>>(nb, mc, r.sorted_f, r.cs, r.blk_first, r.srect, cg,
                                                                  nbits0, table, count_tiles, grp, dc, kc,
                                                                  one_pass ? r.tile_totals : nullptr, one_pass ? r.ntt : 0);
        else
            k_emit_count<false><<<egrid, kEmitSortThreads, 0, s>>>(nb, mc, r.sorted_f, r.cs, r.blk_first, r.srect, cg,
                                                                   nbits0, table, count_tiles, grp, dc, kc,
                                                                   one_pass ? r.tile_totals : nullptr,
                                                                   one_pass ? r.ntt : 0);
        TDGS_LAUNCHED();
    }
    {
        StageScope sc(TDGS_STAGE_TILE_SORT, s);
        if (!grp) {
            k_rs_scan_rows<<<kRsBins, 256, 0, s>>>(table, count_tiles, totals, d_used, kEmitTile);
            TDGS_LAUNCHED();
        }
        // (with one pass the sorted block ids are not written: the block ends come from the
        // digit totals)
        uint16_t* ek = one_pass ? nullptr : c16_alt;
        int32_t* ev = one_pass ? buf->values : buf->sorted_values;
        if ((int64_t)egrid < eblocks) {
            if (cmask)
                k_emit_scatter<true, true><<<egrid, kEmitSortThreads, 0, s>>>(
                    nb, mc, r.sorted_f, r.cs, r.blk_first, r.srect, cg, nbits0, table, totals, count_tiles, grp, ek, ev,
                    cmask, d_err, dc);
            else
                k_emit_scatter<true, false><<<egrid, kEmitSortThreads, 0, s>>>(
                    nb, mc, r.sorted_f, r.cs, r.blk_first, r.srect, cg, nbits0, table, totals, count_tiles, grp, ek, ev,
                    nullptr, d_err, dc);
        } else {
            if (cmask)
                k_emit_scatter<false, true><<<egrid, kEmitSortThreads, 0, s>>>(
                    nb, mc, r.sorted_f, r.cs, r.blk_first, r.srect, cg, nbits0, table, totals, count_tiles, grp, ek, ev,
                    cmask, d_err, dc);
            else
                k_emit_scatter<false, false><<<egrid, kEmitSortThreads, 0, s>>>(
                    nb, mc, r.sorted_f, r.cs, r.blk_first, r.srect, cg, nbits0, table, totals, count_tiles, grp, ek, ev,
                    nullptr, d_err, dc);
        }
        TDGS_LAUNCHED();
        if (!one_pass)
            TDGS_TRY(radix_sort_pairs<uint16_t>(c16_alt, c16, buf->sorted_values, buf->values, c16_alt,
                                                buf->sorted_values, mb, nbits0, cbits, r.rtemp, r.rbytes, s, nullptr,
                                                d_err, nullptr, d_used));
    }
    StageScope sc(TDGS_STAGE_TILE_RANGES, s);
    if (!one_pass) {
        // ends of the blocks' runs (with one pass they are the prefix sums of its digit totals)
        const int64_t rthreads = ceil_div(mb, 8) > nblocks ? ceil_div(mb, 8) : nblocks;
        k_tile_ranges16<<<(unsigned)ceil_div(rthreads, 256), 256, 0, s>>>(mb, c16, nblocks, r.block_end, d_used,
                                                                          r.tile_totals, r.ntt);
        TDGS_LAUNCHED();
    }
    // the tile lists
    BinArgs ba;
    ba.ntx = tiling->nb_tiles_x; ba.nty = tiling->nb_tiles_y; ba.nbx = bg.nbx; ba.sy = bg.sy;
    ba.nblocks = nblocks;
    ba.cvals = buf->values; ba.cend = r.block_end; ba.mc = mb; ba.dmc = d_used;
    ba.totals = one_pass ? totals : nullptr;
    ba.ranges = buf->tile_ranges; ba.cmask = cmask; ba.table = r.tile_counts; ba.tile_totals = r.tile_totals;
    ba.tiles_end = buf->tiles_end;
    ba.out = buf->sorted_values; ba.cap = (int32_t)(kc < INT32_MAX ? kc : INT32_MAX); ba.err = d_err;
    const unsigned bthreads = 4u << (bg.sx + bg.sy);
    const int per = bin_per(bg.sx);
    const int64_t nchunks = ceil_div(mb > 0 ? mb : 1, (int64_t)bthreads * per);
    const unsigned bgrid = (unsigned)(nchunks < kBinMaxGrid ? nchunks : kBinMaxGrid);
    const size_t lds = (size_t)bthreads * per * 2 * sizeof(uint32_t);
    if (bg.sx == 3) k_bin_tiles<3, false><<<bgrid, bthreads, lds, s>>>(ba);
    else k_bin_tiles<4, false><<<bgrid, bthreads, lds, s>>>(ba);
    TDGS_LAUNCHED();
    k_bin_scan<<<1, 1024, 0, s>>>(r.tile_totals, tiling->nb_tiles_x * tiling->nb_tiles_y, buf->tiles_end,
                                  dc ? dc + kCntKeysUsed : nullptr, m, d_err);
    TDGS_LAUNCHED();
    if (bg.sx == 3) k_bin_tiles<3, true><<<bgrid, bthreads, lds, s>>>(ba);
    else k_bin_tiles<4, true><<<bgrid, bthreads, lds, s>>>(ba);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

extern "C" {

int tdgs_project(tdgs_ctx* ctx, void* stream, const tdgs_gaussians* g, const tdgs_camera* cam,
                 const tdgs_tiling* tiling, const tdgs_render_options* opt, tdgs_render_buffers* buf,
                 int32_t* nb_fgaussians_out) {
    TDGS_REQUIRE(ctx && buf && nb_fgaussians_out, "null arguments");
    TDGS_TRY(check_render_args(g, cam, tiling, opt, buf));
    *nb_fgaussians_out = 0;
    if (g->n == 0) return TDGS_OK;
    hipStream_t s = (hipStream_t)stream;
    const RenderScratch r = carve_render_scratch(buf, tiling);
    TDGS_TRY(launch_keep_and_project(s, g, cam, tiling, opt, buf, r, ctx->d_counters, nullptr, nullptr));
    TDGS_TRY(read_counters(ctx, s));
    *nb_fgaussians_out = (int32_t)ctx->h_counters[0];
    return TDGS_OK;
}

int tdgs_fill_keep(void* stream, const tdgs_gaussians* g, const tdgs_camera* cam,
                   const tdgs_render_options* opt, uint8_t* keep) {
    TDGS_TRY(check_gaussians(g, false));
    TDGS_TRY(check_options(opt, g->sh_degree));
    TDGS_REQUIRE(cam && (keep || g->n == 0), "null camera or keep");
    if (g->n == 0) return TDGS_OK;
    KeepEval ev{g->means_opacity, g->kind, *cam, *opt, keep};
    k_fill_keep<<<(unsigned)ceil_div(g->n, 256), 256, 0, (hipStream_t)stream>>>(ev, g->n);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

size_t tdgs_scan_temp_bytes(int64_t n) { return scan_temp_bytes_for(n); }

int tdgs_fill_fgidx_to_gidx(tdgs_ctx* ctx, void* stream, const uint8_t* keep, int32_t n,
                            int32_t* keep_cs, int32_t* fgidx_to_gidx, void* temp, size_t temp_bytes,
                            int32_t* nb_fgaussians_out) {
    TDGS_REQUIRE(ctx && nb_fgaussians_out, "null ctx or output");
    TDGS_REQUIRE(n >= 0, "negative n");
    if (n == 0) { *nb_fgaussians_out = 0; return TDGS_OK; }
    TDGS_REQUIRE(keep && fgidx_to_gidx, "null keep or fgidx_to_gidx");
    hipStream_t s = (hipStream_t)stream;
    TDGS_TRY(device_scan(ItemsU8{keep}, ItemsU8{keep}, CompactOut{fgidx_to_gidx, keep_cs}, n, temp,
                         temp_bytes, ctx->d_counters, s));
    TDGS_TRY(read_counters(ctx, s));
    *nb_fgaussians_out = (int32_t)ctx->h_counters[0];
    return TDGS_OK;
}

int tdgs_scan_counts(tdgs_ctx* ctx, void* stream, const int32_t* counts, int32_t n, int32_t* counts_cs,
                     void* temp, size_t temp_bytes, int64_t* total_out) {
    TDGS_REQUIRE(ctx && total_out, "null ctx or output");
    TDGS_REQUIRE(n >= 0, "negative n");
    if (n == 0) { *total_out = 0; return TDGS_OK; }
    TDGS_REQUIRE(counts && counts_cs, "null arrays");
    hipStream_t s = (hipStream_t)stream;
    TDGS_TRY(device_scan(ItemsI32{counts}, ItemsI32{counts}, WriteInclusiveI32{counts_cs}, n, temp,
                         temp_bytes, ctx->d_counters, s));
    TDGS_TRY(read_counters(ctx, s));
    *total_out = ctx->h_counters[0];
    if (*total_out >= (int64_t)INT32_MAX) {
        set_error("%lld duplicated keys exceed the int32 index range", (long long)*total_out);
        return TDGS_ERR_CAPACITY;
    }
    return TDGS_OK;
}

int tdgs_scan_counts_noalloc(void* stream, const int32_t* counts, int32_t n, int32_t* counts_cs,
                             int64_t* total_dev) {
    TDGS_REQUIRE(n >= 0 && n <= TDGS_SCAN_NOALLOC_MAX_ITEMS, "%d items: the allocation-free scan takes at most %d",
                 n, TDGS_SCAN_NOALLOC_MAX_ITEMS);
    TDGS_REQUIRE(total_dev && (n == 0 || (counts && counts_cs)), "null arrays");
    int64_t* tile_sums = nullptr;
    TDGS_TRY(noalloc_scratch(&tile_sums));
    hipStream_t s = (hipStream_t)stream;
    // n == 0 still runs the one-block total pass so that *total_dev is written (0), in order
    const int64_t nn = n > 0 ? n : 1;
    TDGS_TRY(device_scan(ItemsI32Bounded{counts, n}, ItemsI32Bounded{counts, n}, WriteInclusiveI32Bounded{counts_cs, n},
                         nn, tile_sums, sizeof(int64_t) * kNoAllocScanTiles, total_dev, s));
    return TDGS_OK;
}

int tdgs_emit_keys(void* stream, int32_t nb_fgaussians, const float* depths, const int32_t* tile_ranges,
                   const int32_t* counts_cs, const tdgs_tiling* tiling, int64_t* keys, int32_t* values) {
    TDGS_REQUIRE(nb_fgaussians >= 0 && tiling, "bad arguments");
    if (nb_fgaussians == 0) return TDGS_OK;
    TDGS_REQUIRE(depths && tile_ranges && counts_cs && keys && values, "null arrays");
    k_emit_keys<<<(unsigned)ceil_div(nb_fgaussians, 256), 256, 0, (hipStream_t)stream>>>(
        nb_fgaussians, depths, tile_ranges, counts_cs, tiling->nb_tiles_x, keys, values);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

size_t tdgs_sort_pairs_temp_bytes(int32_t n, int32_t end_bit) {
    (void)end_bit;
    const int64_t nn = n > 0 ? n : 1;
    return align_up((size_t)nn * sizeof(int64_t)) + align_up((size_t)nn * sizeof(int32_t)) +
           radix_temp_bytes(nn);
}

int tdgs_sort_pairs(void* temp, size_t temp_bytes, const int64_t* keys_in, int64_t* keys_out,
                    const int32_t* values_in, int32_t* values_out, int32_t n, int32_t end_bit,
                    void* stream) {
    TDGS_REQUIRE(n >= 0 && end_bit >= 0 && end_bit <= 64, "bad n or end_bit");
    if (n == 0) return TDGS_OK;
    TDGS_REQUIRE(keys_in && keys_out && values_in && values_out && temp, "null arrays");
    TDGS_REQUIRE(keys_in != keys_out && values_in != values_out, "sort_pairs is not in place");
    TDGS_REQUIRE(temp_bytes >= tdgs_sort_pairs_temp_bytes(n, end_bit), "sort scratch too small");
    Arena ar(temp, temp_bytes);
    uint64_t* alt_k = ar.take<uint64_t>(n);
    int32_t* alt_v = ar.take<int32_t>(n);
    const size_t rb = radix_temp_bytes(n);
    void* rtemp = ar.take<char>((int64_t)rb);
    return radix_sort_pairs<uint64_t>((const uint64_t*)keys_in, (uint64_t*)keys_out, values_in, values_out,
                                      alt_k, alt_v, n, 0, end_bit, rtemp, rb, (hipStream_t)stream);
}

int tdgs_tile_ranges(void* stream, int64_t nb_keys, const int64_t* sorted_keys, int32_t nb_tiles,
                     int32_t* tiles_end) {
    TDGS_REQUIRE(nb_keys >= 0 && nb_tiles > 0 && tiles_end, "bad arguments");
    if (nb_keys == 0) return TDGS_OK;
    TDGS_REQUIRE(sorted_keys, "null keys");
    k_tile_ranges<int64_t><<<(unsigned)ceil_div(nb_keys, 256), 256, 0, (hipStream_t)stream>>>(nb_keys, sorted_keys,
                                                                                               nb_tiles, tiles_end);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_render_counts(void* stream, const tdgs_render_buffers* buf, int64_t* counts_out) {
    TDGS_REQUIRE(buf && buf->temp && buf->temp_bytes >= 4 * sizeof(int64_t) && counts_out, "null arguments");
    hipStream_t s = (hipStream_t)stream;
    TDGS_HIP(hipMemcpyAsync(counts_out, frame_counts(buf), 4 * sizeof(int64_t), hipMemcpyDeviceToHost, s));
    TDGS_HIP(hipStreamSynchronize(s));
    return TDGS_OK;
}

int tdgs_render_sorted_keys(void* stream, const tdgs_tiling* tiling, const tdgs_render_buffers* buf,
                            int64_t nb_keys) {
    TDGS_REQUIRE(tiling && tiling->nb_tiles_x > 0 && tiling->nb_tiles_y > 0, "bad tiling");
    TDGS_REQUIRE(buf && nb_keys >= 0 && nb_keys <= buf->key_capacity, "bad buffers or key count");
    if (nb_keys == 0 || (int64_t)tiling->nb_tiles_x * tiling->nb_tiles_y > 65535) return TDGS_OK;
    TDGS_REQUIRE(buf->tiles_end && buf->sorted_values && buf->sorted_keys && buf->depths, "null buffers");
    k_assemble_keys_te<<<(unsigned)ceil_div(nb_keys, 256), 256, 0, (hipStream_t)stream>>>(
        nb_keys, buf->tiles_end, tiling->nb_tiles_x * tiling->nb_tiles_y, buf->sorted_values, buf->depths,
        buf->sorted_keys);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_render_tiles(void* stream, const tdgs_camera* cam, const tdgs_tiling* tiling,
                      const tdgs_render_options* opt, const tdgs_render_buffers* buf,
                      const tdgs_render_outputs* out) {
    TDGS_TRY(check_tiling(tiling, cam));
    TDGS_REQUIRE(opt && buf && out, "null arguments");
    TDGS_REQUIRE(buf->tiles_end && buf->sorted_values && buf->f2d, "null buffers");
    TDGS_TRY(check_thresholds(opt));
    TDGS_REQUIRE(!out->depth || buf->depths, "depth output needs depths");
    return launch_render_tiles((hipStream_t)stream, cam, tiling, opt, buf->key_capacity, buf->tiles_end,
                               buf->sorted_values, buf->f2d, buf->depths, out);
}

int tdgs_blend_evaluations(void* stream, const tdgs_camera* cam, const tdgs_tiling* tiling,
                           const tdgs_render_options* opt, const tdgs_render_buffers* buf, int64_t nb_keys,
                           uint64_t* evaluations_dev) {
    TDGS_TRY(check_tiling(tiling, cam));
    TDGS_REQUIRE(opt && buf && evaluations_dev && buf->tiles_end && buf->sorted_values && buf->f2d,
                 "null arguments");
    TDGS_REQUIRE(nb_keys >= 0 && nb_keys <= buf->key_capacity, "bad key count");
    TDGS_TRY(check_thresholds(opt));
    tdgs_render_outputs none = {nullptr, nullptr, nullptr, nullptr};
    return launch_render_tiles((hipStream_t)stream, cam, tiling, opt, nb_keys, buf->tiles_end, buf->sorted_values,
                               buf->f2d, buf->depths, &none, (unsigned long long*)evaluations_dev);
}

size_t tdgs_render_temp_bytes(int32_t capacity, int64_t key_capacity, const tdgs_tiling* tiling) {
    (void)tiling;
    ArenaSize sz;
    render_layout(sz, capacity, key_capacity, tiling);
    return sz.used + 256;
}

int tdgs_render(tdgs_ctx* ctx, void* stream, const tdgs_gaussians* g, const tdgs_camera* cam,
                const tdgs_tiling* tiling, const tdgs_render_options* opt, tdgs_render_buffers* buf,
                const tdgs_render_outputs* out, int32_t* nb_fgaussians_out, int64_t* nb_keys_out) {
    TDGS_REQUIRE(ctx && buf && out && nb_fgaussians_out && nb_keys_out, "null arguments");
    TDGS_TRY(check_render_args(g, cam, tiling, opt, buf));
    hipStream_t s = (hipStream_t)stream;
    const bool device_counts = (opt->flags & TDGS_FLAG_DEVICE_COUNTS) != 0;
    *nb_fgaussians_out = device_counts ? -1 : 0;
    *nb_keys_out = device_counts ? -1 : 0;
    const int64_t n = g->n;
    if (device_counts) {
        TDGS_REQUIRE((int64_t)tiling->nb_tiles_x * tiling->nb_tiles_y <= 65535,
                     "device counts need at most 65535 tiles (the tiling has %lld)",
                     (long long)tiling->nb_tiles_x * tiling->nb_tiles_y);
        TDGS_REQUIRE(buf->key_capacity >= 1 && buf->keys && buf->values && buf->sorted_values,
                     "device counts need allocated key arrays");
        if (n == 0) {
            // the frame counts of an empty frame
            static const int64_t zeros[4] = {0, 0, 0, 0};
            TDGS_HIP(hipMemcpyAsync(frame_counts(buf), zeros, sizeof(zeros), hipMemcpyHostToDevice, s));
        }
    }
    if (n == 0) return launch_render_void(s, cam, opt, out);
    const RenderScratch r = carve_render_scratch(buf, tiling);
    uint32_t* dkey = r.dkey;
    uint32_t* dkey_alt = r.dkey_alt;
    uint32_t* dkey_sorted = r.dkey_sorted;
    int32_t* dval = r.dval;
    int32_t* dval_alt = r.dval_alt;
    int32_t* sorted_f = r.sorted_f;
    int32_t* cs = r.cs;
    void* stemp = r.stemp;
    const size_t sbytes = r.sbytes;
    void* rtemp = r.rtemp;
    const size_t rbytes = r.rbytes;
    const int64_t ndiff = r.ndiff;
    int32_t* rect_diff = r.rect_diff;
    const int64_t nblk = r.nblk;
    int32_t* blk_first = r.blk_first;
    int64_t* d_nbf = ctx->d_counters;
    int64_t* d_m = ctx->d_counters + 1;
    uint32_t* d_err = ctx_error_word(ctx);

    const bool tile16 = (int64_t)tiling->nb_tiles_x * tiling->nb_tiles_y <= 65535;

    // 1-3: keep counts, compaction + projection
    TDGS_TRY(launch_keep_and_project(s, g, cam, tiling, opt, buf, r, d_nbf, dkey, dval));
    // 4: the N_b non-empty Gaussians by (depth bits, fgidx); empty and culled ones (all-ones
    // depth key) are dropped. By sampled buckets (dsort.hpp), else (more slots than its grouped
    // tables take) by a 4-pass LSD radix sort whose first pass drops them.
    int64_t* d_nb = ctx->d_counters + 4;
    {
        StageScope sc(TDGS_STAGE_DEPTH_SORT, s);
        // (the output gathers the rectangles into depth order and, for the tile lists, sums
        // their packed tile and block counts per scan tile)
        const BinGeom bg = tile16 ? bin_geom(tiling) : BinGeom{};
        const RsGather gather{reinterpret_cast<const int4*>(buf->tile_ranges), r.srect,
                              tile16 ? r.scan_sums : nullptr, bg.sx, bg.sy};
        if (ds_applicable(n, r.ndgrp))
            TDGS_TRY(depth_sort_buckets(dkey, n, r.ds, radix_count_table(rtemp), r.dgrp, sorted_f, gather, d_err, d_nb,
                                        s));
        else
            TDGS_TRY(radix_sort_pairs_grouped<uint32_t>(dkey, dkey_sorted, dval, sorted_f, dkey_alt, dval_alt, n, 0, 32,
                                                        rtemp, rbytes, r.dgrp, r.ndgrp, s, d_err, d_nb, nullptr,
                                                        gather));
    }
    if (tile16) {
        // 5: tiles and blocks touched, in depth order -> the blocks' entries (emission offsets)
        // and M (the scan's tile sums come from the depth sort)
        const BinGeom bg = bin_geom(tiling);
        {
            StageScope sc(TDGS_STAGE_COUNT_SCAN, s);
            const SortedTileBlockCounts stb{r.srect, bg.sx, bg.sy, d_nb};
            TDGS_TRY(device_scan_apply(stb, WriteBlockScan{WriteScanAndBlocks{cs, blk_first, nblk}}, n, r.scan_sums,
                                       ctx->d_counters + kCntCoarse, s, d_nb));
        }
        if (device_counts) {
            // 6-8 sized by the key capacity; the blend copies the counts to the frame counts
            TDGS_TRY(bin_tile_lists(s, tiling, buf, r, n, buf->key_capacity, 0, ctx->d_counters, d_err));
            StageScope sc(TDGS_STAGE_BLEND, s);
            return launch_render_tiles(s, cam, tiling, opt, buf->key_capacity, buf->tiles_end, buf->sorted_values,
                                       buf->f2d, buf->depths, out, nullptr, ctx->d_counters, frame_counts(buf),
                                       ctx->d_counters + kCounters, ctx->h_monitor_dev);
        }
        TDGS_TRY(read_counters(ctx, s));
        const int64_t nbf = ctx->h_counters[0];
        const int64_t m = ctx->h_counters[kCntCoarse] >> 32;
        const int64_t nb = ctx->h_counters[4];
        const int64_t mc = ctx->h_counters[kCntCoarse] & kLow32;
        *nb_fgaussians_out = (int32_t)nbf;
        *nb_keys_out = m;
        if (nbf == 0 || m == 0) return launch_render_void(s, cam, opt, out);
        if (m >= (int64_t)INT32_MAX) {
            set_error("%lld duplicated keys exceed the int32 index range", (long long)m);
            return TDGS_ERR_CAPACITY;
        }
        if (m > buf->key_capacity || !buf->keys || !buf->values || !buf->sorted_keys || !buf->sorted_values) {
            set_error("key buffers hold %lld keys, %lld needed", (long long)buf->key_capacity, (long long)m);
            return TDGS_ERR_CAPACITY;
        }
        // 6-8: the tile lists by coarse binning
        TDGS_TRY(bin_tile_lists(s, tiling, buf, r, nb, mc, m, nullptr, d_err));
        // 9: blending
        StageScope sc(TDGS_STAGE_BLEND, s);
        return launch_render_tiles(s, cam, tiling, opt, m, buf->tiles_end, buf->sorted_values, buf->f2d,
                                   buf->depths, out);
    }
    // more than 65535 tiles: the reference's 64-bit keys, sorted
    // 5: tile counts in depth order -> M
    {
        StageScope sc(TDGS_STAGE_COUNT_SCAN, s);
        TDGS_TRY(device_scan(SortedCounts{r.srect, d_nb}, SortedCounts{r.srect, d_nb},
                             WriteScanAndBlocks{cs, blk_first, nblk}, n, stemp,
                             sbytes, d_m, s, d_nb));
    }
    TDGS_TRY(read_counters(ctx, s));
    const int64_t nbf = ctx->h_counters[0];
    const int64_t m = ctx->h_counters[1];
    const int64_t nb = ctx->h_counters[4];   // non-empty Gaussians: the sorted depth order's length
    *nb_fgaussians_out = (int32_t)nbf;
    *nb_keys_out = m;
    if (nbf == 0 || m == 0) return launch_render_void(s, cam, opt, out);
    if (m >= (int64_t)INT32_MAX) {
        set_error("%lld duplicated keys exceed the int32 index range", (long long)m);
        return TDGS_ERR_CAPACITY;
    }
    if (m > buf->key_capacity || !buf->keys || !buf->values || !buf->sorted_keys || !buf->sorted_values) {
        set_error("key buffers hold %lld keys, %lld needed", (long long)buf->key_capacity, (long long)m);
        return TDGS_ERR_CAPACITY;
    }
    // 6-7: emit the 64-bit keys in depth order (with the first pass's counts), then the stable
    // sort of their tile bits
    const int eb = end_bit_of(tiling);
    const int32_t nb_tiles = tiling->nb_tiles_x * tiling->nb_tiles_y;
    const int passes = radix_passes(32, eb);
    const int nbits0 = radix_digit_bits(32, eb);   // digit of the first tile-sort pass
    const unsigned egrid = (unsigned)ceil_div(m, kEmitTile);
    {
        // the first radix pass writes the output arrays when the pass count is odd and the
        // alternate ones when even; emit into the other
        const bool emit_into_out = (passes % 2) == 0;
        void* ek = emit_into_out ? (void*)buf->sorted_keys : (void*)buf->keys;
        int32_t* ev2 = emit_into_out ? buf->sorted_values : buf->values;
        const int64_t count_tiles = radix_tiles<uint64_t>(m);
        {
            StageScope sc(TDGS_STAGE_EMIT, s);
            k_emit_depth_order<false><<<egrid, kEmitThreads, 0, s>>>(nb, m, sorted_f, cs, blk_first, buf->depths,
                                                                    r.srect, EmitGrid{tiling->nb_tiles_x, 0, 0},
                                                                    ek, ev2, nbits0, radix_count_table(rtemp),
                                                                    count_tiles);
            TDGS_LAUNCHED();
        }
        StageScope sc(TDGS_STAGE_TILE_SORT, s);
        TDGS_TRY(radix_sort_pairs<uint64_t>((const uint64_t*)ek, (uint64_t*)buf->sorted_keys, ev2,
                                            buf->sorted_values, (uint64_t*)buf->keys, buf->values, m, 32, eb,
                                            rtemp, rbytes, s, radix_count_table(rtemp), d_err));
    }
    // 8: tile ranges
    {
        StageScope sc(TDGS_STAGE_TILE_RANGES, s);
        const bool rects = m > kRectKeysPerGaussian * nbf;
        if (rects) {
            k_fill_i32<<<(unsigned)ceil_div(kRectCopies * ndiff, 256), 256, 0, s>>>(rect_diff, kRectCopies * ndiff, 0);
            TDGS_LAUNCHED();
            k_rect_diff<<<(unsigned)ceil_div(nbf, 256), 256, 0, s>>>(nbf, buf->counts, buf->tile_ranges,
                                                                    tiling->nb_tiles_x, rect_diff, ndiff);
            TDGS_LAUNCHED();
            k_merge_rect_diff<<<(unsigned)ceil_div(ndiff, 256), 256, 0, s>>>(rect_diff, ndiff);
            TDGS_LAUNCHED();
            k_tiles_end_from_rects<<<(unsigned)tiling->nb_tiles_y, kTeThreads, 0, s>>>(
                rect_diff, tiling->nb_tiles_x, buf->tiles_end);
        } else {
            k_tile_ranges<int64_t><<<(unsigned)ceil_div(m, 256), 256, 0, s>>>(m, buf->sorted_keys, nb_tiles,
                                                                             buf->tiles_end);
        }
        TDGS_LAUNCHED();
    }
    // 9: blending
    StageScope sc(TDGS_STAGE_BLEND, s);
    return launch_render_tiles(s, cam, tiling, opt, m, buf->tiles_end, buf->sorted_values, buf->f2d,
                               buf->depths, out);
}

}  // extern "C"
