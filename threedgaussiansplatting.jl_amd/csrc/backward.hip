// backward.hip — backward! on gfx950: reverse per-tile blending with reduced atomics, then
// the backward projection to 3D gradients.
//
// Reference: src/backward_core.jl:37-452 (+ helpers :465-964), src/backward_structs.jl:250-257.
//
// Backward blending (backward_render_tiles_kernel!, :96-293): one workgroup per tile, one
// thread per four pixels. The reference lets every pixel start at its own last contributor and
// issues 9 float atomics per (pixel, Gaussian) pair. Here the wavefront walks the tile's
// sorted list back to front in lock step (a lane whose last contributor lies before the
// current entry contributes zero), so every pixel meets its entries in the reference's order;
// the per-pair arithmetic is regrouped (backward_pair_sums) with the same gradients up to
// rounding.
// The 9 gradient contributions of 7 contributing entries at a time are summed over the
// wavefront in one transpose-sum (permlane swaps and DPP, one add per value), stored per
// wavefront in LDS, added over the workgroup's wavefronts, and reach global memory once per
// (tile, Gaussian) — 9 atomics per tile instead of 9 per pixel.
#include "internal.hpp"

namespace tdgs {

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

// (x + y) after v_permlane32_swap / v_permlane16_swap of x and y: lanes whose bit 5 (resp. 4)
// is clear get x summed with its partner lane's x, the others y with the partner's y. The
// empty asm on the second result keeps the compiler from folding the two results of the
// swap into one (this toolchain compiles a plain r[0] + r[1] to r[0] + r[0]).
__device__ __forceinline__ float halve_swap32(float x, float y) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, y),
                                                    false, false);
    uint32_t hi = r[1];
    asm volatile("" : "+v"(hi));
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, hi);
}
__device__ __forceinline__ float halve_swap16(float x, float y) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, y),
                                                    false, false);
    uint32_t hi = r[1];
    asm volatile("" : "+v"(hi));
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, hi);
}

// Sums 64 values per lane over the wavefront by recursive halving: at the step of lane
// distance D each lane keeps the half of its values whose index has the lane's bit D,
// adds the partner lane's copy of that half and passes on the other half. Six steps
// (D = 32, 16 by permlane swaps; 8, 4, 2, 1 by DPP inside a row) and 63 adds in total leave
// in lane l the wavefront sum of v[l]. v is destroyed.
__device__ __forceinline__ float wave_transpose_sum64(float (&v)[64]) {
    const int lane = __lane_id();
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = halve_swap32(v[i], v[i + 32]);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = halve_swap16(v[i], v[i + 16]);
    const bool b3 = lane & 8, b2 = lane & 4, b1 = lane & 2, b0 = lane & 1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float send = b3 ? v[i] : v[i + 8], keep = b3 ? v[i + 8] : v[i];
        v[i] = keep + dpp_f32<0x128>(send);                       // row_ror:8 = lane ^ 8
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float send = b2 ? v[i] : v[i + 4], keep = b2 ? v[i + 4] : v[i];
        // lane ^ 4 by ds_swizzle in bit-mask mode (and 0x1f, xor 4). One unconditional
        // cross-lane read: a select between two DPP rotations gets turned into a branch, and
        // a DPP read from a lane switched off by that branch returns 0.
        v[i] = keep + __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, send), 0x101f));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float send = b1 ? v[i] : v[i + 2], keep = b1 ? v[i + 2] : v[i];
        v[i] = keep + dpp_f32<0x4e>(send);                        // quad_perm [2,3,0,1]
    }
    const float send = b0 ? v[0] : v[1], keep = b0 ? v[1] : v[0];
    return keep + dpp_f32<0xb1>(send);                            // quad_perm [1,0,3,2]
}

__device__ __forceinline__ int wave_max_i32(int v) {
    for (int d = 32; d >= 1; d >>= 1) {
        const int o = __shfl_xor(v, d, kWave);
        v = o > v ? o : v;
    }
    return v;
}

// backward_pair (backward_core.jl:249-272) in the form the wavefront sums. The partial colour
// psi enters only through g . psi, kept as one scalar gpsi; the terms linear in the entry's M
// or carrying a constant factor are summed over the pixels without it, and M and the factors
// are applied to the wavefront's sums after the transpose-sum:
//   dmu = M (sum out[0], sum out[1]),  dM11 = -sum out[3] / 2,  dM21 = -sum out[4],
//   dM22 = -sum out[5] / 2.
// out += [aa du, aa dv, G dalpha, aa du du, aa du dv, aa dv dv, T alpha g] with aa = alpha dalpha
// (out = ... when first: the first of the lane's pixels the step runs for starts the sums).
__device__ __forceinline__ void backward_pair_sums(bool first, float alpha, float inv1ma, float G, float du, float dv,
                                                   const float c[3], const float g[3], float* T, float* gpsi,
                                                   float out[9]) {
    const float Tn = *T * inv1ma;
    *T = Tn;
    const float tgc = Tn * fmaf(g[2], c[2], fmaf(g[1], c[1], g[0] * c[0]));
    *gpsi = fmaf(alpha, tgc, *gpsi);
    const float dalpha = inv1ma * (tgc - *gpsi);
    const float aa = alpha * dalpha;
    const float adu = aa * du, adv = aa * dv;
    const float ta = Tn * alpha;
    if (first) {
        out[0] = adu;
        out[1] = adv;
        out[2] = G * dalpha;
        out[3] = adu * du;
        out[4] = adu * dv;
        out[5] = adv * dv;
        out[6] = ta * g[0];
        out[7] = ta * g[1];
        out[8] = ta * g[2];
    } else {
        out[0] += adu;
        out[1] += adv;
        out[2] = fmaf(G, dalpha, out[2]);
        out[3] = fmaf(adu, du, out[3]);
        out[4] = fmaf(adu, dv, out[4]);
        out[5] = fmaf(adv, dv, out[5]);
        out[6] = fmaf(ta, g[0], out[6]);
        out[7] = fmaf(ta, g[1], out[7]);
        out[8] = fmaf(ta, g[2], out[8]);
    }
}

constexpr int kSlots = 7;   // 7 entries x 9 gradient components = 63 of the 64 lanes

// The exponent is evaluated in base-2 units from a pre-scaled inverse covariance:
// x = log2(e) * (-(M11 du^2 / 2 + M21 du dv + M22 dv^2 / 2)) = du (A du + B dv) + C dv^2, G = 2^x.
struct __align__(16) BackRec {
    float4 a;  // mu_x mu_y A B
    float4 b;  // C cut a r     (cut: x below which a * G < min_alpha)
    float4 c;  // g b f M11     (f: the Gaussian's index, for the flush)
    float4 d;  // M21 M22 - -
};

struct BackBlendArgs {
    int32_t W, H, TW, TH, ntx;
    float bg0, bg1, bg2, min_alpha, max_alpha;
    float log_min_alpha;   // log(min_alpha) - 1e-3 (-inf without a positive min_alpha)
    int64_t m;
    const int32_t* tiles_end;
    const int32_t* sorted_f;
    const float* f2d;
    const float* rgb_grad;
    const float* T;
    const int32_t* last;
    Grads2D g2;
};

// SEP: the 2D gradients are the reference's four arrays (component addresses by select);
// otherwise the interleaved 9 x capacity array (base[0] + 9 f + k).
// PX pixels per lane: lane l of wavefront w takes pixels 64 PX w + 64 p + l, p < PX, of the
// tile (NB = blockDim.x = NT / PX rounded up to whole wavefronts; a pixel index past NT is
// off), so the per-entry record reads, votes, slot bookkeeping and transpose-sum serve 64 PX
// pixels per wavefront; with tiles of 8 x 8 pixel blocks a wavefront holds PX consecutive
// blocks. A batch holds NB entries. Four pixels per lane at four wavefronts per SIMD (128
// VGPRs; a few per-batch values go to scratch) measured 345 us against 378 us for two pixels
// per lane at 1M Gaussians, 1080p (three wavefronts per SIMD at 142 VGPRs: 365 us).
constexpr int kBackPx = 4;
// BPC > 0 (tile sides multiples of 8, BPC = TH / 8 blocks of 8 x 8 pixels per block column,
// BPC dividing PX): slot p's pixels are slot 0's moved by the constant (8 (p / BPC), 8 (p %
// BPC)), so only slot 0's coordinates are kept per lane and the others' offsets from the
// record are slot 0's plus a constant (three fewer register pairs: 323 us against 349 us at 1M
// Gaussians, 1080p, where the loop's scratch spills went from 52 to 12 bytes per lane). The
// subtraction order differs from the per-pixel form by rounding only. BPC = 0: any tile.
template <bool SEP, int PX, int BPC>
__global__ __launch_bounds__(1024 / kBackPx) __attribute__((amdgpu_waves_per_eu(4))) void k_backward_blend(
    BackBlendArgs a) {
    extern __shared__ float4 s_raw4[];
    const int NT = a.TW * a.TH;
    const int NB = (int)blockDim.x;
    BackRec* s_rec = reinterpret_cast<BackRec*>(s_raw4);
    // Per-wavefront sums [wave][NB][9] (at most 4 wavefronts: 1024 / PX threads). A wavefront
    // takes each entry into at most one slot, so its transposed sums are plain stores (an LDS
    // atomic's round trip sat in front of the next entry's record reads); the flush adds the
    // wavefronts' copies.
    const int NW = NB / kWave;
    float* s_acc = reinterpret_cast<float*>(s_rec + NB);
    float* s_accw = s_acc + (threadIdx.x / kWave) * (NB * 9);
    __shared__ int s_max_last;
    const int t = threadIdx.x;
    const int lane = __lane_id();
    // Row-major tile order. Dealing the tiles over bands of the grid, so that concurrent
    // workgroups flush onto different Gaussians, paid off (0.66 ms against 0.76 ms at 1M
    // Gaussians, 1080p) while every (tile, Gaussian) flush was 9 scattered atomic instructions
    // per 64 entries; with the transposed flush row-major is faster (581 us against 595-602 us
    // for 32 to 1024 bands).
    const int tx = blockIdx.x + 1, ty = blockIdx.y + 1;
    const int tile = tx + (ty - 1) * a.ntx;
    int64_t end = a.tiles_end[tile - 1];
    int64_t beg = tile == 1 ? 0 : a.tiles_end[tile - 2];
    if (end > a.m) end = a.m;
    if (beg < 0) beg = 0;
    if (beg > end) beg = end;

    float T[PX], gpsi[PX], g[PX][3], cu[PX], cv[PX];
    int32_t last[PX];
    bool on[PX];
#pragma unroll
    for (int p = 0; p < PX; ++p) {
        const int q = (t / kWave) * (kWave * PX) + p * kWave + (t % kWave);
        int u_in = 1, v_in = 1;
        if (q < NT) tile_pixel(q, a.TW, a.TH, &u_in, &v_in);
        const int U = u_in + (tx - 1) * a.TW, V = v_in + (ty - 1) * a.TH;
        on[p] = q < NT && U <= a.W && V <= a.H;
        T[p] = 0.0f;
        last[p] = 0;
        g[p][0] = g[p][1] = g[p][2] = 0.0f;
        if (on[p]) {
            const int64_t px = (int64_t)(V - 1) + (int64_t)a.H * (U - 1);
            T[p] = a.T[px];
            last[p] = a.last[px];
            g[p][0] = a.rgb_grad[3 * px];
            g[p][1] = a.rgb_grad[3 * px + 1];
            g[p][2] = a.rgb_grad[3 * px + 2];
        }
        gpsi[p] = T[p] * fmaf(g[p][2], a.bg2, fmaf(g[p][1], a.bg1, g[p][0] * a.bg0));   // g . psi, psi = T bg
        cu[p] = (float)U - 0.5f;
        cv[p] = (float)V - 0.5f;
    }
    static_assert(BPC == 0 || PX % BPC == 0, "slot offsets are constant when BPC divides PX");
    const int slot = lane / 9, comp = lane - 9 * slot;
    const int partner = comp == 0 ? lane + 1 : comp == 1 ? lane - 1 : lane;
    const float scale = comp == 4 ? -1.0f : (comp == 3 || comp == 5) ? -0.5f : 1.0f;
    // entries past the last contributor of every pixel of the wavefront / tile are skipped
    int lane_last = last[0];
#pragma unroll
    for (int p = 1; p < PX; ++p) lane_last = last[p] > lane_last ? last[p] : lane_last;
    const int wave_last = wave_max_i32(lane_last);
    if (t == 0) s_max_last = 0;
    for (int k = t; k < NW * NB * 9; k += NB) s_acc[k] = 0.0f;
    __syncthreads();
    if (lane == 0) atomicMax(&s_max_last, wave_last);
    __syncthreads();
    int64_t hi = s_max_last < end ? (int64_t)s_max_last : end;  // exclusive (0-based)

    // The records of the next batch are gathered into registers (pf, pr) while the current
    // batch is blended, so the gather's latency is not spent behind a barrier.
    int32_t pf = 0;
    float pr[9];
    auto gather = [&](int64_t lo_, int nb_) {
        if (t < nb_) {
            pf = a.sorted_f[lo_ + t] - 1;
            const float* r = a.f2d + 9 * (int64_t)pf;
#pragma unroll
            for (int k = 0; k < 9; ++k) pr[k] = r[k];
        }
    };
    if (hi > beg) gather(hi - NB > beg ? hi - NB : beg, (int)(hi - (hi - NB > beg ? hi - NB : beg)));
    while (hi > beg) {
        const int64_t lo = hi - NB > beg ? hi - NB : beg;
        const int nb = (int)(hi - lo);
        if (t < nb) {
            BackRec rec;
            rec.a = make_float4(pr[0], pr[1], -0.5f * kLog2e * pr[3], -kLog2e * pr[4]);
            // a 2^x < min_alpha for x < cut (log_f error ~1e-7 absolute, inside the 1e-3 margin
            // of log_min_alpha; a NaN cut never skips)
            rec.b = make_float4(-0.5f * kLog2e * pr[5], kLog2e * (a.log_min_alpha - log_f(pr[2])), pr[2], pr[6]);
            rec.c = make_float4(pr[7], pr[8], __builtin_bit_cast(float, pf), pr[3]);
            rec.d = make_float4(pr[4], pr[5], 0.0f, 0.0f);
            s_rec[t] = rec;
        }
        __syncthreads();
        if (lo > beg) gather(lo - NB > beg ? lo - NB : beg, (int)(lo - (lo - NB > beg ? lo - NB : beg)));
        const int jtop = (int)((int64_t)wave_last - lo < nb ? (int64_t)wave_last - lo : nb);
        // entry jj of the batch is before pixel p's last contributor iff jj < last_rel[p]
        int last_rel[PX];
#pragma unroll
        for (int p = 0; p < PX; ++p) last_rel[p] = (int)((int64_t)last[p] - lo);
        // Entries back to front; the 9 contributions of up to kSlots consecutive contributing
        // entries are kept per lane and summed over the wavefront in one transpose-sum, after
        // which lane l holds component l % 9 of slot l / 9 and adds it to the tile's LDS sum.
        int j = __builtin_amdgcn_readfirstlane(jtop - 1);   // wave-uniform: scalar loop control
        // after a transpose-sum lane l holds component comp = l % 9 of slot l / 9
        const float max_alpha = a.max_alpha;
        while (j >= 0) {
            float v[64];
            int js[kSlots];
#pragma unroll
            for (int e = 0; e < kSlots; ++e) {
                js[e] = -1;
                float* o = v + 9 * e;
                while (j >= 0) {
                    const int jj = j--;
                    const float4 ra = s_rec[jj].a, rb = s_rec[jj].b;
                    const float2 rc = *reinterpret_cast<const float2*>(&s_rec[jj].c);
                    float du[PX], dv[PX], x[PX];
                    bool live[PX];
                    uint64_t any[PX], any_all = 0;
#pragma unroll
                    for (int p = 0; p < PX; ++p) {
                        if (BPC == 0 || p == 0) {
                            du[p] = cu[p] - ra.x;
                            dv[p] = cv[p] - ra.y;
                        } else {
                            // (tile_pixel's blocks w PX + p, column-major, BPC per column)
                            du[p] = du[0] + (float)(8 * (p / (BPC > 0 ? BPC : 1)));
                            dv[p] = dv[0] + (float)(8 * (p % (BPC > 0 ? BPC : 1)));
                        }
                        x[p] = fmaf(fmaf(ra.z, du[p], ra.w * dv[p]), du[p], rb.x * dv[p] * dv[p]);
                        // (an off pixel has last = 0, so jj < last_rel fails for it)
                        const bool before = jj < last_rel[p], above = !(x[p] < rb.y);
                        live[p] = before & above;
                        // the vote as masks of the two compares (the mask of their conjunction
                        // takes two more instructions)
                        any[p] = __builtin_amdgcn_ballot_w64(before) & __builtin_amdgcn_ballot_w64(above);
                        any_all |= any[p];
                    }
                    if (any_all == 0) continue;
                    const float c[3] = {rb.w, rc.x, rc.y};
#pragma unroll
                    for (int p = 0; p < PX; ++p) {
                        // A pixel slot no lane of the wavefront is live in is skipped as a whole
                        // (a wave-uniform branch): its steps would leave T, g . psi and the sums
                        // unchanged. When it is the first slot, the others add to zeroed sums.
                        if (any[p] == 0) {
                            if (p == 0) {
#pragma unroll
                                for (int k = 0; k < 9; ++k) o[k] = 0.0f;
                            }
                            continue;
                        }
                        // G by the hardware base-2 exponential (v_exp_f32, ~1 ulp over the whole
                        // float range): the gradients are checked at relative L2, and the forward
                        // pass's bit-exact exp_f decides the contributors
                        const float G = __builtin_amdgcn_exp2f(x[p]);
                        const float aG = rb.z * G;
                        // min(aG, max_alpha) (v_min_f32: a NaN aG gives max_alpha)
                        float alpha;
                        asm("v_min_f32 %0, %1, %2" : "=v"(alpha) : "s"(max_alpha), "v"(aG));
                        const bool cp = live[p] & !(alpha < a.min_alpha);
                        // Branch-free: a lane that does not contribute runs the same steps with
                        // alpha = G = 0, so 1 / (1 - alpha) = 1 exactly and T, g . psi and the
                        // sums are left unchanged.
                        const float al = cp ? alpha : 0.0f;
                        backward_pair_sums(p == 0, al, __builtin_amdgcn_rcpf(1.0f - al), cp ? G : 0.0f, du[p], dv[p],
                                           c, g[p], &T[p], &gpsi[p], o);
                    }
                    // The entry takes a slot when some lane of the wavefront is live for it (its
                    // sums are zero if no lane's alpha reaches min_alpha after all).
                    js[e] = __builtin_amdgcn_readfirstlane(jj);
                    break;
                }
                if (js[e] < 0) {   // a slot left empty at the end of the batch sums zeros
#pragma unroll
                    for (int k = 0; k < 9; ++k) o[k] = 0.0f;
                }
            }
            if (js[0] < 0) break;
            v[63] = 0.0f;
            const float sum = wave_transpose_sum64(v);
            int jl = -1;
#pragma unroll
            for (int e = 0; e < kSlots; ++e) jl = slot == e ? js[e] : jl;
            // The sums become gradient components: dmu = M (sum 0, sum 1) takes the partner
            // lane's sum of the same slot, dM11, dM21, dM22 their factors.
            const float other = __shfl(sum, partner, kWave);
            const int je = jl < 0 ? 0 : jl;
            const float m11 = s_rec[je].c.w;
            const float2 m2 = *reinterpret_cast<const float2*>(&s_rec[je].d);   // M21 M22
            const float mixed = fmaf(comp == 0 ? m11 : m2.y, sum, m2.x * other);
            const float val = comp < 2 ? mixed : sum * scale;
            if (lane < 9 * kSlots && jl >= 0) s_accw[9 * jl + comp] = val;
        }
        __syncthreads();
        // Flush with lane i on component i % 9 of entry i / 9: one atomic instruction covers
        // the 36-byte slots of ~7 Gaussians instead of one scattered word of 64. Each element
        // is cleared for the next batch by the thread that reads it.
        for (int i = t; i < 9 * nb; i += NB) {
            int ii = i;
            asm volatile("" : "+v"(ii));   // (keeps the element index 32-bit: no 64-bit induction variables)
            float v = 0.0f;
            bool nz = false;
            for (int w = 0; w < NW; ++w) {
                const float x = s_acc[w * (NB * 9) + ii];
                v += x;
                nz |= x != 0.0f;
            }
            if (nz) {
                for (int w = 0; w < NW; ++w) s_acc[w * (NB * 9) + ii] = 0.0f;
            }
            if (v != 0.0f) {
                const int e = ii / 9, k = ii - 9 * e;
                const int32_t f = __builtin_bit_cast(int32_t, s_rec[e].c.z);
                unsafeAtomicAdd(SEP ? a.g2.at_dynamic(k, f) : a.g2.base[0] + (9 * (int64_t)f + k), v);
            }
        }
        __syncthreads();
        hi = lo;
    }
}

__global__ void k_zero_f32(float* p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// Adam applied in place of writing the 3D gradients (k_backward_project<true>): the moments,
// the six learning rates and the step constants of update! (optimizer.jl:941-1009).
struct AdamInPlace {
    float* m_means;
    float* m_op;
    float* m_sc;
    float* m_rot;
    float* m_sh;
    float lr[6];        // means, opacity, scaling, rotation, sh dc, sh rest
    float beta1, beta2, omb1, omb2, bc1, bc2, eps;
};

struct BackProjectArgs {
    tdgs_gaussians g;
    tdgs_camera cam;
    tdgs_render_options opt;
    int64_t nbf;
    const int64_t* frame;   // device counts (nbf is then the capacity bound): N_f, status
    const int32_t* fgidx_to_gidx;
    const float* f2d;
    const int32_t* counts;
    tdgs_gradients gr;
    Grads2D g2;
    AdamInPlace adam;
    // or null: update_adc_stats_kernel! folded in (acc[gi] += |dmu| scaled by the half image
    // extent, cnt[gi] += 1, for each filtered Gaussian with a nonzero 2D mean gradient)
    float* adc_acc;
    int32_t* adc_cnt;
    double adc_sw, adc_sh;
};

// The SH Adam moments (384 of the 472 bytes of moments per Gaussian at SH3) are read and
// written once per step: non-temporal accesses, so that they do not displace the parameters,
// which the next step's projection reads, from the 256 MB Infinity Cache (measured at 1M
// Gaussians: projection 64 -> 45 us, this kernel +6 us; the geometry moments' float2 and
// float4 runs made non-temporal as well cost this kernel 27 us more than they saved).
typedef float NtF4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 nt_load4(const float4* p) {
    const NtF4 x = __builtin_nontemporal_load(reinterpret_cast<const NtF4*>(p));
    return make_float4(x.x, x.y, x.z, x.w);
}
__device__ __forceinline__ void nt_store4(float4* p, const float4& v) {
    const NtF4 x = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(x, reinterpret_cast<NtF4*>(p));
}

__device__ __forceinline__ void adam_in_place(const AdamInPlace& d, float& p, float g, float& m1, float& m2, float lr) {
    adam_scalar(p, g, m1, m2, lr, d.beta1, d.beta2, d.omb1, d.omb2, d.bc1, d.bc2, d.eps);
}

// The geometry part of update! for Gaussian gi (0-based) with its 11 gradient components, in
// the operation order of k_adam's geometry items.
__device__ __forceinline__ void adam_geometry(const BackProjectArgs& a, int64_t gi, const float dm[3], float dlogit,
                                              const float dlogs[3], const float dq[4]) {
    // every load before the first store (a store could alias a later load, which would
    // otherwise make each load wait for the stores before it)
    const AdamInPlace& d = a.adam;
    float4 mo = reinterpret_cast<const float4*>(a.g.means_opacity)[gi];
    float2* mm = reinterpret_cast<float2*>(d.m_means) + 3 * gi;
    float2 m0 = mm[0], m1 = mm[1], m2 = mm[2];
    float2 mop = reinterpret_cast<const float2*>(d.m_op)[gi];
    float sc[3];
    float2 msc[3];
    float2* ms = reinterpret_cast<float2*>(d.m_sc) + 3 * gi;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        sc[k] = a.g.scaling[3 * gi + k];
        msc[k] = ms[k];
    }
    float4 r = reinterpret_cast<const float4*>(a.g.rotation)[gi];
    float4* mr = reinterpret_cast<float4*>(d.m_rot) + 2 * gi;
    float4 ma = mr[0], mb = mr[1];
    adam_in_place(d, mo.x, dm[0], m0.x, m0.y, d.lr[0]);
    adam_in_place(d, mo.y, dm[1], m1.x, m1.y, d.lr[0]);
    adam_in_place(d, mo.z, dm[2], m2.x, m2.y, d.lr[0]);
    adam_in_place(d, mo.w, dlogit, mop.x, mop.y, d.lr[1]);
#pragma unroll
    for (int k = 0; k < 3; ++k) adam_in_place(d, sc[k], dlogs[k], msc[k].x, msc[k].y, d.lr[2]);
    adam_in_place(d, r.x, dq[0], ma.x, ma.y, d.lr[3]);
    adam_in_place(d, r.y, dq[1], ma.z, ma.w, d.lr[3]);
    adam_in_place(d, r.z, dq[2], mb.x, mb.y, d.lr[3]);
    adam_in_place(d, r.w, dq[3], mb.z, mb.w, d.lr[3]);
    reinterpret_cast<float4*>(a.g.means_opacity)[gi] = mo;
    mm[0] = m0; mm[1] = m1; mm[2] = m2;
    reinterpret_cast<float2*>(d.m_op)[gi] = mop;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        a.g.scaling[3 * gi + k] = sc[k];
        ms[k] = msc[k];
    }
    reinterpret_cast<float4*>(a.g.rotation)[gi] = r;
    mr[0] = ma;
    mr[1] = mb;
}

// backward_project_fgaussians_kernel! (backward_core.jl:309-452) + compute_sh_coeffs_grad!
// A workgroup takes kBpThreads consecutive filtered Gaussians. Its non-empty ones (count > 0)
// are compacted to the first lanes, so only ceil(active / 64) wavefronts run the projection
// chain; empty ones get zero gradients. SH coefficient blocks (read) and SH gradient blocks
// (written) pass through one LDS array with an odd row stride, so global memory sees
// contiguous runs instead of one 192-byte block per lane.
constexpr int kBpThreads = 256;
constexpr int kShRow = 49;   // >= 48 coefficients, odd: rows of consecutive lanes hit distinct banks
constexpr int kBpUnroll = 16;

//
// ADAM: instead of writing the 3D gradients, the kernel applies update! (k_adam's arithmetic)
// to each filtered Gaussian's parameters and moments (empty ones with zero gradients), so the
// 236 bytes per Gaussian of SH3 gradients are neither written nor read back. Used by the
// trainer when no density control runs between the backward pass and the optimiser.
template <bool ADAM>
__global__ __launch_bounds__(kBpThreads) void k_backward_project(BackProjectArgs a) {
    __shared__ float s_sh[kBpThreads * kShRow];   // row = local index of the Gaussian
    __shared__ int32_t s_gi[kBpThreads];          // gidx (0-based) of active Gaussians, else -1
    __shared__ int32_t s_gall[ADAM ? kBpThreads : 1];   // gidx (0-based) of every valid row, else -1
    __shared__ int16_t s_list[kBpThreads];        // local indices of the active Gaussians
    __shared__ int32_t s_wcnt[kBpThreads / kWave];
    const int t = threadIdx.x, lane = __lane_id(), wave = t / kWave;
    const int64_t f0 = (int64_t)blockIdx.x * kBpThreads;
    int64_t nbf = a.nbf;
    if (a.frame) {   // device counts; nothing to do for a frame whose keys did not fit
        const int64_t fc = a.frame[0];
        nbf = a.frame[3] != kFrameOk ? 0 : fc < nbf ? fc : nbf;
    }
    if (f0 >= nbf) return;   // (uniform over the workgroup)
    const int64_t fz = f0 + t;
    const bool valid = fz < nbf;
    const bool active = valid && a.counts[fz] != 0;
    const int32_t gz = valid ? a.fgidx_to_gidx[fz] - 1 : -1;
    s_gi[t] = active ? gz : -1;
    if (ADAM) s_gall[t] = gz;
    const uint64_t act = __ballot(active);
    if (lane == 0) s_wcnt[wave] = __popcll(act);
    if (ADAM && valid && !active && gz >= 0) {
        const float z[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        adam_geometry(a, gz, z, 0.0f, z, z);
    }
    if (!ADAM && valid && !active) {
        a.gr.mean3d[3 * fz] = 0.0f; a.gr.mean3d[3 * fz + 1] = 0.0f; a.gr.mean3d[3 * fz + 2] = 0.0f;
        a.gr.opacity_feature[fz] = 0.0f;
        a.gr.scaling_features[3 * fz] = 0.0f; a.gr.scaling_features[3 * fz + 1] = 0.0f;
        a.gr.scaling_features[3 * fz + 2] = 0.0f;
        reinterpret_cast<float4*>(a.gr.rotation_features)[fz] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const int hg = (a.gr.sh_degree + 1) * (a.gr.sh_degree + 1);
    const int hr = (a.opt.sh_degree + 1) * (a.opt.sh_degree + 1);
    const int hs = (a.g.sh_degree + 1) * (a.g.sh_degree + 1);
    __syncthreads();
    int before = 0, n_act = 0;
    for (int w = 0; w < kBpThreads / kWave; ++w) {
        if (w < wave) before += s_wcnt[w];
        n_act += s_wcnt[w];
    }
    if (active) s_list[before + __popcll(act & lanemask_lt())] = (int16_t)t;
    // coefficients of the active Gaussians: thread t moves flat items i = t + kBpThreads r
    // (r < 3hs) of the [kBpThreads][3hs] block, (row j, column e) stepped without a division;
    // kBpUnroll loads are issued before their LDS stores so they overlap
    if (hs == 16) {
        // 48-float rows as 12 float4 each: thread t moves float4 items t + kBpThreads r (r < 12),
        // all in flight at once
        float4 val[12];
#pragma unroll
        for (int r = 0; r < 12; ++r) {
            const int i = t + kBpThreads * r, j = i / 12, q = i - 12 * j;
            const int32_t gj = s_gi[j];
            if (gj >= 0) val[r] = reinterpret_cast<const float4*>(a.g.sh)[(int64_t)12 * gj + q];
        }
#pragma unroll
        for (int r = 0; r < 12; ++r) {
            const int i = t + kBpThreads * r, j = i / 12, q = i - 12 * j;
            if (s_gi[j] >= 0) {
                float* d = s_sh + j * kShRow + 4 * q;
                d[0] = val[r].x; d[1] = val[r].y; d[2] = val[r].z; d[3] = val[r].w;
            }
        }
    } else {
        const int w = 3 * hs, dj = kBpThreads / w, de = kBpThreads - dj * w;
        int j = t / w, e = t - j * w;
        for (int r0 = 0; r0 < w; r0 += kBpUnroll) {
            float val[kBpUnroll];
            int dst[kBpUnroll];
#pragma unroll
            for (int u = 0; u < kBpUnroll; ++u) {
                dst[u] = -1;
                if (r0 + u < w) {
                    const int32_t gj = s_gi[j];
                    if (gj >= 0) {
                        val[u] = a.g.sh[(int64_t)w * gj + e];
                        dst[u] = j * kShRow + e;
                    }
                    j += dj;
                    e += de;
                    if (e >= w) { e -= w; ++j; }
                }
            }
#pragma unroll
            for (int u = 0; u < kBpUnroll; ++u)
                if (dst[u] >= 0) s_sh[dst[u]] = val[u];
        }
    }
    __syncthreads();
    const bool worker = t < n_act;
    const int jl = worker ? s_list[t] : 0;
    const int64_t f = f0 + jl;
    float b[16];
    float dcol[3] = {0.0f, 0.0f, 0.0f};
    if (worker) {
        const int64_t gi = s_gi[jl];
        // the density-control accumulators, read before the projection's work so that their
        // loads are in flight during it
        float acc0 = 0.0f;
        int32_t cnt0 = 0;
        if (ADAM && a.adc_acc) {
            acc0 = a.adc_acc[gi];
            cnt0 = a.adc_cnt[gi];
        }
        BackwardProjectIn in;
        const float4 mo = reinterpret_cast<const float4*>(a.g.means_opacity)[gi];
        in.m[0] = mo.x; in.m[1] = mo.y; in.m[2] = mo.z;
        in.logit = mo.w;
        in.logs[0] = a.g.scaling[3 * gi];
        in.logs[1] = a.g.scaling[3 * gi + 1];
        in.logs[2] = a.g.scaling[3 * gi + 2];
        const float4 q = reinterpret_cast<const float4*>(a.g.rotation)[gi];
        in.q[0] = q.x; in.q[1] = q.y; in.q[2] = q.z; in.q[3] = q.w;
        in.sh = s_sh + jl * kShRow;
        in.h_storage = hs;
        const float* r = a.f2d + 9 * f;
        in.mux = r[0]; in.muy = r[1]; in.a = r[2]; in.m11 = r[3]; in.m21 = r[4]; in.m22 = r[5];
        in.rgb[0] = r[6]; in.rgb[1] = r[7]; in.rgb[2] = r[8];
#pragma unroll
        for (int k = 0; k < 9; ++k) in.g2[k] = *a.g2.at(k, f);
        const BackwardProjectOut o = backward_project(in, a.cam, a.opt);
        if (ADAM && a.adc_acc) {
            // (k_adc_stats's operations: the inactive Gaussians' 2D gradients are zero)
            const float gx = in.g2[0], gy = in.g2[1];
            if (gx != 0.0f || gy != 0.0f) {
                const double nrm = sqrt((double)(gx * gx) * a.adc_sw + (double)(gy * gy) * a.adc_sh);
                a.adc_acc[gi] = (float)((double)acc0 + nrm);
                a.adc_cnt[gi] = cnt0 + 1;
            }
        }
        if (ADAM) {
            adam_geometry(a, gi, o.dm, o.dlogit, o.dlogs, o.dq);
        } else {
            for (int k = 0; k < 3; ++k) a.gr.mean3d[3 * f + k] = o.dm[k];
            a.gr.opacity_feature[f] = o.dlogit;
            for (int k = 0; k < 3; ++k) a.gr.scaling_features[3 * f + k] = o.dlogs[k];
            reinterpret_cast<float4*>(a.gr.rotation_features)[f] = make_float4(o.dq[0], o.dq[1], o.dq[2], o.dq[3]);
        }
        sh_grad_basis(a.cam, a.opt.sh_degree, in.m, b);
        dcol[0] = in.g2[6]; dcol[1] = in.g2[7]; dcol[2] = in.g2[8];
    }
    __syncthreads();   // every coefficient read is done: s_sh now takes the SH gradients
    // SH gradients: channel c, coefficient k at column c * hg + k (k < hr); the rows of empty
    // Gaussians are zero; columns k >= hr are left untouched in global memory
    if (worker)
        for (int c = 0; c < 3; ++c)
            for (int k = 0; k < hr; ++k) s_sh[jl * kShRow + c * hg + k] = dcol[c] * b[k];
    if (!active)
        for (int c = 0; c < 3; ++c)
            for (int k = 0; k < hr; ++k) s_sh[t * kShRow + c * hg + k] = 0.0f;
    __syncthreads();
    const int nrows = (int)(nbf - f0 < kBpThreads ? nbf - f0 : kBpThreads);
    if constexpr (ADAM) {
        // update! on the SH coefficients k < hr of every row (k_adam's SH items)
        const AdamInPlace& d = a.adam;
        if (hs == hg && hg == hr && (3 * hr) % 4 == 0) {
            // kBpGroup items per thread at a time, all their loads issued before any store
            // (the parameter and moment stores could alias the next items' loads, so a plain
            // loop would wait on every load in turn)
            constexpr int kBpGroup = 4;
            const int q4 = 3 * hr / 4;
            const int items = nrows * q4;
            for (int base = 0; base < items; base += kBpGroup * kBpThreads) {
                float4 p[kBpGroup], m0[kBpGroup], m1[kBpGroup];
                int64_t gi[kBpGroup];
                int jq[kBpGroup][2];
#pragma unroll
                for (int u = 0; u < kBpGroup; ++u) {
                    const int i = base + t + kBpThreads * u;
                    const int j = i / q4, q = i - j * q4;
                    jq[u][0] = j;
                    jq[u][1] = q;
                    gi[u] = i < items ? s_gall[j] : -1;
                    if (gi[u] >= 0) {
                        p[u] = reinterpret_cast<const float4*>(a.g.sh + (int64_t)3 * hs * gi[u])[q];
                        const float4* mp = reinterpret_cast<const float4*>(d.m_sh + (int64_t)6 * hs * gi[u]) + 2 * q;
                        m0[u] = nt_load4(mp);
                        m1[u] = nt_load4(mp + 1);
                    }
                }
#pragma unroll
                for (int u = 0; u < kBpGroup; ++u) {
                    if (gi[u] < 0) continue;
                    const int j = jq[u][0], q = jq[u][1];
                    const int k0 = (4 * q) % hr;
                    const float* sv = s_sh + j * kShRow + 4 * q;
                    adam_in_place(d, p[u].x, sv[0], m0[u].x, m0[u].y, k0 == 0 ? d.lr[4] : d.lr[5]);
                    adam_in_place(d, p[u].y, sv[1], m0[u].z, m0[u].w, d.lr[5]);
                    adam_in_place(d, p[u].z, sv[2], m1[u].x, m1[u].y, d.lr[5]);
                    adam_in_place(d, p[u].w, sv[3], m1[u].z, m1[u].w, d.lr[5]);
                    reinterpret_cast<float4*>(a.g.sh + (int64_t)3 * hs * gi[u])[q] = p[u];
                    float4* mp = reinterpret_cast<float4*>(d.m_sh + (int64_t)6 * hs * gi[u]) + 2 * q;
                    nt_store4(mp, m0[u]);
                    nt_store4(mp + 1, m1[u]);
                }
            }
        } else {
            const int per = 3 * hr;
            for (int i = t; i < nrows * per; i += kBpThreads) {
                const int j = i / per, e = i - j * per, c = e / hr, k = e - c * hr;
                const int64_t gi = s_gall[j];
                if (gi < 0) continue;
                const int64_t pi = (int64_t)3 * hs * gi + (int64_t)c * hs + k;
                float p = a.g.sh[pi];
                float2 m = reinterpret_cast<float2*>(d.m_sh)[pi];
                adam_in_place(d, p, s_sh[j * kShRow + c * hg + k], m.x, m.y, k == 0 ? d.lr[4] : d.lr[5]);
                a.g.sh[pi] = p;
                reinterpret_cast<float2*>(d.m_sh)[pi] = m;
            }
        }
        return;
    }
    float* dsh = a.gr.sh + (int64_t)3 * hg * f0;
    if (hg == 16 && hr == 16) {
        // every column written: float4 stores of 12 items per thread
#pragma unroll
        for (int r = 0; r < 12; ++r) {
            const int i = t + kBpThreads * r, j = i / 12, q = i - 12 * j;
            if (j < nrows) {
                const float* sv = s_sh + j * kShRow + 4 * q;
                reinterpret_cast<float4*>(dsh)[i] = make_float4(sv[0], sv[1], sv[2], sv[3]);
            }
        }
    } else {
        const int w = 3 * hg, dj = kBpThreads / w, de = kBpThreads - dj * w;
        int j = t / w, e = t - j * w;
        for (int r0 = 0; r0 < w; r0 += kBpUnroll) {
            float val[kBpUnroll];
            bool st[kBpUnroll];
#pragma unroll
            for (int u = 0; u < kBpUnroll; ++u) {
                st[u] = false;
                if (r0 + u < w) {
                    const int k = e - (e >= hg ? hg : 0) - (e >= 2 * hg ? hg : 0);   // e mod hg
                    st[u] = j < nrows && k < hr;
                    if (st[u]) val[u] = s_sh[j * kShRow + e];
                    j += dj;
                    e += de;
                    if (e >= w) { e -= w; ++j; }
                }
            }
#pragma unroll
            for (int u = 0; u < kBpUnroll; ++u)
                if (st[u]) dsh[t + kBpThreads * (r0 + u)] = val[u];
        }
    }
}

static int check_gradients(const tdgs_gradients* gr, int64_t nbf, int data_degree) {
    TDGS_REQUIRE(gr != nullptr, "null gradients");
    TDGS_REQUIRE(gr->capacity >= nbf, "gradient buffers hold %d, need %lld", gr->capacity, (long long)nbf);
    TDGS_REQUIRE(gr->sh_degree >= 0 && gr->sh_degree <= 3, "bad gradient SH degree");
    (void)data_degree;
    if (nbf > 0) {
        Grads2D v;
        TDGS_TRY(grads2d_view(gr, &v));
        TDGS_REQUIRE(gr->mean3d && gr->opacity_feature && gr->scaling_features && gr->rotation_features && gr->sh,
                     "null gradient arrays");
    }
    return TDGS_OK;
}

// zero_2d_grads! (backward_structs.jl:250-257) on the first nbf entries.
static int zero_grads2d(hipStream_t s, const tdgs_gradients* gr, int64_t nbf) {
    if (gr->grads2d) {
        k_zero_f32<<<(unsigned)ceil_div(9 * nbf, 256), 256, 0, s>>>(gr->grads2d, 9 * nbf);
        TDGS_LAUNCHED();
        return TDGS_OK;
    }
    float* const arr[4] = {gr->mean2d_grads, gr->opacity_grads, gr->licov2d_grads, gr->color_grads};
    const int comps[4] = {2, 1, 3, 3};
    for (int k = 0; k < 4; ++k) {
        k_zero_f32<<<(unsigned)ceil_div(comps[k] * nbf, 256), 256, 0, s>>>(arr[k], comps[k] * nbf);
        TDGS_LAUNCHED();
    }
    return TDGS_OK;
}

}  // namespace tdgs

using namespace tdgs;

extern "C" {

int tdgs_backward_render_tiles(void* stream, tdgs_gradients* grads, const float* rgb_grad,
                               const tdgs_render_outputs* out, const tdgs_camera* cam,
                               const tdgs_tiling* tiling, const tdgs_render_options* opt,
                               const tdgs_render_buffers* buf) {
    TDGS_TRY(check_tiling(tiling, cam));
    TDGS_REQUIRE(grads && rgb_grad && out && out->T && out->last && opt && buf,
                 "backward blending needs gradients, rgb_grad, T and last");
    Grads2D g2v;
    TDGS_TRY(grads2d_view(grads, &g2v));
    TDGS_REQUIRE(buf->tiles_end && buf->sorted_values && buf->f2d, "null render buffers");
    TDGS_TRY(check_thresholds(opt));
    hipStream_t s = (hipStream_t)stream;
    StageScope sc(TDGS_STAGE_BACKWARD_BLEND, s);
    BackBlendArgs a;
    a.W = cam->width; a.H = cam->height; a.TW = tiling->tile_width; a.TH = tiling->tile_height;
    a.ntx = tiling->nb_tiles_x;
    a.bg0 = opt->background[0]; a.bg1 = opt->background[1]; a.bg2 = opt->background[2];
    a.min_alpha = opt->min_alpha; a.max_alpha = opt->max_alpha;
    a.log_min_alpha = opt->min_alpha > 0.0f ? (float)(std::log((double)opt->min_alpha) - 1e-3) : -__builtin_inff();
    a.m = buf->key_capacity;
    a.tiles_end = buf->tiles_end; a.sorted_f = buf->sorted_values; a.f2d = buf->f2d;
    a.rgb_grad = rgb_grad; a.T = out->T; a.last = out->last; a.g2 = g2v;
    // kBackPx pixels per thread, in whole wavefronts (the transpose-sum reads all 64 lanes;
    // the pixels past the tile's are off)
    const int nt = ((tiling->tile_width * tiling->tile_height + kBackPx - 1) / kBackPx + kWave - 1) / kWave * kWave;
    const size_t lds = (size_t)nt * (sizeof(BackRec) + (size_t)(nt / kWave) * 9 * sizeof(float));
    const dim3 grid(tiling->nb_tiles_x, tiling->nb_tiles_y);
    // tiles of 8 x 8 pixel blocks with 1, 2 or 4 blocks per column take the constant slot offsets
    const int bpc = tiling->tile_width % 8 == 0 && tiling->tile_height % 8 == 0 ? tiling->tile_height / 8 : 0;
#define TDGS_BB(SEP_, BPC_) k_backward_blend<SEP_, kBackPx, BPC_><<<grid, nt, lds, s>>>(a)
    if (grads->grads2d) {
        if (bpc == 1) TDGS_BB(false, 1);
        else if (bpc == 2) TDGS_BB(false, 2);
        else if (bpc == 4) TDGS_BB(false, 4);
        else TDGS_BB(false, 0);
    } else {
        if (bpc == 1) TDGS_BB(true, 1);
        else if (bpc == 2) TDGS_BB(true, 2);
        else if (bpc == 4) TDGS_BB(true, 4);
        else TDGS_BB(true, 0);
    }
#undef TDGS_BB
    TDGS_LAUNCHED();
    return TDGS_OK;
}

// The filtered count of a backward entry point: nb_fgaussians, or with nb_fgaussians < 0 the
// capacity bound of a device-count render (*frame then points at its counts).
static int filtered_count(int32_t nb_fgaussians, const tdgs_render_buffers* buf, const tdgs_gradients* grads,
                          int64_t* nbf, const int64_t** frame) {
    *frame = nullptr;
    *nbf = nb_fgaussians;
    if (nb_fgaussians >= 0) return TDGS_OK;
    TDGS_REQUIRE(buf && buf->temp && buf->temp_bytes >= 4 * sizeof(int64_t),
                 "nb_fgaussians < 0 reads the counts of a device-count render from its buffers");
    TDGS_REQUIRE(!grads || grads->capacity >= buf->capacity, "gradient buffers hold %d, the render buffers %d",
                 grads ? grads->capacity : 0, buf->capacity);
    *nbf = buf->capacity;
    *frame = frame_counts(buf);
    return TDGS_OK;
}

int tdgs_backward_project(void* stream, tdgs_gradients* grads, const tdgs_gaussians* g,
                          const tdgs_camera* cam, const tdgs_render_options* opt,
                          const tdgs_render_buffers* buf, int32_t nb_fgaussians) {
    TDGS_TRY(check_gaussians(g, true));
    TDGS_TRY(check_options(opt, g->sh_degree));
    int64_t nbf;
    const int64_t* frame;
    TDGS_TRY(filtered_count(nb_fgaussians, buf, grads, &nbf, &frame));
    TDGS_TRY(check_gradients(grads, nbf, g->sh_degree));
    TDGS_REQUIRE(grads->sh_degree >= opt->sh_degree, "gradient SH storage below the render degree");
    TDGS_REQUIRE(cam && buf && buf->fgidx_to_gidx && buf->f2d && buf->counts, "null arguments");
    if (nbf <= 0) return TDGS_OK;
    hipStream_t s = (hipStream_t)stream;
    StageScope sc(TDGS_STAGE_BACKWARD_PROJECT, s);
    BackProjectArgs a;
    a.g = *g; a.cam = *cam; a.opt = *opt; a.nbf = nbf; a.frame = frame;
    a.fgidx_to_gidx = buf->fgidx_to_gidx; a.f2d = buf->f2d; a.counts = buf->counts; a.gr = *grads;
    TDGS_TRY(grads2d_view(grads, &a.g2));
    a.adc_acc = nullptr;
    a.adc_cnt = nullptr;
    k_backward_project<false><<<(unsigned)ceil_div(nbf, kBpThreads), kBpThreads, 0, s>>>(a);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

static int backward_project_adam(void* stream, const tdgs_gradients* grads, tdgs_gaussians* g, tdgs_adam_state* st,
                                 const tdgs_camera* cam, const tdgs_render_options* opt,
                                 const tdgs_render_buffers* buf, int32_t nb_fgaussians, tdgs_adc_buffers* adc) {
    TDGS_TRY(check_gaussians(g, true));
    TDGS_TRY(check_options(opt, g->sh_degree));
    int64_t nbf;
    const int64_t* frame;
    TDGS_TRY(filtered_count(nb_fgaussians, buf, grads, &nbf, &frame));
    TDGS_REQUIRE(grads && grads->capacity >= nbf && grads->sh_degree >= 0 && grads->sh_degree <= 3,
                 "bad gradient buffers");
    TDGS_REQUIRE(grads->sh_degree >= opt->sh_degree, "gradient SH storage below the render degree");
    TDGS_REQUIRE(st && cam && buf && buf->fgidx_to_gidx && buf->f2d && buf->counts, "null arguments");
    if (nbf > 0) {
        TDGS_REQUIRE(st->means_moments && st->opacity_moments && st->scaling_moments && st->rotation_moments &&
                         st->sh_moments,
                     "null arrays");
        hipStream_t s = (hipStream_t)stream;
        StageScope sc(TDGS_STAGE_BACKWARD_PROJECT, s);
        BackProjectArgs a;
        a.g = *g; a.cam = *cam; a.opt = *opt; a.nbf = nbf; a.frame = frame;
        a.fgidx_to_gidx = buf->fgidx_to_gidx; a.f2d = buf->f2d; a.counts = buf->counts; a.gr = *grads;
        TDGS_TRY(grads2d_view(grads, &a.g2));
        AdamInPlace& d = a.adam;
        d.m_means = st->means_moments; d.m_op = st->opacity_moments; d.m_sc = st->scaling_moments;
        d.m_rot = st->rotation_moments; d.m_sh = st->sh_moments;
        d.lr[0] = st->lr_means; d.lr[1] = st->lr_opacity; d.lr[2] = st->lr_scaling;
        d.lr[3] = st->lr_rotation; d.lr[4] = st->lr_sh_dc; d.lr[5] = st->lr_sh_rest;
        d.beta1 = st->beta1; d.beta2 = st->beta2;
        d.omb1 = 1.0f - st->beta1; d.omb2 = 1.0f - st->beta2;
        const double tt = (double)st->update_count + 1.0;
        d.bc1 = (float)(1.0 - pow((double)st->beta1, tt));
        d.bc2 = (float)(1.0 - pow((double)st->beta2, tt));
        d.eps = st->epsilon;
        a.adc_acc = adc ? adc->accum_grad_norms : nullptr;
        a.adc_cnt = adc ? adc->contribution_counts : nullptr;
        a.adc_sw = (double)cam->width * cam->width / 4.0;
        a.adc_sh = (double)cam->height * cam->height / 4.0;
        k_backward_project<true><<<(unsigned)ceil_div(nbf, kBpThreads), kBpThreads, 0, s>>>(a);
        TDGS_LAUNCHED();
    }
    st->update_count += 1;
    return TDGS_OK;
}

int tdgs_backward_project_adam(void* stream, const tdgs_gradients* grads, tdgs_gaussians* g, tdgs_adam_state* st,
                               const tdgs_camera* cam, const tdgs_render_options* opt,
                               const tdgs_render_buffers* buf, int32_t nb_fgaussians) {
    return backward_project_adam(stream, grads, g, st, cam, opt, buf, nb_fgaussians, nullptr);
}

int tdgs_backward_project_adam_adc(void* stream, const tdgs_gradients* grads, tdgs_gaussians* g,
                                   tdgs_adam_state* st, const tdgs_camera* cam, const tdgs_render_options* opt,
                                   const tdgs_render_buffers* buf, int32_t nb_fgaussians, tdgs_adc_buffers* adc) {
    TDGS_REQUIRE(adc && adc->accum_grad_norms && adc->contribution_counts, "null ADC arrays");
    TDGS_REQUIRE(g && adc->capacity >= g->n, "ADC buffers hold %d Gaussians, need %d", adc ? adc->capacity : 0,
                 g ? g->n : 0);
    return backward_project_adam(stream, grads, g, st, cam, opt, buf, nb_fgaussians, adc);
}

int tdgs_backward(void* stream, tdgs_gradients* grads, const float* rgb_grad, const tdgs_render_outputs* out,
                  const tdgs_gaussians* g, const tdgs_camera* cam, const tdgs_tiling* tiling,
                  const tdgs_render_options* opt, const tdgs_render_buffers* buf, int32_t nb_fgaussians) {
    int64_t nbf;
    const int64_t* frame;
    TDGS_TRY(filtered_count(nb_fgaussians, buf, grads, &nbf, &frame));
    TDGS_TRY(check_gradients(grads, nbf, g ? g->sh_degree : 0));
    if (nbf <= 0) return TDGS_OK;
    hipStream_t s = (hipStream_t)stream;
    TDGS_TRY(zero_grads2d(s, grads, nbf));   // (with device counts: the whole capacity)
    TDGS_TRY(tdgs_backward_render_tiles(stream, grads, rgb_grad, out, cam, tiling, opt, buf));
    return tdgs_backward_project(stream, grads, g, cam, opt, buf, nb_fgaussians);
}

}  // extern "C"
