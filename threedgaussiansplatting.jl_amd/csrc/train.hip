// train.hip — optimiser and training helpers on gfx950: fused sparse Adam, adaptive density
// control (statistics, plan, compaction, index remap), L1 loss gradient, opacity reset,
// spherical-harmonics degree resize.
//
// Reference: src/optimizer.jl:941-1009, 1084-1248, 1304-1378; src/training.jl:173-580;
// src/gaussians.jl:1093-1101, 1526-1694; src/misc.jl:100-125.
#include "internal.hpp"
#include "scan.hpp"

namespace tdgs {

// ------------------------------------------------------------------------------------
// Adam (update!, optimizer.jl:964-1009) over the filtered Gaussians; entries whose
// fgidx_to_gidx is 0 (removed by adaptive density control) are skipped. The reference runs five
// launches (one per component); here one launch streams every component, as two kinds of
// items in one grid:
//   SH items        the first (d+1)^2 coefficients of each colour channel (d = render SH
//                   degree). When the parameter, gradient and render blocks coincide and
//                   hold a multiple of 4 floats, an item is a float4 of parameters with its
//                   float4 of gradients and two float4 of (m, v) moment pairs, so every
//                   array is streamed in 16-byte pieces; otherwise an item is one scalar.
//   geometry items  one Gaussian: mean (3), opacity logit, log-scales (3), quaternion (4).
// ------------------------------------------------------------------------------------

struct AdamArgs {
    float* mo;
    float* sc;
    float* rot;
    float* sh;
    float* m_means;
    float* m_op;
    float* m_sc;
    float* m_rot;
    float* m_sh;
    const float* g_mean;
    const float* g_op;
    const float* g_sc;
    const float* g_rot;
    const float* g_sh;
    const int32_t* fgidx_to_gidx;
    int64_t nbf;
    int hs, hg, hr;
    int vec;            // SH items are float4 (hs == hg == hr, 3 hr % 4 == 0)
    int64_t sh_items;   // number of SH items
    int64_t sh_blocks;  // blocks [0, sh_blocks) take SH items, the rest geometry items
    float lr[6];        // means, opacity, scaling, rotation, sh dc, sh rest
    float beta1, beta2, omb1, omb2, bc1, bc2, eps;
};

__device__ __forceinline__ void adam1(const AdamArgs& a, float& p, float g, float& m1, float& m2, float lr) {
    adam_scalar(p, g, m1, m2, lr, a.beta1, a.beta2, a.omb1, a.omb2, a.bc1, a.bc2, a.eps);
}

__global__ __launch_bounds__(256) void k_adam(AdamArgs a) {
    if ((int64_t)blockIdx.x < a.sh_blocks) {
        const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (i >= a.sh_items) return;
        if (a.vec) {
            const int q4 = 3 * a.hr / 4;                 // float4 per Gaussian block
            const int64_t f = i / q4;
            const int q = (int)(i - f * q4);
            const int64_t gi = (int64_t)a.fgidx_to_gidx[f] - 1;
            if (gi < 0) return;                          // entry removed by density control
            const int k0 = (4 * q) % a.hr;               // coefficient index of the first lane
            float4* pp = reinterpret_cast<float4*>(a.sh + (int64_t)3 * a.hs * gi) + q;
            float4* mp = reinterpret_cast<float4*>(a.m_sh + (int64_t)6 * a.hs * gi) + 2 * q;
            const float4 g = reinterpret_cast<const float4*>(a.g_sh + (int64_t)3 * a.hg * f)[q];
            float4 p = *pp, m0 = mp[0], m1 = mp[1];
            adam1(a, p.x, g.x, m0.x, m0.y, k0 == 0 ? a.lr[4] : a.lr[5]);
            adam1(a, p.y, g.y, m0.z, m0.w, a.lr[5]);
            adam1(a, p.z, g.z, m1.x, m1.y, a.lr[5]);
            adam1(a, p.w, g.w, m1.z, m1.w, a.lr[5]);
            *pp = p;
            mp[0] = m0;
            mp[1] = m1;
        } else {
            const int per = 3 * a.hr;
            const int64_t f = i / per;
            const int e = (int)(i - f * per), c = e / a.hr, k = e - c * a.hr;
            const int64_t gi = (int64_t)a.fgidx_to_gidx[f] - 1;
            if (gi < 0) return;
            const int64_t pi = (int64_t)3 * a.hs * gi + (int64_t)c * a.hs + k;
            float p = a.sh[pi];
            float2 m = reinterpret_cast<float2*>(a.m_sh)[pi];
            adam1(a, p, a.g_sh[(int64_t)3 * a.hg * f + (int64_t)c * a.hg + k], m.x, m.y, k == 0 ? a.lr[4] : a.lr[5]);
            a.sh[pi] = p;
            reinterpret_cast<float2*>(a.m_sh)[pi] = m;
        }
        return;
    }
    const int64_t f = ((int64_t)blockIdx.x - a.sh_blocks) * blockDim.x + threadIdx.x;
    if (f >= a.nbf) return;
    const int64_t gi = (int64_t)a.fgidx_to_gidx[f] - 1;
    if (gi < 0) return;
    float4 mo = reinterpret_cast<float4*>(a.mo)[gi];
    float2* mm = reinterpret_cast<float2*>(a.m_means) + 3 * gi;
    float2 m0 = mm[0], m1 = mm[1], m2 = mm[2];
    adam1(a, mo.x, a.g_mean[3 * f], m0.x, m0.y, a.lr[0]);
    adam1(a, mo.y, a.g_mean[3 * f + 1], m1.x, m1.y, a.lr[0]);
    adam1(a, mo.z, a.g_mean[3 * f + 2], m2.x, m2.y, a.lr[0]);
    float2 mop = reinterpret_cast<float2*>(a.m_op)[gi];
    adam1(a, mo.w, a.g_op[f], mop.x, mop.y, a.lr[1]);
    reinterpret_cast<float4*>(a.mo)[gi] = mo;
    mm[0] = m0; mm[1] = m1; mm[2] = m2;
    reinterpret_cast<float2*>(a.m_op)[gi] = mop;
    float2* ms = reinterpret_cast<float2*>(a.m_sc) + 3 * gi;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        float p = a.sc[3 * gi + k];
        float2 m = ms[k];
        adam1(a, p, a.g_sc[3 * f + k], m.x, m.y, a.lr[2]);
        a.sc[3 * gi + k] = p;
        ms[k] = m;
    }
    float4 r = reinterpret_cast<float4*>(a.rot)[gi];
    const float4 gr = reinterpret_cast<const float4*>(a.g_rot)[f];
    float4* mr = reinterpret_cast<float4*>(a.m_rot) + 2 * gi;
    float4 ma = mr[0], mb = mr[1];
    adam1(a, r.x, gr.x, ma.x, ma.y, a.lr[3]);
    adam1(a, r.y, gr.y, ma.z, ma.w, a.lr[3]);
    adam1(a, r.z, gr.z, mb.x, mb.y, a.lr[3]);
    adam1(a, r.w, gr.w, mb.z, mb.w, a.lr[3]);
    reinterpret_cast<float4*>(a.rot)[gi] = r;
    mr[0] = ma;
    mr[1] = mb;
}

// ------------------------------------------------------------------------------------
// Adaptive density control
// ------------------------------------------------------------------------------------

// update_adc_stats_kernel! (training.jl:472-497). ((h^2, w^2) ./ 4 is a Float64 pair there,
// so the norm is formed in double precision.)
// mean2d: the x component of the first mean gradient, the y component follows it; stride
// floats from one filtered Gaussian to the next (9 interleaved, 2 for the reference's array).
// frame (device counts, may be null): N_f and the frame status of a device-count render; nbf
// is then the capacity bound.
__global__ void k_adc_stats(const float* __restrict__ mean2d, int32_t stride, const int32_t* __restrict__ f2g,
                            int64_t nbf, double sw, double sh, float* __restrict__ acc, int32_t* __restrict__ cnt,
                            const int64_t* frame) {
    const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (frame) nbf = frame[3] != kFrameOk ? 0 : frame[0] < nbf ? frame[0] : nbf;
    if (f >= nbf) return;
    const float gx = mean2d[stride * f], gy = mean2d[stride * f + 1];
    if (gx != 0.0f || gy != 0.0f) {
        const int64_t gi = (int64_t)f2g[f] - 1;
        const double nrm = sqrt((double)(gx * gx) * sw + (double)(gy * gy) * sh);
        acc[gi] = (float)((double)acc[gi] + nrm);
        cnt[gi] += 1;
    }
}

// Masks of one Gaussian (training.jl:325-363); returns its new count (0, 1 or 2).
struct AdcMasks {
    const float* mo;
    const float* sc;
    const float* acc;
    const int32_t* cnt;
    uint8_t* prune;
    uint8_t* densify;
    uint8_t* clone;
    float prune_logit, log_max_scale, grad_threshold, log_size_threshold;
    int use_max_scale;
    __device__ int32_t operator()(int64_t i) const {
        const int32_t c = cnt[i];
        const float avg = c >= 1 ? acc[i] / (float)c : 0.0f;
        const float smax = fmaxf(fmaxf(sc[3 * i], sc[3 * i + 1]), sc[3 * i + 2]);
        bool pr = mo[4 * i + 3] < prune_logit;
        if (use_max_scale) pr = pr || smax > log_max_scale;
        const bool de = !pr && avg >= grad_threshold;
        const bool cl = de && smax <= log_size_threshold;
        prune[i] = pr;
        densify[i] = de;
        clone[i] = cl;
        return (pr ? 0 : 1) + (de ? 1 : 0);
    }
};

struct AdcCounts {
    const uint8_t* prune;
    const uint8_t* densify;
    __device__ int32_t operator()(int64_t i) const { return (prune[i] ? 0 : 1) + (densify[i] ? 1 : 0); }
};

// new_gaussian_counts_cs + fill_ngidx_to_gidx_kernel! (training.jl:382-397, 557-580).
struct AdcPlanOut {
    int32_t* cs;
    int32_t* ngidx;
    int64_t cap;
    __device__ void operator()(int64_t i, int64_t incl, int32_t item) const {
        cs[i] = (int32_t)incl;
        if (item >= 1 && incl <= cap) ngidx[incl - 1] = (int32_t)(i + 1);
        if (item == 2 && incl <= cap) ngidx[incl - 2] = (int32_t)(i + 1);
    }
};

struct AdcApplyArgs {
    tdgs_gaussians src, dst;
    tdgs_adam_state sm, dm;
    const uint8_t* prune;
    const uint8_t* densify;
    const uint8_t* clone;
    const int32_t* cs;
    int64_t n;
    int h;
    float log_split;
    uint64_t seed;
};

__device__ __forceinline__ void copy_block(const float* s, float* d, int count) {
    for (int k = 0; k < count; ++k) d[k] = s[k];
}
__device__ __forceinline__ void zero_block(float* d, int count) {
    for (int k = 0; k < count; ++k) d[k] = 0.0f;
}

// fill_means_opacity_features_adc_kernel!, fill_scaling_features_adc_kernel! (gaussians.jl
// :1589-1694), the indexlastaxis gathers (:1563-1571) and fill_adam_moments_component_kernel!
// (optimizer.jl:1342-1378), fused: one thread per old Gaussian writes all its new slots.
__global__ __launch_bounds__(256) void k_adc_apply(AdcApplyArgs a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n || a.prune[i]) return;
    const int h = a.h;
    const int64_t last = (int64_t)a.cs[i] - 1;
    const bool dens = a.densify[i], cl = a.clone[i];
    const int64_t first = dens ? last - 1 : last;
    const float4 mo = reinterpret_cast<const float4*>(a.src.means_opacity)[i];
    const float s0 = a.src.scaling[3 * i], s1 = a.src.scaling[3 * i + 1], s2 = a.src.scaling[3 * i + 2];
    const float4 q = reinterpret_cast<const float4*>(a.src.rotation)[i];
    float z[6] = {0, 0, 0, 0, 0, 0};
    float R[9];
    float sc[3];
    const bool split = dens && !cl;
    if (split) {
        quat_to_rot(q.x, q.y, q.z, q.w, R);
        sc[0] = exp_f(s0); sc[1] = exp_f(s1); sc[2] = exp_f(s2);
        normal_pair(a.seed, (uint64_t)i, 0, &z[0], &z[1]);
        normal_pair(a.seed, (uint64_t)i, 1, &z[2], &z[3]);
        normal_pair(a.seed, (uint64_t)i, 2, &z[4], &z[5]);
    }
    for (int64_t ni = first; ni <= last; ++ni) {
        const int j = (int)(ni - first);
        float4 nm = mo;
        float ns0 = s0, ns1 = s1, ns2 = s2;
        if (split) {
            const float w0 = z[3 * j] * sc[0], w1 = z[3 * j + 1] * sc[1], w2 = z[3 * j + 2] * sc[2];
            nm.x = mo.x + fmaf(R[2], w2, fmaf(R[1], w1, R[0] * w0));
            nm.y = mo.y + fmaf(R[5], w2, fmaf(R[4], w1, R[3] * w0));
            nm.z = mo.z + fmaf(R[8], w2, fmaf(R[7], w1, R[6] * w0));
            ns0 = s0 + a.log_split; ns1 = s1 + a.log_split; ns2 = s2 + a.log_split;
        }
        reinterpret_cast<float4*>(a.dst.means_opacity)[ni] = nm;
        a.dst.scaling[3 * ni] = ns0;
        a.dst.scaling[3 * ni + 1] = ns1;
        a.dst.scaling[3 * ni + 2] = ns2;
        reinterpret_cast<float4*>(a.dst.rotation)[ni] = q;
        copy_block(a.src.sh + (int64_t)3 * h * i, a.dst.sh + (int64_t)3 * h * ni, 3 * h);
        // moments: carried over and first clone keep theirs, second clone and splits start at 0
        const bool keep_m = !dens || (cl && ni == first);
        if (keep_m) {
            copy_block(a.sm.means_moments + 6 * i, a.dm.means_moments + 6 * ni, 6);
            copy_block(a.sm.opacity_moments + 2 * i, a.dm.opacity_moments + 2 * ni, 2);
            copy_block(a.sm.scaling_moments + 6 * i, a.dm.scaling_moments + 6 * ni, 6);
            copy_block(a.sm.rotation_moments + 8 * i, a.dm.rotation_moments + 8 * ni, 8);
            copy_block(a.sm.sh_moments + (int64_t)6 * h * i, a.dm.sh_moments + (int64_t)6 * h * ni, 6 * h);
        } else {
            zero_block(a.dm.means_moments + 6 * ni, 6);
            zero_block(a.dm.opacity_moments + 2 * ni, 2);
            zero_block(a.dm.scaling_moments + 6 * ni, 6);
            zero_block(a.dm.rotation_moments + 8 * ni, 8);
            zero_block(a.dm.sh_moments + (int64_t)6 * h * ni, 6 * h);
        }
    }
}

// adjust_fgidx_to_gidx_adc_kernel! (training.jl:514-541).
__global__ void k_adc_remap(const uint8_t* prune, const uint8_t* densify, const uint8_t* clone,
                            const int32_t* cs, int32_t* f2g, int64_t nbf) {
    const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= nbf) return;
    const int64_t gi = (int64_t)f2g[f] - 1;
    int32_t ng = 0;
    if (gi >= 0 && !prune[gi]) {
        if (densify[gi]) {
            if (clone[gi]) ng = cs[gi] - 1;
        } else {
            ng = cs[gi];
        }
    }
    f2g[f] = ng;
}

__global__ void k_fill_i32_f32(float* a, int32_t* b, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (a) a[i] = 0.0f;
    if (b) b[i] = 0;
}

// ------------------------------------------------------------------------------------
// Loss, opacity reset, SH resize
// ------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_l1_grad(const float* __restrict__ r, const float* __restrict__ gt,
                                                 int64_t count, float w, float dw, const float* __restrict__ dg,
                                                 float* __restrict__ grad, double* __restrict__ l1) {
    __shared__ double s_part[256 / kWave];
    const int64_t base = (int64_t)blockIdx.x * blockDim.x * 4 + threadIdx.x;
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + (int64_t)k * blockDim.x;
        if (i < count) {
            const float a = r[i], b = gt[i];
            acc += fabs((double)a - (double)b);
            const float s = a > b ? w : -w;   // ties take -w (training.jl:214-215)
            grad[i] = dg ? s + dw * dg[i] : s;   // product rounded, then the sum (no FMA)
        }
    }
    if (!l1) return;
    for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d, kWave);
    if (__lane_id() == 0) s_part[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int k = 0; k < 256 / kWave; ++k) t += s_part[k];
        atomicAdd(l1, t);
    }
}

__global__ void k_opacity_reset(float* mo, float max_logit, float* mom, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = mo[4 * i + 3];
    mo[4 * i + 3] = fminf(v, max_logit);
    if (mom) {
        mom[2 * i] = 0.0f;
        mom[2 * i + 1] = 0.0f;
    }
}

// dst[(e, k, c, i)] = k < h_src ? src[(e, k, c, i)] : 0 for interleave slot e.
__global__ void k_sh_resize(const float* __restrict__ src, int hs, float* __restrict__ dst, int hd, int64_t n,
                            int il) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per = (int64_t)il * hd * 3;
    if (t >= per * n) return;
    const int64_t i = t / per;
    const int64_t r = t - i * per;
    const int c = (int)(r / ((int64_t)il * hd));
    const int rk = (int)(r - (int64_t)c * il * hd);
    const int k = rk / il, e = rk - k * il;
    dst[t] = k < hs ? src[i * il * hs * 3 + (int64_t)c * il * hs + (int64_t)k * il + e] : 0.0f;
}

}  // namespace tdgs

using namespace tdgs;

extern "C" {

int tdgs_adam_step(void* stream, tdgs_gaussians* g, tdgs_adam_state* st, const tdgs_gradients* grads,
                   const int32_t* fgidx_to_gidx, int32_t nb_fgaussians, int32_t sh_degree) {
    TDGS_TRY(check_gaussians(g, true));
    TDGS_REQUIRE(st && grads, "null optimiser state or gradients");
    TDGS_REQUIRE(sh_degree >= 0 && sh_degree <= g->sh_degree && sh_degree <= grads->sh_degree,
                 "SH degree %d exceeds the stored degrees", sh_degree);
    TDGS_REQUIRE(nb_fgaussians >= 0 && grads->capacity >= nb_fgaussians, "bad filtered count");
    if (nb_fgaussians > 0) {
        TDGS_REQUIRE(fgidx_to_gidx && st->means_moments && st->opacity_moments && st->scaling_moments &&
                         st->rotation_moments && st->sh_moments,
                     "null arrays");
        hipStream_t s = (hipStream_t)stream;
        StageScope sc(TDGS_STAGE_ADAM, s);
        AdamArgs a;
        a.mo = g->means_opacity; a.sc = g->scaling; a.rot = g->rotation; a.sh = g->sh;
        a.m_means = st->means_moments; a.m_op = st->opacity_moments; a.m_sc = st->scaling_moments;
        a.m_rot = st->rotation_moments; a.m_sh = st->sh_moments;
        a.g_mean = grads->mean3d; a.g_op = grads->opacity_feature; a.g_sc = grads->scaling_features;
        a.g_rot = grads->rotation_features; a.g_sh = grads->sh;
        a.fgidx_to_gidx = fgidx_to_gidx;
        a.nbf = nb_fgaussians;
        a.hs = (g->sh_degree + 1) * (g->sh_degree + 1);
        a.hg = (grads->sh_degree + 1) * (grads->sh_degree + 1);
        a.hr = (sh_degree + 1) * (sh_degree + 1);
        a.lr[0] = st->lr_means; a.lr[1] = st->lr_opacity; a.lr[2] = st->lr_scaling;
        a.lr[3] = st->lr_rotation; a.lr[4] = st->lr_sh_dc; a.lr[5] = st->lr_sh_rest;
        a.beta1 = st->beta1; a.beta2 = st->beta2;
        a.omb1 = 1.0f - st->beta1; a.omb2 = 1.0f - st->beta2;
        const double t = (double)st->update_count + 1.0;
        a.bc1 = (float)(1.0 - pow((double)st->beta1, t));
        a.bc2 = (float)(1.0 - pow((double)st->beta2, t));
        a.eps = st->epsilon;
        a.vec = (a.hs == a.hg && a.hg == a.hr && (3 * a.hr) % 4 == 0) ? 1 : 0;
        a.sh_items = (int64_t)nb_fgaussians * (a.vec ? 3 * a.hr / 4 : 3 * a.hr);
        a.sh_blocks = ceil_div(a.sh_items, 256);
        const int64_t blocks = a.sh_blocks + ceil_div(nb_fgaussians, 256);
        k_adam<<<(unsigned)blocks, 256, 0, s>>>(a);
        TDGS_LAUNCHED();
    }
    st->update_count += 1;
    return TDGS_OK;
}

int tdgs_adc_stats(void* stream, tdgs_adc_buffers* adc, const tdgs_gradients* grads, const int32_t* fgidx_to_gidx,
                   int32_t nb_fgaussians, int32_t width, int32_t height) {
    TDGS_REQUIRE(adc && grads && fgidx_to_gidx, "null arguments");
    if (nb_fgaussians <= 0) return TDGS_OK;
    TDGS_REQUIRE(adc->accum_grad_norms && adc->contribution_counts, "null arrays");
    Grads2D g2;
    TDGS_TRY(grads2d_view(grads, &g2));
    hipStream_t s = (hipStream_t)stream;
    StageScope sc(TDGS_STAGE_ADC, s);
    const double sw = (double)width * width / 4.0, sh = (double)height * height / 4.0;
    k_adc_stats<<<(unsigned)ceil_div(nb_fgaussians, 256), 256, 0, s>>>(g2.base[0], g2.stride[0], fgidx_to_gidx,
                                                                       nb_fgaussians,
                                                                       sw, sh, adc->accum_grad_norms,
                                                                       adc->contribution_counts, nullptr);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_adc_stats_frame(void* stream, tdgs_adc_buffers* adc, const tdgs_gradients* grads,
                         const tdgs_render_buffers* buf, int32_t width, int32_t height) {
    TDGS_REQUIRE(adc && grads && buf && buf->fgidx_to_gidx && buf->temp && buf->temp_bytes >= 4 * sizeof(int64_t),
                 "null arguments");
    TDGS_REQUIRE(adc->accum_grad_norms && adc->contribution_counts, "null arrays");
    TDGS_REQUIRE(grads->capacity >= buf->capacity, "gradient buffers hold %d, the render buffers %d",
                 grads->capacity, buf->capacity);
    if (buf->capacity <= 0) return TDGS_OK;
    Grads2D g2;
    TDGS_TRY(grads2d_view(grads, &g2));
    hipStream_t s = (hipStream_t)stream;
    StageScope sc(TDGS_STAGE_ADC, s);
    const double sw = (double)width * width / 4.0, sh = (double)height * height / 4.0;
    k_adc_stats<<<(unsigned)ceil_div(buf->capacity, 256), 256, 0, s>>>(g2.base[0], g2.stride[0], buf->fgidx_to_gidx,
                                                                       buf->capacity, sw, sh, adc->accum_grad_norms,
                                                                       adc->contribution_counts, frame_counts(buf));
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_adc_plan(tdgs_ctx* ctx, void* stream, tdgs_adc_buffers* adc, const tdgs_gaussians* g, float prune_logit,
                  int32_t use_max_scale, float log_max_scale, float grad_threshold, float log_size_threshold,
                  int32_t* n_new_out) {
    TDGS_REQUIRE(ctx && adc && n_new_out, "null arguments");
    TDGS_TRY(check_gaussians(g, true));
    TDGS_REQUIRE(adc->capacity >= g->n, "ADC buffers hold %d Gaussians, need %d", adc->capacity, g->n);
    *n_new_out = 0;
    if (g->n == 0) return TDGS_OK;
    TDGS_REQUIRE(adc->prune && adc->densify && adc->clone && adc->new_counts_cs && adc->ngidx_to_gidx &&
                     adc->accum_grad_norms && adc->contribution_counts && adc->temp,
                 "null ADC arrays");
    hipStream_t s = (hipStream_t)stream;
    {
        StageScope sc(TDGS_STAGE_ADC, s);
        AdcMasks masks{g->means_opacity, g->scaling, adc->accum_grad_norms, adc->contribution_counts,
                       adc->prune, adc->densify, adc->clone, prune_logit, log_max_scale, grad_threshold,
                       log_size_threshold, use_max_scale};
        TDGS_TRY(device_scan(masks, AdcCounts{adc->prune, adc->densify},
                             AdcPlanOut{adc->new_counts_cs, adc->ngidx_to_gidx, adc->new_capacity}, g->n,
                             adc->temp, adc->temp_bytes, ctx->d_counters + 2, s));
    }
    TDGS_TRY(read_counters(ctx, s));
    const int64_t nn = ctx->h_counters[2];
    *n_new_out = (int32_t)nn;
    if (nn > adc->new_capacity) {
        set_error("ngidx_to_gidx holds %d entries, %lld needed", adc->new_capacity, (long long)nn);
        return TDGS_ERR_CAPACITY;
    }
    return TDGS_OK;
}

int tdgs_adc_apply(void* stream, const tdgs_adc_buffers* adc, const tdgs_gaussians* src, tdgs_gaussians* dst,
                   const tdgs_adam_state* src_m, tdgs_adam_state* dst_m, float log_split_factor, uint64_t seed) {
    TDGS_TRY(check_gaussians(src, true));
    TDGS_TRY(check_gaussians(dst, true));
    TDGS_REQUIRE(adc && src_m && dst_m, "null arguments");
    TDGS_REQUIRE(src->sh_degree == dst->sh_degree, "SH degree mismatch");
    if (src->n == 0) return TDGS_OK;
    hipStream_t s = (hipStream_t)stream;
    StageScope sc(TDGS_STAGE_ADC, s);
    AdcApplyArgs a;
    a.src = *src; a.dst = *dst; a.sm = *src_m; a.dm = *dst_m;
    a.prune = adc->prune; a.densify = adc->densify; a.clone = adc->clone; a.cs = adc->new_counts_cs;
    a.n = src->n;
    a.h = (src->sh_degree + 1) * (src->sh_degree + 1);
    a.log_split = log_split_factor;
    a.seed = seed;
    k_adc_apply<<<(unsigned)ceil_div(src->n, 256), 256, 0, s>>>(a);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_adc_remap_fgidx(void* stream, const tdgs_adc_buffers* adc, int32_t* fgidx_to_gidx, int32_t nb_fgaussians) {
    TDGS_REQUIRE(adc && (fgidx_to_gidx || nb_fgaussians == 0), "null arguments");
    if (nb_fgaussians <= 0) return TDGS_OK;
    hipStream_t s = (hipStream_t)stream;
    k_adc_remap<<<(unsigned)ceil_div(nb_fgaussians, 256), 256, 0, s>>>(adc->prune, adc->densify, adc->clone,
                                                                       adc->new_counts_cs, fgidx_to_gidx,
                                                                       nb_fgaussians);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_adc_reset_stats(void* stream, tdgs_adc_buffers* adc, int32_t n) {
    TDGS_REQUIRE(adc && n >= 0 && n <= adc->capacity, "bad arguments");
    if (n == 0) return TDGS_OK;
    k_fill_i32_f32<<<(unsigned)ceil_div(n, 256), 256, 0, (hipStream_t)stream>>>(adc->accum_grad_norms,
                                                                              adc->contribution_counts, n);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_l1_loss_grad(void* stream, const float* rendered, const float* gt, int64_t count, float l1_weight,
                      float dssim_weight, const float* dssim_grad, float* grad_out, double* l1_sum_dev) {
    TDGS_REQUIRE(count >= 0, "negative count");
    if (count == 0) return TDGS_OK;
    TDGS_REQUIRE(rendered && gt && grad_out, "null arrays");
    hipStream_t s = (hipStream_t)stream;
    StageScope sc(TDGS_STAGE_LOSS, s);
    const float w = l1_weight / (float)count;
    k_l1_grad<<<(unsigned)ceil_div(count, 1024), 256, 0, s>>>(rendered, gt, count, w, dssim_weight, dssim_grad,
                                                              grad_out, l1_sum_dev);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_opacity_reset(void* stream, tdgs_gaussians* g, float max_logit, float* opacity_moments) {
    TDGS_TRY(check_gaussians(g, true));
    if (g->n == 0) return TDGS_OK;
    k_opacity_reset<<<(unsigned)ceil_div(g->n, 256), 256, 0, (hipStream_t)stream>>>(g->means_opacity, max_logit,
                                                                                  opacity_moments, g->n);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

int tdgs_sh_resize(void* stream, const float* src, int32_t h_src, float* dst, int32_t h_dst, int64_t n,
                   int32_t interleave) {
    TDGS_REQUIRE(h_src >= 1 && h_src <= 16 && h_dst >= 1 && h_dst <= 16, "bad coefficient counts");
    TDGS_REQUIRE(interleave == 1 || interleave == 2, "interleave must be 1 or 2");
    TDGS_REQUIRE(n >= 0 && src != dst, "bad arguments");
    if (n == 0) return TDGS_OK;
    TDGS_REQUIRE(src && dst, "null arrays");
    const int64_t total = (int64_t)interleave * h_dst * 3 * n;
    k_sh_resize<<<(unsigned)ceil_div(total, 256), 256, 0, (hipStream_t)stream>>>(src, h_src, dst, h_dst, n,
                                                                               interleave);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

}  // extern "C"
