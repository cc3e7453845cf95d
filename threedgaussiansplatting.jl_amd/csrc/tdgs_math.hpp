// tdgs_math.hpp — per-element mathematics of the render/train core, compiled both for
// gfx950 (hipcc) and for the host (g++ / host pass of hipcc).
//
// Every function here runs the same sequence of IEEE-754 single precision operations on
// the CPU and on the GPU: no FMA contraction (all translation units are built with
// -ffp-contract=off; fused multiply-adds are written as explicit fmaf), correctly rounded
// division and square root, and our own exp/log below instead of the platform libm. That
// is what makes keys, culling, tile rectangles, per-tile lists and last-contributor
// indices identical between the GPU kernels and the CPU restatement.
//
// Reference semantics followed (paths in the reference repository):
//   projection / culling   src/forward_core.jl:326-355, 411-517, src/cameras.jl:679-774
//   bounding boxes         src/forward_structs.jl:1303-1411
//   spherical harmonics    src/sh.jl:1-267
//   rotation / sigmoid     src/misc.jl:133-141, 235-237
//   tile blending          src/forward_core.jl:870-968
//   backward blending      src/backward_core.jl:226-286
//   backward projection    src/backward_core.jl:309-964
//   Adam                   src/optimizer.jl:941-953
#pragma once

#include <stdint.h>
#include <math.h>

#include "../../include/tdgs.h"

#ifdef __HIPCC__
#define TDGS_HD __host__ __device__ __forceinline__
#else
#define TDGS_HD inline
#endif

namespace tdgs {

// ------------------------------------------------------------------------------------
// Bits and elementary functions
// ------------------------------------------------------------------------------------

TDGS_HD uint32_t float_bits(float x) { return __builtin_bit_cast(uint32_t, x); }
TDGS_HD float bits_float(uint32_t u) { return __builtin_bit_cast(float, u); }
TDGS_HD int32_t float_bits_signed(float x) { return __builtin_bit_cast(int32_t, x); }

constexpr float kLn2Hi = 0.693145751953125f;          // 15 significant bits: n*kLn2Hi exact
constexpr float kLn2Lo = 1.42860682030941723212e-6f;  // ln 2 - kLn2Hi
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kInf = __builtin_inff();

// exp(r) for |r| <= ln2/2 (+ rounding): 1 + r + c2 r^2 + ... + c6 r^6 in Horner form. The
// coefficients are a least-squares fit of the relative error on that interval, reweighted
// towards equal ripple (Lawson's iteration) with the constant and linear terms held at 1,
// then rounded to float: fit error 4e-9 relative (the degree-7 Taylor polynomial this
// replaced needs one more FMA for 6e-9). The blending kernel's instruction sequence carries
// the same constants (kExpC*).
constexpr float kExpC2 = 0x1.fffffcp-2f, kExpC3 = 0x1.555492p-3f, kExpC4 = 0x1.5558f2p-5f,
                kExpC5 = 0x1.1239d8p-7f, kExpC6 = 0x1.6a2446p-10f;
TDGS_HD float exp_poly(float r) {
    float p = fmaf(kExpC6, r, kExpC5);
    p = fmaf(p, r, kExpC4);
    p = fmaf(p, r, kExpC3);
    p = fmaf(p, r, kExpC2);
    p = fmaf(p, r, 1.0f);
    return fmaf(p, r, 1.0f);
}

// exp(x). Cody & Waite (1980) argument reduction x = n ln2 + r, |r| <= ln2/2 (+ rounding),
// with ln2 split into an exactly multipliable head and a tail; exp(r) by exp_poly; result
// scaled by 2^n through the exponent field. Results below FLT_MIN flush to 0. Within 0.91
// ulp of exp in double on [-87, 88] (a sweep of every seventh float there).
TDGS_HD float exp_f(float x) {
    if (!(x > -87.33654475f)) return (x != x) ? x : 0.0f;
    if (x > 88.72283935f) return kInf;
    const float n = rintf(x * kLog2e);
    float r = fmaf(n, -kLn2Hi, x);
    r = fmaf(n, -kLn2Lo, r);
    float p = exp_poly(r);
    int ni = (int)n;                         // in [-126, 128]
    if (ni > 127) { p = p * 2.0f; ni = 127; }
    return p * bits_float((uint32_t)(ni + 127) << 23);
}

// exp_f without branches, for wavefront loops: the same operations on a clamped copy of x
// (identical to x wherever exp_f takes its polynomial path), the special cases chosen by
// selects. Equal to exp_f(x) bit for bit for every x, NaN and infinities included.
TDGS_HD float exp_f_sel(float x) {
    const float xc = fminf(fmaxf(x, -88.0f), 89.0f);
    const float n = rintf(xc * kLog2e);
    float r = fmaf(n, -kLn2Hi, xc);
    r = fmaf(n, -kLn2Lo, r);
    float p = exp_poly(r);
    int ni = (int)n;                         // in [-127, 128] after the clamp
    const bool big = ni > 127;
    p = big ? p * 2.0f : p;
    ni = big ? 127 : ni;
    const float v = p * bits_float((uint32_t)((ni + 127) & 0xff) << 23);
    return x > 88.72283935f ? kInf : (x > -87.33654475f ? v : ((x != x) ? x : 0.0f));
}

// exp_f on its polynomial range only: equal to exp_f(x) bit for bit for -87 <= x <= 88
// (there n = rint(x log2 e) lies in [-126, 127], so neither special case nor the overflow
// adjustment of exp_f applies). Callers check the range.
TDGS_HD float exp_f_core(float x) {
    const float n = rintf(x * kLog2e);
    float r = fmaf(n, -kLn2Hi, x);
    r = fmaf(n, -kLn2Lo, r);
    return exp_poly(r) * bits_float((uint32_t)((int)n + 127) << 23);
}

// log(x) for x > 0. x = m 2^e with m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(s),
// s = (m-1)/(m+1), by the odd series of atanh to s^11 (|s| <= 0.1716, remainder < 1e-11);
// e ln2 added with the split constant. About 1 ulp. Subnormal inputs are scaled first.
TDGS_HD float log_f(float x) {
    if (!(x > 0.0f)) return (x == 0.0f) ? -kInf : bits_float(0x7fc00000u);
    if (x == kInf) return kInf;
    int bias = 0;
    if (x < 1.17549435e-38f) { x = x * 8388608.0f; bias = -23; }
    const uint32_t u = float_bits(x);
    int e = (int)(u >> 23) - 127 + bias;
    float m = bits_float((u & 0x007fffffu) | 0x3f800000u);
    if (m > 1.41421354f) { m = m * 0.5f; e += 1; }
    const float f = m - 1.0f;                 // exact
    const float s = f / (m + 1.0f);
    const float z = s * s;
    float p = 1.0f / 11.0f;
    p = fmaf(p, z, 1.0f / 9.0f);
    p = fmaf(p, z, 1.0f / 7.0f);
    p = fmaf(p, z, 1.0f / 5.0f);
    p = fmaf(p, z, 1.0f / 3.0f);
    const float s2 = s + s;
    const float logm = fmaf(s2 * z, p, s2);
    const float ef = (float)e;
    return fmaf(ef, kLn2Hi, fmaf(ef, kLn2Lo, logm));
}

// sigmoid (src/misc.jl:235-237).
TDGS_HD float sigmoid_f(float x) { return 1.0f / (1.0f + exp_f(-x)); }

// cos(2 pi t) and sin(2 pi t) for t in [0, 1): quadrant reduction on 4t, then Taylor
// polynomials of cos/sin on |y| <= pi/4 (degree 8 / 9). Used only by the split sampler.
TDGS_HD void sincos_2pi(float t, float* s_out, float* c_out) {
    const float q = rintf(t * 4.0f);           // quadrant 0..4
    const float y = (t * 4.0f - q) * 1.57079632679489662f;   // |y| <= pi/4
    const float y2 = y * y;
    float c = 2.48015873015873e-5f;            // 1/8!
    c = fmaf(c, y2, -1.38888888888889e-3f);
    c = fmaf(c, y2, 4.16666666666667e-2f);
    c = fmaf(c, y2, -0.5f);
    c = fmaf(c, y2, 1.0f);
    float s = 2.75573192239859e-6f;            // 1/9!
    s = fmaf(s, y2, -1.98412698412698e-4f);
    s = fmaf(s, y2, 8.33333333333333e-3f);
    s = fmaf(s, y2, -1.66666666666667e-1f);
    s = fmaf(s * y2, y, y);
    const int qi = ((int)q) & 3;
    float so, co;
    if (qi == 0) { so = s; co = c; }
    else if (qi == 1) { so = c; co = -s; }
    else if (qi == 2) { so = -s; co = -c; }
    else { so = -c; co = s; }
    *s_out = so;
    *c_out = co;
}

// Counter-based generator: a 64-bit mix (splitmix64 finaliser) of (seed, stream, draw).
TDGS_HD uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Two standard normal draws for (seed, stream, pair) by the Box-Muller transform.
TDGS_HD void normal_pair(uint64_t seed, uint64_t stream, uint32_t pair, float* n0, float* n1) {
    const uint64_t h = mix64(seed ^ mix64(stream * 0x100000001b3ull + pair));
    // 24-bit uniforms; u1 in (0, 1], u2 in [0, 1)
    const float u1 = (float)((uint32_t)(h >> 40) + 1u) * 5.9604644775390625e-8f;
    const float u2 = (float)((uint32_t)(h >> 8) & 0xffffffu) * 5.9604644775390625e-8f;
    const float rad = sqrtf(-2.0f * log_f(u1));
    float s, c;
    sincos_2pi(u2, &s, &c);
    *n0 = rad * c;
    *n1 = rad * s;
}

// ------------------------------------------------------------------------------------
// Camera, projection, covariance
// ------------------------------------------------------------------------------------

// depth = P[3,1:3] . m + P[3,4]  (src/cameras.jl:679-682); same expression as the third
// homogeneous coordinate in project().
TDGS_HD float depth_of(const float* P, float x, float y, float z) {
    return fmaf(P[10], z, fmaf(P[9], y, P[8] * x)) + P[11];
}

// project_with_depth (src/cameras.jl:714-722).
TDGS_HD void project_point(const float* P, float x, float y, float z, float* mux, float* muy,
                           float* depth) {
    const float p = fmaf(P[2], z, fmaf(P[1], y, P[0] * x)) + P[3];
    const float q = fmaf(P[6], z, fmaf(P[5], y, P[4] * x)) + P[7];
    const float r = depth_of(P, x, y, z);
    *mux = p / r;
    *muy = q / r;
    *depth = r;
}

TDGS_HD float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }

// get_linearized_projection_2d (src/cameras.jl:755-774):
// J = (1/r) [1 0 -mu_x; 0 1 -mu_y] P[1:3,1:3], row-major 2x3.
TDGS_HD void jacobian(const float* P, float mux, float muy, float depth, float J[6]) {
    const float id = 1.0f / depth;
    for (int j = 0; j < 3; ++j) {
        J[j] = fmaf(-mux, P[8 + j], P[j]) * id;
        J[3 + j] = fmaf(-muy, P[8 + j], P[4 + j]) * id;
    }
}

// quaternion_to_rotation_matrix (src/misc.jl:133-141), row-major R[3*i + j].
TDGS_HD void quat_to_rot(float q0, float q1, float q2, float q3, float R[9]) {
    const float ss = fmaf(q3, q3, fmaf(q2, q2, fmaf(q1, q1, q0 * q0)));
    const float k = sqrtf(2.0f / ss);
    const float r = q0 * k, x = q1 * k, y = q2 * k, z = q3 * k;
    R[0] = 1.0f - fmaf(y, y, z * z);
    R[1] = fmaf(x, y, -(r * z));
    R[2] = fmaf(x, z, r * y);
    R[3] = fmaf(x, y, r * z);
    R[4] = 1.0f - fmaf(x, x, z * z);
    R[5] = fmaf(y, z, -(r * x));
    R[6] = fmaf(x, z, -(r * y));
    R[7] = fmaf(y, z, r * x);
    R[8] = 1.0f - fmaf(x, x, y * y);
}

// Lower half [S11, S21, S22] of (J R diag(s)) (J R diag(s))^T (src/gaussians.jl:1328-1331).
TDGS_HD void cov2d_trainable(const float J[6], const float R[9], const float s[3], float out[3]) {
    float T[6];
    for (int i = 0; i < 2; ++i) {
        for (int k = 0; k < 3; ++k) {
            const float jr = fmaf(J[3 * i + 2], R[6 + k], fmaf(J[3 * i + 1], R[3 + k], J[3 * i] * R[k]));
            T[3 * i + k] = jr * s[k];
        }
    }
    out[0] = fmaf(T[2], T[2], fmaf(T[1], T[1], T[0] * T[0]));
    out[1] = fmaf(T[5], T[2], fmaf(T[4], T[1], T[3] * T[0]));
    out[2] = fmaf(T[5], T[5], fmaf(T[4], T[4], T[3] * T[3]));
}

// Lower half of J V J^T for V given by its lower half (src/gaussians.jl:1324-1327).
TDGS_HD void cov2d_from_cov3d(const float J[6], const float v[6], float out[3]) {
    const float V[9] = {v[0], v[1], v[2], v[1], v[3], v[4], v[2], v[4], v[5]};
    float JV[6];
    for (int i = 0; i < 2; ++i)
        for (int k = 0; k < 3; ++k)
            JV[3 * i + k] = fmaf(J[3 * i + 2], V[6 + k], fmaf(J[3 * i + 1], V[3 + k], J[3 * i] * V[k]));
    out[0] = fmaf(JV[2], J[2], fmaf(JV[1], J[1], JV[0] * J[0]));
    out[1] = fmaf(JV[5], J[2], fmaf(JV[4], J[1], JV[3] * J[0]));
    out[2] = fmaf(JV[5], J[5], fmaf(JV[4], J[4], JV[3] * J[3]));
}

// ------------------------------------------------------------------------------------
// Spherical harmonics (src/sh.jl)
// ------------------------------------------------------------------------------------

constexpr float kSH[16] = {
    0.28209479177387814f,  0.4886025119029199f,  0.4886025119029199f,  0.4886025119029199f,
    1.0925484305920792f,  -1.0925484305920792f,  0.31539156525252005f, -1.0925484305920792f,
    0.5462742152960396f,  -0.5900435899266435f,  2.890611442640554f,   -0.4570457994644658f,
    0.3731763325901154f,  -0.4570457994644658f,  1.445305721320277f,   -0.5900435899266435f};

// evaluate_sh_basis_function (src/sh.jl:123-149) for all (degree+1)^2 basis functions.
TDGS_HD void sh_basis(int degree, float x, float y, float z, float b[16]) {
    b[0] = kSH[0];
    if (degree < 1) return;
    b[1] = -y * kSH[1];
    b[2] = z * kSH[2];
    b[3] = -x * kSH[3];
    if (degree < 2) return;
    const float xx = x * x, yy = y * y, zz = z * z;
    b[4] = x * y * kSH[4];
    b[5] = y * z * kSH[5];
    b[6] = (2.0f * zz - xx - yy) * kSH[6];
    b[7] = x * z * kSH[7];
    b[8] = (xx - yy) * kSH[8];
    if (degree < 3) return;
    b[9] = y * (3.0f * xx - yy) * kSH[9];
    b[10] = x * y * z * kSH[10];
    b[11] = y * (4.0f * zz - xx - yy) * kSH[11];
    b[12] = z * (2.0f * zz - 3.0f * (xx + yy)) * kSH[12];
    b[13] = x * (4.0f * zz - xx - yy) * kSH[13];
    b[14] = z * (xx - yy) * kSH[14];
    b[15] = x * (xx - 3.0f * yy) * kSH[15];
}

// sh_coeffs_to_color (src/sh.jl:38-112): per channel sum_k b_k c_k + 0.5, clamped below
// at 0; only the first (degree+1)^2 coefficients of each channel are used. This is one
// channel, cc pointing at its coefficients.
TDGS_HD float sh_channel_to_color(int degree, const float* cc, const float b[16]) {
    float v = b[0] * cc[0];
    if (degree >= 1) {
        v += fmaf(b[3], cc[3], fmaf(b[2], cc[2], b[1] * cc[1]));
        if (degree >= 2) {
            float t = b[4] * cc[4];
            for (int k = 5; k < 9; ++k) t = fmaf(b[k], cc[k], t);
            v += t;
            if (degree >= 3) {
                float u = b[9] * cc[9];
                for (int k = 10; k < 16; ++k) u = fmaf(b[k], cc[k], u);
                v += u;
            }
        }
    }
    v += 0.5f;
    return v < 0.0f ? 0.0f : v;
}

// All three channels; coeffs points at one Gaussian's (h_storage, 3) block.
TDGS_HD void sh_to_color(int degree, const float* coeffs, int h_storage, const float b[16],
                         float rgb[3]) {
    for (int c = 0; c < 3; ++c) rgb[c] = sh_channel_to_color(degree, coeffs + c * h_storage, b);
}

// ------------------------------------------------------------------------------------
// Culling and projection of one Gaussian
// ------------------------------------------------------------------------------------

// Opacity of Gaussian g as the renderer sees it (sigmoid of the logit when trainable).
TDGS_HD float opacity_of(int kind, float stored) {
    return kind == TDGS_TRAINABLE ? sigmoid_f(stored) : stored;
}

TDGS_HD bool on_extended_screen(const tdgs_render_options& o, float mux, float muy) {
    return o.clip_x_min < mux && mux <= o.clip_x_max && o.clip_y_min < muy && muy <= o.clip_y_max;
}

// fill_keep_gaussians_kernel! (src/forward_core.jl:326-355).
TDGS_HD bool keep_gaussian(const tdgs_camera& cam, const tdgs_render_options& o, float x,
                           float y, float z, float a) {
    if (!(a >= o.min_alpha)) return false;
    if (o.clip_mode == TDGS_CLIP_FILTER) {
        float mux, muy, d;
        project_point(cam.P, x, y, z, &mux, &muy, &d);
        return on_extended_screen(o, mux, muy) && cam.near_z < d && d <= cam.far_z &&
               a > o.min_alpha;
    }
    const float d = depth_of(cam.P, x, y, z);
    return cam.near_z < d && d <= cam.far_z;
}

// Result of projecting one kept Gaussian (project_fgaussians_kernel!, forward_core.jl:411-517).
struct Projected {
    float mux, muy, a, m11, m21, m22, depth;
    int32_t rect[4];   // tile ids [tx_min, ty_min, tx_max, ty_max] (valid when count > 0)
    int32_t count;     // overlapped tiles; 0 means empty bounding box
};

// Geometry part of the projection: everything except the colour. params holds for a
// trainable Gaussian [log s (3), quaternion (4)], for a render-only one the 6 lower
// covariance entries.
TDGS_HD Projected project_geometry(const tdgs_camera& cam, const tdgs_render_options& o,
                                   const tdgs_tiling& t, int kind, float x, float y, float z,
                                   float a, const float* params) {
    Projected pr;
    float mux, muy, depth;
    project_point(cam.P, x, y, z, &mux, &muy, &depth);
    float J[6];
    if (o.clip_mode == TDGS_CLIP_CLAMP) {
        jacobian(cam.P, clampf(mux, o.clip_x_min, o.clip_x_max),
                 clampf(muy, o.clip_y_min, o.clip_y_max), depth, J);
    } else {
        jacobian(cam.P, mux, muy, depth, J);
    }
    float cov[3];
    if (kind == TDGS_TRAINABLE) {
        float R[9];
        quat_to_rot(params[3], params[4], params[5], params[6], R);
        const float s[3] = {exp_f(params[0]), exp_f(params[1]), exp_f(params[2])};
        cov2d_trainable(J, R, s, cov);
    } else {
        cov2d_from_cov3d(J, params, cov);
    }
    float det0 = 0.0f;
    if (o.antialiasing) det0 = fmaxf(fmaf(cov[0], cov[2], -(cov[1] * cov[1])), 0.0f);
    cov[0] += o.dilation_x;
    cov[2] += o.dilation_y;
    const float idet = 1.0f / fmaf(cov[0], cov[2], -(cov[1] * cov[1]));
    if (o.antialiasing) a = a * fmaxf(o.aa_min_factor, sqrtf(det0 * idet));

    pr.mux = mux;
    pr.muy = muy;
    pr.a = a;
    pr.depth = depth;
    pr.m11 = cov[2] * idet;
    pr.m21 = -cov[1] * idet;
    pr.m22 = cov[0] * idet;
    pr.count = 0;
    pr.rect[0] = pr.rect[1] = pr.rect[2] = pr.rect[3] = 0;

    // _get_bbox_cts_px_cov + _get_bbox_discrete_px (src/forward_structs.jl:1303-1411)
    if (!(a >= o.min_alpha)) return pr;
    const float gamma = 2.0f * log_f(a / o.min_alpha);
    const float rx = sqrtf(gamma * cov[0]);
    const float ry = sqrtf(gamma * cov[2]);
    const float l = ceilf((mux - rx) + 0.5f);
    const float tp = ceilf((muy - ry) + 0.5f);
    const float rt = rintf(mux + rx);          // round half to even, as Julia's round
    const float bt = rintf(muy + ry);
    if (l != l || tp != tp || rt != rt || bt != bt) return pr;
    const float left = fmaxf(1.0f, l), top = fmaxf(1.0f, tp);
    const float right = fminf((float)cam.width, rt), bottom = fminf((float)cam.height, bt);
    if (left > right || top > bottom) return pr;
    const int32_t il = (int32_t)left, itp = (int32_t)top, ir = (int32_t)right, ib = (int32_t)bottom;
    // rectangle_to_tile_ids(..., Val(false)): ceil(k / tile) on integers >= 1
    pr.rect[0] = (il + t.tile_width - 1) / t.tile_width;
    pr.rect[1] = (itp + t.tile_height - 1) / t.tile_height;
    pr.rect[2] = (ir + t.tile_width - 1) / t.tile_width;
    pr.rect[3] = (ib + t.tile_height - 1) / t.tile_height;
    pr.count = (pr.rect[2] - pr.rect[0] + 1) * (pr.rect[3] - pr.rect[1] + 1);
    return pr;
}

// Colour of a projected Gaussian: SH evaluated along normalize(m - camera position).
TDGS_HD void view_sh_basis(const tdgs_camera& cam, int degree, float x, float y, float z, float b[16]) {
    if (degree > 0) {
        const float vx = x - cam.position[0], vy = y - cam.position[1], vz = z - cam.position[2];
        const float inv = 1.0f / sqrtf(fmaf(vz, vz, fmaf(vy, vy, vx * vx)));
        sh_basis(degree, vx * inv, vy * inv, vz * inv, b);
    } else {
        b[0] = kSH[0];
    }
}

TDGS_HD void project_color(const tdgs_camera& cam, int degree, const float* coeffs,
                           int h_storage, float x, float y, float z, float rgb[3]) {
    float b[16];
    view_sh_basis(cam, degree, x, y, z, b);
    sh_to_color(degree, coeffs, h_storage, b, rgb);
}

// Key of one duplicated Gaussian (forward_core.jl:583-587). The depth bits are
// sign-extended into the 64-bit key exactly as Int64(tile) << 32 | Int64(::Int32) does.
TDGS_HD int64_t make_key(int32_t tile, float depth) {
    const int64_t hi = (int64_t)tile << 32;
    return hi | (int64_t)float_bits_signed(depth);
}

// ------------------------------------------------------------------------------------
// Tile blending
// ------------------------------------------------------------------------------------

// Per-record evaluation parameters in tile-local pixel coordinates, with the opacity folded
// into the exponent (render_tiles_kernel!, forward_core.jl:870-889):
// exponent(u, v) = p0 u^2 + p1 v^2 + p2 u v + p3 u + p4 v + p5, u = px_in_tile - 0.5.
TDGS_HD void blend_params(float mux, float muy, float a, float m11, float m21, float m22,
                          float u0, float v0, float p[6]) {
    const float du = mux - u0, dv = muy - v0;
    const float m11du = m11 * du, m21du = m21 * du, m22dv = m22 * dv;
    p[0] = -0.5f * m11;
    p[1] = -0.5f * m22;
    p[2] = -m21;
    p[3] = fmaf(m21, dv, m11du);
    p[4] = m21du + m22dv;
    const float q = fmaf(m11du, du, m22dv * dv);
    p[5] = fmaf(-0.5f, q, fmaf(-m21du, dv, log_f(a)));
}

TDGS_HD float blend_exponent(const float p[6], float u, float v, float uu, float uv, float vv) {
    return fmaf(p[0], uu, fmaf(p[1], vv, fmaf(p[2], uv, fmaf(p[3], u, fmaf(p[4], v, p[5])))));
}

// Exponent of the Gaussian in the backward pass (direct form, backward_core.jl:236-240), at
// global continuous pixel coordinates (cu, cv) = (u - 0.5, v - 0.5).
TDGS_HD float backward_exponent(float cu, float cv, float mux, float muy, float m11, float m21,
                                float m22, float* du_out, float* dv_out) {
    const float du = cu - mux, dv = cv - muy;
    *du_out = du;
    *dv_out = dv;
    const float q = fmaf(m11 * du, du, m22 * dv * dv);
    return fmaf(-0.5f, q, -(m21 * du) * dv);
}

// Gaussian value in the backward pass (direct form, backward_core.jl:236-240).
TDGS_HD float backward_gaussian(float cu, float cv, float mux, float muy, float m11, float m21,
                                float m22, float* du_out, float* dv_out) {
    return exp_f(backward_exponent(cu, cv, mux, muy, m11, m21, m22, du_out, dv_out));
}

// Per-(pixel, Gaussian) gradient contribution of the backward blend
// (backward_core.jl:249-272). T is the transmittance after this Gaussian on entry and
// before it on exit; psi (partial colour) is updated. out = [dmu_x, dmu_y, da, dM11,
// dM21, dM22, dr, dg, db].
// inv1ma is 1 / (1 - alpha) (the CPU restatement divides; the GPU kernel uses the hardware
// reciprocal, within 1 ulp).
TDGS_HD void backward_pair(float alpha, float inv1ma, float G, float du, float dv, float m11, float m21,
                           float m22, const float c[3], const float g[3], float* T,
                           float psi[3], float out[9]) {
    const float Tn = *T * inv1ma;
    *T = Tn;
    const float tc0 = Tn * c[0], tc1 = Tn * c[1], tc2 = Tn * c[2];
    psi[0] = fmaf(alpha, tc0, psi[0]);
    psi[1] = fmaf(alpha, tc1, psi[1]);
    psi[2] = fmaf(alpha, tc2, psi[2]);
    const float dot = fmaf(g[2], tc2 - psi[2], fmaf(g[1], tc1 - psi[1], g[0] * (tc0 - psi[0])));
    const float dalpha = inv1ma * dot;
    const float aa = alpha * dalpha;
    out[0] = aa * fmaf(m21, dv, m11 * du);
    out[1] = aa * fmaf(m22, dv, m21 * du);
    out[2] = G * dalpha;
    const float h = -0.5f * aa;
    out[3] = h * (du * du);
    out[4] = h * (2.0f * du * dv);
    out[5] = h * (dv * dv);
    const float ta = Tn * alpha;
    out[6] = ta * g[0];
    out[7] = ta * g[1];
    out[8] = ta * g[2];
}

// ------------------------------------------------------------------------------------
// Backward projection of one filtered Gaussian (backward_core.jl:309-964)
// ------------------------------------------------------------------------------------

// transposed_color_normalized_direction_jacobian (src/sh.jl:175-267): Jt[3*i + c] =
// d colour_c / d dir_i. With exact == false the degree-3 term of basis 16 reads
// coefficient 15, as src/sh.jl:249 does.
TDGS_HD void color_dir_jacobian_t(int degree, const float rgb[3], float x, float y, float z,
                                  const float* coeffs, int h_storage, bool exact, float Jt[9]) {
    for (int i = 0; i < 9; ++i) Jt[i] = 0.0f;
    if (degree == 0) return;
    for (int c = 0; c < 3; ++c) {
        if (rgb[c] <= 0.0f) continue;
        const float* cc = coeffs + c * h_storage;
        float dx = -kSH[3] * cc[3];
        float dy = -kSH[1] * cc[1];
        float dz = kSH[2] * cc[2];
        if (degree >= 2) {
            float s = kSH[4] * cc[4];
            dx = fmaf(y, s, dx); dy = fmaf(x, s, dy);
            s = kSH[5] * cc[5];
            dy = fmaf(z, s, dy); dz = fmaf(y, s, dz);
            s = kSH[6] * cc[6];
            dx = fmaf(-2.0f * x, s, dx); dy = fmaf(-2.0f * y, s, dy); dz = fmaf(4.0f * z, s, dz);
            s = kSH[7] * cc[7];
            dx = fmaf(z, s, dx); dz = fmaf(x, s, dz);
            s = kSH[8] * cc[8];
            dx = fmaf(2.0f * x, s, dx); dy = fmaf(-2.0f * y, s, dy);
            if (degree >= 3) {
                const float xx = x * x, yy = y * y, zz = z * z;
                s = kSH[9] * cc[9];
                dx = fmaf(6.0f * x * y, s, dx); dy = fmaf(3.0f * (xx - yy), s, dy);
                s = kSH[10] * cc[10];
                dx = fmaf(y * z, s, dx); dy = fmaf(x * z, s, dy); dz = fmaf(x * y, s, dz);
                s = kSH[11] * cc[11];
                dx = fmaf(-2.0f * x * y, s, dx); dy = fmaf(4.0f * zz - xx - 3.0f * yy, s, dy);
                dz = fmaf(8.0f * y * z, s, dz);
                s = kSH[12] * cc[12];
                dx = fmaf(-6.0f * x * z, s, dx); dy = fmaf(-6.0f * y * z, s, dy);
                dz = fmaf(3.0f * (2.0f * zz - xx - yy), s, dz);
                s = kSH[13] * cc[13];
                dx = fmaf(4.0f * zz - 3.0f * xx - yy, s, dx); dy = fmaf(-2.0f * x * y, s, dy);
                dz = fmaf(8.0f * x * z, s, dz);
                s = kSH[14] * cc[14];
                dx = fmaf(2.0f * x * z, s, dx); dy = fmaf(-2.0f * y * z, s, dy);
                dz = fmaf(xx - yy, s, dz);
                s = kSH[15] * cc[exact ? 15 : 14];
                dx = fmaf(3.0f * (xx - yy), s, dx); dy = fmaf(-6.0f * x * y, s, dy);
            }
        }
        Jt[c] = dx;
        Jt[3 + c] = dy;
        Jt[6 + c] = dz;
    }
}

struct BackwardProjectIn {
    // 3D parameters
    float m[3];
    float logit;
    float logs[3];
    float q[4];
    const float* sh;   // (h_storage, 3) block of this Gaussian
    int h_storage;
    // 2D record (f2d)
    float mux, muy, a, m11, m21, m22, rgb[3];
    // 2D gradients [dmu_x, dmu_y, da, dM11, dM21, dM22, dr, dg, db]
    float g2[9];
};

struct BackwardProjectOut {
    float dm[3];
    float dlogit;
    float dlogs[3];
    float dq[4];
};

// backward_project_fgaussians_kernel! for a trainable Gaussian. SH coefficient gradients
// (compute_sh_coeffs_grad!) are written by sh_grad() below.
TDGS_HD BackwardProjectOut backward_project(const BackwardProjectIn& in, const tdgs_camera& cam,
                                            const tdgs_render_options& o) {
    BackwardProjectOut out;
    const float* P = cam.P;
    const float a0 = sigmoid_f(in.logit);
    const float da = in.g2[2];
    // opacity feature
    out.dlogit = o.antialiasing ? da * in.a * (1.0f - a0) : da * a0 * (1.0f - a0);

    // compute_cov2d_lower_grad (backward_core.jl:465-493)
    const float A = in.m11, B = in.m21, D = in.m22;
    const float gA = in.g2[3], gB = in.g2[4], gD = in.g2[5];
    const float a_sq = A * A, ab = A * B, b_sq = B * B, bd = B * D, d_sq = D * D, ad = A * D;
    float dS[3];
    dS[0] = -fmaf(b_sq, gD, fmaf(ab, gB, a_sq * gA));
    dS[1] = -fmaf(2.0f * bd, gD, fmaf(b_sq + ad, gB, 2.0f * ab * gA));
    dS[2] = -fmaf(d_sq, gD, fmaf(bd, gB, b_sq * gA));
    if (o.antialiasing) {
        // opacity correction f = sqrt(det0 / det) (backward_core.jl:480-490): the reference adds
        // a0 dL/da d(f^2)/dSigma, in terms of M = Sigma^-1 = [A B; B D]:
        //   d(f^2)/dSigma = [A^2 Dx + B^2 Dy - A delta, 2 B (A Dx + D Dy - delta), B^2 Dx + D^2 Dy - D delta]
        // with delta = (AD - B^2) Dx Dy, written with B^2 Dx in the first entry as the reference
        // does (the same for equal dilations). TDGS_FLAG_EXACT_AA_GRADIENT divides by 2 f (the
        // derivative of f itself), and gives 0 where f was clamped to aa_min.
        const float Dx = o.dilation_x, Dy = o.dilation_y;
        const float det = (ad - b_sq) * Dx * Dy;
        float k = a0 * da;
        const bool exact = (o.flags & TDGS_FLAG_EXACT_AA_GRADIENT) != 0;
        if (exact) {
            const float f = in.a / a0;
            k = f > o.aa_min_factor ? k / (2.0f * f) : 0.0f;
        }
        dS[0] = fmaf(k, a_sq * Dx + b_sq * (exact ? Dy : Dx) - A * det, dS[0]);
        dS[1] = fmaf(k, 2.0f * B * (A * Dx + D * Dy - det), dS[1]);
        dS[2] = fmaf(k, b_sq * Dx + d_sq * Dy - D * det, dS[2]);
    }

    // mean3d gradient from the 2D mean
    const float depth = depth_of(P, in.m[0], in.m[1], in.m[2]);
    const bool clamp_mode = o.clip_mode == TDGS_CLIP_CLAMP;
    const float mcx = clamp_mode ? clampf(in.mux, o.clip_x_min, o.clip_x_max) : in.mux;
    const float mcy = clamp_mode ? clampf(in.muy, o.clip_y_min, o.clip_y_max) : in.muy;
    float Jc[6];
    jacobian(P, mcx, mcy, depth, Jc);
    const float gx = in.g2[0], gy = in.g2[1];
    float dm[3];
    if (!clamp_mode) {
        for (int k = 0; k < 3; ++k) dm[k] = fmaf(Jc[3 + k], gy, Jc[k] * gx);
    } else {
        const float id = 1.0f / depth;
        const float w0 = id * gx, w1 = id * gy, w2 = id * -fmaf(in.muy, gy, in.mux * gx);
        for (int k = 0; k < 3; ++k) dm[k] = fmaf(P[8 + k], w2, fmaf(P[4 + k], w1, P[k] * w0));
    }

    // 3D covariance V = (R S)(R S)^T
    float R[9];
    quat_to_rot(in.q[0], in.q[1], in.q[2], in.q[3], R);
    const float s[3] = {exp_f(in.logs[0]), exp_f(in.logs[1]), exp_f(in.logs[2])};
    float V[9];
    for (int i = 0; i < 3; ++i) {
        for (int j = 0; j < 3; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < 3; ++k) {
                const float rik = R[3 * i + k] * s[k];
                acc = fmaf(rik, R[3 * j + k] * s[k], acc);
            }
            V[3 * i + j] = acc;
        }
    }
    // symmetrise from the lower half (lower_matrix_sv)
    V[1] = V[3]; V[2] = V[6]; V[5] = V[7];

    // Transposed_dsigma_dm (backward_core.jl:789-922): dm_k += -1/r^2 sum_p T(k,p) dS_p with
    // T(k,(i,j)) = S_k[i][j] + S_k[j][i], S_k = Dk V Jc^T and Dk = dJ/dm_k (prefactor removed).
    const bool dx_in = clamp_mode ? (o.clip_x_min < mcx && mcx <= o.clip_x_max) : true;
    const bool dy_in = clamp_mode ? (o.clip_y_min < mcy && mcy <= o.clip_y_max) : true;
    float dJp[2][3][3];  // [row i][col j][p component]
    for (int j = 0; j < 3; ++j) {
        const float p3j = P[8 + j];
        dJp[0][j][0] = dx_in ? p3j : 0.0f;
        dJp[1][j][0] = 0.0f;
        dJp[0][j][1] = 0.0f;
        dJp[1][j][1] = dy_in ? p3j : 0.0f;
        dJp[0][j][2] = fmaf(-(mcx + mcx), p3j, P[j]);
        dJp[1][j][2] = fmaf(-(mcy + mcy), p3j, P[4 + j]);
    }
    float W[6];  // V Jc^T, 3x2 row-major W[2*a + j]
    for (int r = 0; r < 3; ++r)
        for (int j = 0; j < 2; ++j)
            W[2 * r + j] = fmaf(V[3 * r + 2], Jc[3 * j + 2],
                                fmaf(V[3 * r + 1], Jc[3 * j + 1], V[3 * r] * Jc[3 * j]));
    const float mrsq = -1.0f / (depth * depth);
    for (int k = 0; k < 3; ++k) {
        float Dk[6];
        for (int i = 0; i < 2; ++i)
            for (int j = 0; j < 3; ++j)
                Dk[3 * i + j] = fmaf(dJp[i][j][2], P[8 + k],
                                     fmaf(dJp[i][j][1], P[4 + k], dJp[i][j][0] * P[k]));
        float S[4];
        for (int i = 0; i < 2; ++i)
            for (int j = 0; j < 2; ++j)
                S[2 * i + j] = fmaf(Dk[3 * i + 2], W[4 + j],
                                    fmaf(Dk[3 * i + 1], W[2 + j], Dk[3 * i] * W[j]));
        const float t = fmaf(2.0f * S[3], dS[2], fmaf(S[2] + S[1], dS[1], 2.0f * S[0] * dS[0]));
        dm[k] = fmaf(mrsq, t, dm[k]);
    }

    // colour path: (1/|v|)(I - n n^T) Jt_SH dc
    const float vx = in.m[0] - cam.position[0], vy = in.m[1] - cam.position[1],
                vz = in.m[2] - cam.position[2];
    const float inv_vn = 1.0f / sqrtf(fmaf(vz, vz, fmaf(vy, vy, vx * vx)));
    const float nx = vx * inv_vn, ny = vy * inv_vn, nz = vz * inv_vn;
    float Jt[9];
    color_dir_jacobian_t(o.sh_degree, in.rgb, nx, ny, nz, in.sh, in.h_storage,
                         (o.flags & TDGS_FLAG_EXACT_SH_JACOBIAN) != 0, Jt);
    const float* dc = in.g2 + 6;
    float dn[3];
    for (int i = 0; i < 3; ++i)
        dn[i] = fmaf(Jt[3 * i + 2], dc[2], fmaf(Jt[3 * i + 1], dc[1], Jt[3 * i] * dc[0]));
    const float nd = fmaf(nz, dn[2], fmaf(ny, dn[1], nx * dn[0]));
    dm[0] = fmaf(inv_vn, fmaf(-nx, nd, dn[0]), dm[0]);
    dm[1] = fmaf(inv_vn, fmaf(-ny, nd, dn[1]), dm[1]);
    dm[2] = fmaf(inv_vn, fmaf(-nz, nd, dn[2]), dm[2]);
    out.dm[0] = dm[0]; out.dm[1] = dm[1]; out.dm[2] = dm[2];

    // dV (lower 6) = Transposed_dsigma_dv(Jc) dS (backward_core.jl:513-563)
    // sigma lower index p -> (pi, qi): (0,0), (1,0), (1,1); v lower index -> (r, s).
    const int vr[6] = {0, 1, 2, 1, 2, 2};
    const int vs[6] = {0, 0, 0, 1, 1, 2};
    const int sp[3] = {0, 1, 1};
    const int sq[3] = {0, 0, 1};
    float dv[6];
    for (int jv = 0; jv < 6; ++jv) {
        const int r = vr[jv], c = vs[jv];
        float acc = 0.0f;
        for (int i = 0; i < 3; ++i) {
            const float* J0 = Jc + 3 * sp[i];
            const float* J1 = Jc + 3 * sq[i];
            float term = J0[r] * J1[c];
            if (r != c) term = fmaf(J0[c], J1[r], term);
            acc = fmaf(term, dS[i], acc);
        }
        dv[jv] = acc;
    }
    // scaling: ds_j = 2 s_j sum_i dv_i R[p_i, j] R[q_i, j]; d(log s) = ds * s
    for (int j = 0; j < 3; ++j) {
        float acc = 0.0f;
        for (int iv = 0; iv < 6; ++iv) acc = fmaf(dv[iv], R[3 * vr[iv] + j] * R[3 * vs[iv] + j], acc);
        const float ds = 2.0f * (s[j] * acc);
        out.dlogs[j] = ds * s[j];
    }
    // rotation: dR[k][l] = s_l^2 (dv[phi(k,k)] R[k][l] + sum_i dv[phi(i,k)] R[i][l])
    const int phi[9] = {0, 1, 2, 1, 3, 4, 2, 4, 5};
    float dR[9];
    for (int k = 0; k < 3; ++k) {
        for (int l = 0; l < 3; ++l) {
            float acc = dv[phi[4 * k]] * R[3 * k + l];
            for (int i = 0; i < 3; ++i) acc = fmaf(dv[phi[3 * i + k]], R[3 * i + l], acc);
            dR[3 * k + l] = (s[l] * s[l]) * acc;
        }
    }
    // compute_normed_q_grad (backward_core.jl:734-774) and the normalisation Jacobian
    const float qn2 = fmaf(in.q[3], in.q[3], fmaf(in.q[2], in.q[2], fmaf(in.q[1], in.q[1], in.q[0] * in.q[0])));
    const float inv_qn = 1.0f / sqrtf(qn2);
    const float r = in.q[0] * inv_qn, x = in.q[1] * inv_qn, y = in.q[2] * inv_qn, z = in.q[3] * inv_qn;
    const float m2x = -(x + x), m2y = -(y + y), m2z = -(z + z);
    const float Ar[9] = {0.0f, -z, y, z, 0.0f, -x, -y, x, 0.0f};
    const float Ax[9] = {0.0f, y, z, y, m2x, -r, z, r, m2x};
    const float Ay[9] = {m2y, x, r, x, 0.0f, z, -r, z, m2y};
    const float Az[9] = {m2z, -r, x, r, m2z, y, x, y, 0.0f};
    float dqh[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < 9; ++i) {
        dqh[0] = fmaf(Ar[i], dR[i], dqh[0]);
        dqh[1] = fmaf(Ax[i], dR[i], dqh[1]);
        dqh[2] = fmaf(Ay[i], dR[i], dqh[2]);
        dqh[3] = fmaf(Az[i], dR[i], dqh[3]);
    }
    for (int i = 0; i < 4; ++i) dqh[i] = 2.0f * dqh[i];
    const float qh[4] = {r, x, y, z};
    const float qd = fmaf(qh[3], dqh[3], fmaf(qh[2], dqh[2], fmaf(qh[1], dqh[1], qh[0] * dqh[0])));
    for (int i = 0; i < 4; ++i) out.dq[i] = inv_qn * fmaf(-qh[i], qd, dqh[i]);
    return out;
}

// compute_sh_coeffs_grad! (backward_core.jl:936-964): dsh[k + c h] = dc_c * b_k(dir) for
// the first (degree+1)^2 coefficients of each channel (the colour >= 0 gate always holds).
TDGS_HD void sh_grad_basis(const tdgs_camera& cam, int degree, const float m[3], float b[16]) {
    if (degree > 0) {
        const float vx = m[0] - cam.position[0], vy = m[1] - cam.position[1], vz = m[2] - cam.position[2];
        const float inv = 1.0f / sqrtf(fmaf(vz, vz, fmaf(vy, vy, vx * vx)));
        sh_basis(degree, vx * inv, vy * inv, vz * inv, b);
    } else {
        b[0] = kSH[0];
    }
}

// ------------------------------------------------------------------------------------
// Adam (src/optimizer.jl:941-953). bc1 = 1 - beta1^t, bc2 = 1 - beta2^t are computed once
// per step by the host.
// ------------------------------------------------------------------------------------
TDGS_HD void adam_scalar(float& p, float g, float& m1, float& m2, float lr, float beta1,
                         float beta2, float omb1, float omb2, float bc1, float bc2, float eps) {
    const float n1 = fmaf(beta1, m1, omb1 * g);
    const float n2 = fmaf(beta2, m2, omb2 * (g * g));
    const float h1 = n1 / bc1;
    const float h2 = n2 / bc2;
    p = p - (lr * h1) / (sqrtf(h2) + eps);
    m1 = n1;
    m2 = n2;
}

}  // namespace tdgs
