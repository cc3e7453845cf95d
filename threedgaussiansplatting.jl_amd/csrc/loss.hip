// loss.hip — training loss of training_step! (src/training.jl:196-217) on gfx950:
// L = (1 - lambda) * mean|K - I| + lambda * DSSIM(K, I), DSSIM = 1 - SSIM
// (docs/src/math.md:125-126), and dL/dK.
//
// SSIM (Wang et al. 2004): per colour channel, an 11 x 11 Gaussian window with sigma 1.5
// (normalised), C1 = 0.01^2, C2 = 0.03^2, zero padding outside the image, averaged over
// every pixel and channel. Two launches:
//   k_ssim_forward   filters x, y, x^2, y^2, xy with the separable window (LDS tile with a
//                    5-pixel halo), evaluates the SSIM map S and its partial derivatives
//                    D1 = dS/dmu_x, D2 = dS/dE[x^2], D3 = dS/dE[xy] per pixel, and sums S
//                    and |x - y| per workgroup (one partial pair per workgroup; workgroup 0
//                    of the backward launch adds them to the caller's sums, so no workgroup
//                    waits on an atomic to a shared address)
//   k_ssim_backward  filters D1, D2, D3 with the same window and forms
//                    dL/dx = (1-lambda) sign(x - y)/N - lambda/N (G*D1 + 2 x G*D2 + y G*D3)
// Images use the reference layout 3 x h x w (pixel (v, u) channel c at 3 (v + h u) + c).
// The reference computes DSSIM with FastCUDASSIM.jl, whose source is not available; its
// window and boundary conventions are therefore not pinned.
#include "internal.hpp"

namespace tdgs {

constexpr int kSsimT = 16;             // output tile: 16 x 16 pixels
constexpr int kSsimR = 5;              // window radius
constexpr int kSsimIn = kSsimT + 2 * kSsimR;
constexpr float kC1 = 0.01f * 0.01f;
constexpr float kC2 = 0.03f * 0.03f;

// Both kernels filter with sliding windows held in registers. Pass 1 (along v, the contiguous
// image axis): a thread takes one input column of the 26 x 26 tile and one quantity (or one
// colour channel), loads the 26 (or 18 for half a column) inputs once and produces 16 (or 8)
// outputs. Pass 2 (along u): a thread takes one output row and one filtered quantity, loads its
// 26 pass-1 values and produces the 16 outputs. Each LDS value is read about once per pass
// instead of once per window tap. LDS rows have 27 entries (odd), so lanes reading the same
// entry of consecutive rows fall on distinct banks.
constexpr int kRow = kSsimIn + 1;      // 27: LDS row length of a column / filtered row
constexpr int kQF = 15;                // forward filtered quantities: 5 per channel
constexpr int kQB = 9;                 // backward filtered quantities: D1, D2, D3 per channel
constexpr int kOutPitch = 17;          // pass-2 output: value q of pixel (ou, ov) at (ou*16+ov)*17+q

// XCD-aware tile order (xcd_band_item): each XCD takes one contiguous band of tiles (v
// fastest), whose shared halos then stay in that XCD's L2.
__device__ __forceinline__ void ssim_tile(int ntv, int n, int* tv, int* tu) {
    const int L = xcd_band_item(blockIdx.x, n);
    *tv = L % ntv;
    *tu = L / ntv;
}

struct SsimWindow {
    float w[2 * kSsimR + 1];
};

// The backward pass reads the derivative maps through a buffer descriptor: one uniform base,
// 32-bit offsets (map q at the scalar offset 4 q P), and a range check that returns 0 for the
// taps outside the image (offset kNoTap, past the buffer: tdgs_loss_grad takes images of fewer
// than 2^31 / 36 pixels) instead of a select per load. Word 3 of the descriptor sets
// DATA_FORMAT = 32 bits (0x00020000, as for raw buffers on the gfx9 family). Only 4-byte loads
// at distinct scalar offsets go through it: a 12-byte buffer load with this descriptor (and
// the compiler merges three adjacent 4-byte ones into one) returned the first word three
// times, so the images keep plain loads.
using Rsrc = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ Rsrc ssim_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
constexpr uint32_t kNoTap = 0x80000000u;

// k_ssim_forward LDS: one buffer, in turn the input (x, y) pairs of the 26 x 26 tile per
// (column, channel), the pass-1 values of the 15 quantities per (quantity, output row), columns
// contiguous, and the pass-2 output (15 values per pixel). Each pass reads its inputs into
// registers and passes a barrier before it overwrites them, so the tile needs 26 KB of LDS
// (6 workgroups per CU) instead of 43 KB for separate buffers (3 per CU); |x - y| of the
// tile's own pixels is summed while the inputs are loaded.
constexpr int kSsimFwdLds = (kSsimIn * 3 * kRow * 2 > kQF * kSsimT * kRow) ? kSsimIn * 3 * kRow * 2 : kQF * kSsimT * kRow;
__global__ __launch_bounds__(256) void k_ssim_forward(const float* __restrict__ x, const float* __restrict__ y,
                                                      int W, int H, SsimWindow win, float* __restrict__ dmap,
                                                      double* __restrict__ partials) {
    __shared__ float4 s_buf4[kSsimFwdLds / 4 + 1];
    __shared__ double s_red[2][256 / kWave];
    float2* const s_in = reinterpret_cast<float2*>(s_buf4);   // (iu, c, iv) at (iu*3 + c)*kRow + iv
    float* const s_v = reinterpret_cast<float*>(s_buf4);      // (q, ov, iu) at (q*16 + ov)*kRow + iu
    float* const s_out = s_v;                          // (ou, ov, q) at (ou*16 + ov)*kOutPitch + q
    static_assert(kSsimT * kSsimT * kOutPitch <= kSsimFwdLds, "pass-2 output fits");
    const int t = threadIdx.x;
    int tv, tu;
    ssim_tile((H + kSsimT - 1) / kSsimT, gridDim.x, &tv, &tu);
    const int v0 = tv * kSsimT - kSsimR, u0 = tu * kSsimT - kSsimR;
    // the tile's inputs: pixel k = t + 256 i (i < 3) of the 26 x 26 tile, all loads issued
    // before the first LDS store (pixel indices are 32-bit: tdgs_loss_grad takes images of fewer
    // than 2^31 / 9 pixels)
    float l1 = 0.0f;   // this thread's |x - y| (at most 9 terms), summed in double over the workgroup
    constexpr int kLoads = (kSsimIn * kSsimIn + 255) / 256;
    float2 xy[kLoads][3];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int k = t + 256 * i;
        const int iv = k % kSsimIn, iu = k / kSsimIn;
        const int v = v0 + iv, u = u0 + iu;
        const bool in = k < kSsimIn * kSsimIn && v >= 0 && v < H && u >= 0 && u < W;
        const uint32_t p = (uint32_t)(v + H * u);
        // one 12-byte load per pixel and image (the three channels are contiguous)
        const float3 xp = in ? reinterpret_cast<const float3*>(x)[p] : make_float3(0.0f, 0.0f, 0.0f);
        const float3 yp = in ? reinterpret_cast<const float3*>(y)[p] : make_float3(0.0f, 0.0f, 0.0f);
        xy[i][0] = make_float2(xp.x, yp.x);
        xy[i][1] = make_float2(xp.y, yp.y);
        xy[i][2] = make_float2(xp.z, yp.z);
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int k = t + 256 * i;
        if (k >= kSsimIn * kSsimIn) break;
        const int iv = k % kSsimIn, iu = k / kSsimIn;
        const bool own = iv >= kSsimR && iv < kSsimR + kSsimT && iu >= kSsimR && iu < kSsimR + kSsimT;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            s_in[(iu * 3 + c) * kRow + iv] = xy[i][c];
            if (own) l1 += fabsf(xy[i][c].x - xy[i][c].y);   // (zero outside the image)
        }
    }
    __syncthreads();
    // pass 1: thread (iu, c, part) filters output rows ov = o0 .. o0 + no - 1 of column iu,
    // channel c, the 16 rows split 6 + 5 + 5 over three parts (234 of the 256 threads)
    const bool p1 = t < kSsimIn * 3 * 3;
    const int p1_iu = t % kSsimIn, p1_c = (t / kSsimIn) % 3, p1_part = t / (3 * kSsimIn);
    const int o0 = p1_part == 0 ? 0 : 1 + 5 * p1_part, no = p1_part == 0 ? 6 : 5;
    float a[16], b[16];
    if (p1) {
        const float2* src = s_in + (p1_iu * 3 + p1_c) * kRow + o0;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float2 ab = k < no + 2 * kSsimR ? src[k] : make_float2(0.0f, 0.0f);
            a[k] = ab.x;
            b[k] = ab.y;
        }
    }
    __syncthreads();   // s_v overwrites s_in
    if (p1) {
        const int iu = p1_iu, c = p1_c;
#pragma unroll
        for (int o = 0; o < 6; ++o) {
            if (o >= no) break;
            // (the first tap as a product: no zeroed accumulators)
            const float w0 = win.w[0], a0 = a[o], b0 = b[o];
            float m0 = w0 * a0, m1 = w0 * b0, m2 = w0 * (a0 * a0), m3 = w0 * (b0 * b0), m4 = w0 * (a0 * b0);
#pragma unroll
            for (int d = 1; d < 2 * kSsimR + 1; ++d) {
                const float wd = win.w[d], av = a[o + d], bv = b[o + d];
                m0 = fmaf(wd, av, m0);
                m1 = fmaf(wd, bv, m1);
                m2 = fmaf(wd, av * av, m2);
                m3 = fmaf(wd, bv * bv, m3);
                m4 = fmaf(wd, av * bv, m4);
            }
            const int ov = o0 + o;
            float* dst = s_v + ((5 * c) * kSsimT + ov) * kRow + iu;
            dst[0] = m0;
            dst[kSsimT * kRow] = m1;
            dst[2 * kSsimT * kRow] = m2;
            dst[3 * kSsimT * kRow] = m3;
            dst[4 * kSsimT * kRow] = m4;
        }
    }
    __syncthreads();
    // pass 2: thread (ov, q) filters row ov of quantity q along u
    float f[kSsimIn];
    const bool p2 = t < kSsimT * kQF;
    const int p2_ov = t % kSsimT, p2_q = t / kSsimT;
    if (p2) {
        const float* src = s_v + (p2_q * kSsimT + p2_ov) * kRow;
#pragma unroll
        for (int k = 0; k < kSsimIn; ++k) f[k] = src[k];
    }
    __syncthreads();   // s_out overwrites s_v
    if (p2) {
#pragma unroll
        for (int ou = 0; ou < kSsimT; ++ou) {
            float m = win.w[0] * f[ou];
#pragma unroll
            for (int d = 1; d < 2 * kSsimR + 1; ++d) m = fmaf(win.w[d], f[ou + d], m);
            s_out[(ou * kSsimT + p2_ov) * kOutPitch + p2_q] = m;
        }
    }
    __syncthreads();
    const int ov = t % kSsimT, ou = t / kSsimT;
    const int v = v0 + kSsimR + ov, u = u0 + kSsimR + ou;
    const bool on = v < H && u < W;
    float m[kQF];
#pragma unroll
    for (int q = 0; q < kQF; ++q) m[q] = s_out[(ou * kSsimT + ov) * kOutPitch + q];
    float ssum = 0.0f;   // this thread's S (3 terms), summed in double over the workgroup
    if (on) {
        const uint32_t p = (uint32_t)(v + H * u);
        const uint32_t P = (uint32_t)W * (uint32_t)H;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float mx = m[5 * c], my = m[5 * c + 1], sxx = m[5 * c + 2], syy = m[5 * c + 3], sxy = m[5 * c + 4];
            const float a1 = 2.0f * mx * my + kC1;
            const float a2 = 2.0f * (sxy - mx * my) + kC2;
            const float b1 = mx * mx + my * my + kC1;
            const float b2 = (sxx - mx * mx) + (syy - my * my) + kC2;
            // two divisions per channel: 1/b1 and 1/b2 (B = b1 b2), the quotients as products
            const float r1 = 1.0f / b1, r2 = 1.0f / b2;
            const float rB = r1 * r2;
            const float S = (a1 * a2) * rB;
            const float dA = 2.0f * my * (a2 - a1);
            const float dB = 2.0f * mx * (b2 - b1);
            // planar maps (plane q of W H values, pixel order of the image): consecutive lanes
            // (consecutive v) write consecutive words
            (dmap + c * P)[p] = (dA - S * dB) * rB;     // dS/dmu_x
            (dmap + (3 + c) * P)[p] = -S * r2;          // dS/dE[x^2]
            (dmap + (6 + c) * P)[p] = 2.0f * a1 * rB;   // dS/dE[xy]
            ssum += S;
        }
    }
    double ssd = ssum, l1d = l1;
    for (int d = 32; d >= 1; d >>= 1) {
        ssd += __shfl_xor(ssd, d, kWave);
        l1d += __shfl_xor(l1d, d, kWave);
    }
    if (__lane_id() == 0) {
        s_red[0][t / kWave] = ssd;
        s_red[1][t / kWave] = l1d;
    }
    __syncthreads();
    if (t == 0) {
        double a = 0.0, b = 0.0;
        for (int k = 0; k < 256 / kWave; ++k) { a += s_red[0][k]; b += s_red[1][k]; }
        const int64_t blk = blockIdx.x;
        partials[2 * blk] = b;      // sum |x - y|
        partials[2 * blk + 1] = a;  // sum of the SSIM map
    }
}

// Workgroup of 256 threads: sums[k] += sum over the nblk partial pairs (run by workgroup 0 of
// k_ssim_backward, after k_ssim_forward wrote the partials: no launch of its own).
__device__ void ssim_add_partials(const double* __restrict__ partials, int64_t nblk, double* __restrict__ sums) {
    __shared__ double s_red[2][256 / kWave];
    double a = 0.0, b = 0.0;
    for (int64_t i = threadIdx.x; i < nblk; i += 256) {
        a += partials[2 * i];
        b += partials[2 * i + 1];
    }
    for (int d = 32; d >= 1; d >>= 1) {
        a += __shfl_xor(a, d, kWave);
        b += __shfl_xor(b, d, kWave);
    }
    if (__lane_id() == 0) {
        s_red[0][threadIdx.x / kWave] = a;
        s_red[1][threadIdx.x / kWave] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double ta = 0.0, tb = 0.0;
        for (int k = 0; k < 256 / kWave; ++k) { ta += s_red[0][k]; tb += s_red[1][k]; }
        sums[0] += ta;
        sums[1] += tb;
    }
}

__global__ __launch_bounds__(256) void k_ssim_backward(const float* __restrict__ x, const float* __restrict__ y,
                                                       int W, int H, SsimWindow win,
                                                       const float* __restrict__ dmap, float w_l1, float w_ssim,
                                                       float* __restrict__ grad, const double* __restrict__ partials,
                                                       int64_t nblk, double* __restrict__ sums) {
    // one buffer, in turn the input columns, the pass-1 values and the pass-2 output (as in
    // k_ssim_forward: every pass reads its inputs into registers before a barrier)
    __shared__ float s_in[kSsimIn * kQB * kRow];       // (iu, q, iv) at (iu*9 + q)*kRow + iv
    float* const s_v = s_in;                           // (q, ov, iu) at (q*16 + ov)*kRow + iu
    float* const s_out = s_in;                         // (ou, ov, q) at (ou*16 + ov)*kOutPitch + q
    static_assert(kSsimT * kSsimT * kOutPitch <= kSsimIn * kQB * kRow, "pass-2 output fits");
    static_assert(kQB * kSsimT * kRow <= kSsimIn * kQB * kRow, "pass-1 output fits");
    const int t = threadIdx.x;
    int tv, tu;
    ssim_tile((H + kSsimT - 1) / kSsimT, gridDim.x, &tv, &tu);
    const int v0 = tv * kSsimT - kSsimR, u0 = tu * kSsimT - kSsimR;
    if (blockIdx.x == 0) ssim_add_partials(partials, nblk, sums);
    // this thread's output pixel and its inputs (read now, used at the end)
    const int ov = t % kSsimT, ou = t / kSsimT;
    const int v = v0 + kSsimR + ov, u = u0 + kSsimR + ou;
    const bool on = v < H && u < W;
    const uint32_t p = (uint32_t)(v + H * u);   // (32-bit, as in k_ssim_forward)
    const uint32_t P = (uint32_t)W * (uint32_t)H;
    float xv[3], yv[3];
    {
        const float3 xp = on ? reinterpret_cast<const float3*>(x)[p] : make_float3(0.0f, 0.0f, 0.0f);
        const float3 yp = on ? reinterpret_cast<const float3*>(y)[p] : make_float3(0.0f, 0.0f, 0.0f);
        xv[0] = xp.x; xv[1] = xp.y; xv[2] = xp.z;
        yv[0] = yp.x; yv[1] = yp.y; yv[2] = yp.z;
    }
    // the tile's nine maps: pixel k = t + 256 i (i < 3) of the 26 x 26 tile, all loads issued
    // before the first LDS store
    constexpr int kLoads = (kSsimIn * kSsimIn + 255) / 256;
    const Rsrc rm = ssim_rsrc(dmap, 4u * kQB * P);
    float dv[kLoads][kQB];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int k = t + 256 * i;
        const int iv = k % kSsimIn, iu = k / kSsimIn;
        const int v = v0 + iv, u = u0 + iu;
        const bool in = k < kSsimIn * kSsimIn && v >= 0 && v < H && u >= 0 && u < W;
        const uint32_t off = in ? 4u * (uint32_t)(v + H * u) : kNoTap;
        // (off + 4 q P stays past the buffer for kNoTap)
#pragma unroll
        for (int q = 0; q < kQB; ++q)
            dv[i][q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, off, 4u * q * P, 0));
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int k = t + 256 * i;
        if (k >= kSsimIn * kSsimIn) break;
        const int iv = k % kSsimIn, iu = k / kSsimIn;
#pragma unroll
        for (int q = 0; q < kQB; ++q) s_in[(iu * kQB + q) * kRow + iv] = dv[i][q];
    }
    __syncthreads();
    // pass 1: thread (iu, q) filters the whole column iu of quantity q along v
    const bool p1 = t < kSsimIn * kQB;
    float a[kSsimIn];
    if (p1) {
        const float* src = s_in + t * kRow;   // t = iu * 9 + q
#pragma unroll
        for (int k = 0; k < kSsimIn; ++k) a[k] = src[k];
    }
    __syncthreads();   // s_v overwrites s_in
    if (p1) {
        const int iu = t / kQB, q = t % kQB;
#pragma unroll
        for (int ov = 0; ov < kSsimT; ++ov) {
            float m = win.w[0] * a[ov];
#pragma unroll
            for (int d = 1; d < 2 * kSsimR + 1; ++d) m = fmaf(win.w[d], a[ov + d], m);
            s_v[(q * kSsimT + ov) * kRow + iu] = m;
        }
    }
    __syncthreads();
    // pass 2: thread (ov, q) filters row ov of quantity q along u
    const bool p2 = t < kSsimT * kQB;
    float b[kSsimIn];
    if (p2) {
        const int ov = t % kSsimT, q = t / kSsimT;
        const float* src = s_v + (q * kSsimT + ov) * kRow;
#pragma unroll
        for (int k = 0; k < kSsimIn; ++k) b[k] = src[k];
    }
    __syncthreads();   // s_out overwrites s_v
    if (p2) {
        const int ov = t % kSsimT, q = t / kSsimT;
#pragma unroll
        for (int ou = 0; ou < kSsimT; ++ou) {
            float m = win.w[0] * b[ou];
#pragma unroll
            for (int d = 1; d < 2 * kSsimR + 1; ++d) m = fmaf(win.w[d], b[ou + d], m);
            s_out[(ou * kSsimT + ov) * kOutPitch + q] = m;
        }
    }
    __syncthreads();
    if (!on) return;
    float f[kQB];
#pragma unroll
    for (int q = 0; q < kQB; ++q) f[q] = s_out[(ou * kSsimT + ov) * kOutPitch + q];
    float gr[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float dssim = -(f[c] + 2.0f * xv[c] * f[3 + c] + yv[c] * f[6 + c]);
        const float s = xv[c] > yv[c] ? w_l1 : -w_l1;   // ties take -w_l1 (training.jl:214-215)
        gr[c] = s + w_ssim * dssim;   // product rounded, then the sum, as the reference's broadcast
    }
    reinterpret_cast<float3*>(grad)[p] = make_float3(gr[0], gr[1], gr[2]);
}

static SsimWindow gaussian_window() {
    SsimWindow w;
    double g[2 * kSsimR + 1], s = 0.0;
    for (int k = 0; k <= 2 * kSsimR; ++k) {
        const double d = k - kSsimR;
        g[k] = exp(-d * d / (2.0 * 1.5 * 1.5));
        s += g[k];
    }
    for (int k = 0; k <= 2 * kSsimR; ++k) w.w[k] = (float)(g[k] / s);
    return w;
}

}  // namespace tdgs

using namespace tdgs;

extern "C" {

// Scratch: the 9 SSIM partial-derivative maps (planar: map q of W H values, in the image's
// pixel order), then one (|x - y|, S) sum pair per workgroup.
static size_t loss_dmap_bytes(int32_t width, int32_t height) {
    return align_up((size_t)9 * sizeof(float) * (size_t)(width > 0 ? width : 1) * (size_t)(height > 0 ? height : 1));
}
static int64_t loss_blocks(int32_t width, int32_t height) {
    return ceil_div(height > 0 ? height : 1, kSsimT) * ceil_div(width > 0 ? width : 1, kSsimT);
}

size_t tdgs_loss_temp_bytes(int32_t width, int32_t height) {
    return loss_dmap_bytes(width, height) + align_up((size_t)loss_blocks(width, height) * 2 * sizeof(double));
}

int tdgs_loss_grad(void* stream, const float* rendered, const float* gt, int32_t width, int32_t height,
                   float dssim_weight, float* grad_out, double* sums_dev, void* temp, size_t temp_bytes) {
    TDGS_REQUIRE(width > 0 && height > 0, "bad image size");
    TDGS_REQUIRE((int64_t)width * height * 36 < ((int64_t)1 << 31), "image too large for the loss kernels (32-bit offsets)");
    TDGS_REQUIRE(rendered && gt && grad_out && sums_dev && temp, "null arrays");
    TDGS_REQUIRE(temp_bytes >= tdgs_loss_temp_bytes(width, height), "loss scratch too small");
    hipStream_t s = (hipStream_t)stream;
    StageScope sc(TDGS_STAGE_LOSS, s);
    const SsimWindow win = gaussian_window();
    const int64_t count = 3 * (int64_t)width * height;
    const unsigned grid = (unsigned)loss_blocks(width, height);
    double* partials = (double*)((char*)temp + loss_dmap_bytes(width, height));
    k_ssim_forward<<<grid, 256, 0, s>>>(rendered, gt, width, height, win, (float*)temp, partials);
    TDGS_LAUNCHED();
    const float w_l1 = (1.0f - dssim_weight) / (float)count;
    const float w_ssim = dssim_weight / (float)count;
    k_ssim_backward<<<grid, 256, 0, s>>>(rendered, gt, width, height, win, (const float*)temp, w_l1, w_ssim,
                                         grad_out, partials, loss_blocks(width, height), sums_dev);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

}  // extern "C"
