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
//                    and |x - y| per workgroup (one partial pair per workgroup; a one-block
//                    launch adds the partials to the caller's sums, so no workgroup waits on
//                    an atomic to a shared address)
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

// LDS layouts: a pixel's values are an odd number of words apart and a tile column starts at
// a word offset = 16 (mod 32). A half-wavefront reads 16 consecutive rows of two adjacent
// columns, so its 32 words fall on 32 distinct banks.
constexpr int kInF = 7;                // forward input: x, y (3 channels each) + 1 pad
constexpr int kPitchF = 208;           // >= kSsimIn * kInF, = 16 (mod 32)
constexpr int kInB = 9;                // backward input: D1, D2, D3 (3 channels each)
constexpr int kPitchB = 240;           // >= kSsimIn * kInB, = 16 (mod 32)
static_assert(kPitchF >= kSsimIn * kInF && kPitchF % 32 == 16, "forward pitch");
static_assert(kPitchB >= kSsimIn * kInB && kPitchB % 32 == 16, "backward pitch");
static_assert((kSsimT * 15) % 32 == 16 && (kSsimT * 9) % 32 == 16, "filtered column pitch");

// XCD-aware tile order: workgroups are handed to the 8 XCDs round-robin by linear id, so the
// workgroups with id = x (mod 8) all run on XCD x. They get one contiguous band of tiles (v
// fastest), whose shared halos then stay in that XCD's L2. A bijection on the first
// 8 * floor(n / 8) ids; the remainder keeps its own index.
constexpr int kXcds = 8;
__device__ __forceinline__ void ssim_tile(int ntv, int n, int* tv, int* tu) {
    const int b = blockIdx.x;
    const int per = n / kXcds;
    const int L = b < per * kXcds ? (b % kXcds) * per + b / kXcds : b;
    *tv = L % ntv;
    *tu = L / ntv;
}

struct SsimWindow {
    float w[2 * kSsimR + 1];
};

// k_ssim_forward LDS layout: input x/y (3 channels each) for the 26 x 26 input tile, then the
// v-filtered values of 5 quantities x 3 channels for 26 columns x 16 rows.
__global__ __launch_bounds__(256) void k_ssim_forward(const float* __restrict__ x, const float* __restrict__ y,
                                                      int W, int H, SsimWindow win, float* __restrict__ dmap,
                                                      double* __restrict__ partials) {
    __shared__ float s_in[kSsimIn * kPitchF];      // (column iu, row iv, value) at iu*kPitchF + iv*kInF
    __shared__ float s_v[kSsimIn][kSsimT][15];
    __shared__ double s_red[2][256 / kWave];
    const int t = threadIdx.x;
    int tv, tu;
    ssim_tile((H + kSsimT - 1) / kSsimT, gridDim.x, &tv, &tu);
    const int v0 = tv * kSsimT - kSsimR, u0 = tu * kSsimT - kSsimR;
    for (int k = t; k < kSsimIn * kSsimIn; k += 256) {
        const int iv = k % kSsimIn, iu = k / kSsimIn;
        const int v = v0 + iv, u = u0 + iu;
        const bool in = v >= 0 && v < H && u >= 0 && u < W;
        const int64_t p = 3 * ((int64_t)v + (int64_t)H * u);
        float* d = s_in + iu * kPitchF + iv * kInF;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            d[c] = in ? x[p + c] : 0.0f;
            d[3 + c] = in ? y[p + c] : 0.0f;
        }
    }
    __syncthreads();
    // filter along v (the contiguous image axis)
    for (int k = t; k < kSsimIn * kSsimT; k += 256) {
        const int ov = k % kSsimT, iu = k / kSsimT;
        float acc[15];
#pragma unroll
        for (int q = 0; q < 15; ++q) acc[q] = 0.0f;
#pragma unroll
        for (int d = 0; d < 2 * kSsimR + 1; ++d) {
            const float* s = s_in + iu * kPitchF + (ov + d) * kInF;
            const float wd = win.w[d];
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const float a = s[c], b = s[3 + c];
                acc[5 * c] = fmaf(wd, a, acc[5 * c]);
                acc[5 * c + 1] = fmaf(wd, b, acc[5 * c + 1]);
                acc[5 * c + 2] = fmaf(wd, a * a, acc[5 * c + 2]);
                acc[5 * c + 3] = fmaf(wd, b * b, acc[5 * c + 3]);
                acc[5 * c + 4] = fmaf(wd, a * b, acc[5 * c + 4]);
            }
        }
#pragma unroll
        for (int q = 0; q < 15; ++q) s_v[iu][ov][q] = acc[q];
    }
    __syncthreads();
    const int ov = t % kSsimT, ou = t / kSsimT;
    const int v = v0 + kSsimR + ov, u = u0 + kSsimR + ou;
    const bool on = v < H && u < W;
    float m[15];
#pragma unroll
    for (int q = 0; q < 15; ++q) m[q] = 0.0f;
#pragma unroll
    for (int d = 0; d < 2 * kSsimR + 1; ++d) {
        const float wd = win.w[d];
#pragma unroll
        for (int q = 0; q < 15; ++q) m[q] = fmaf(wd, s_v[ou + d][ov][q], m[q]);
    }
    double ssum = 0.0, l1 = 0.0;
    if (on) {
        const int64_t p = 3 * ((int64_t)v + (int64_t)H * u);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float mx = m[5 * c], my = m[5 * c + 1], sxx = m[5 * c + 2], syy = m[5 * c + 3], sxy = m[5 * c + 4];
            const float a1 = 2.0f * mx * my + kC1;
            const float a2 = 2.0f * (sxy - mx * my) + kC2;
            const float b1 = mx * mx + my * my + kC1;
            const float b2 = (sxx - mx * mx) + (syy - my * my) + kC2;
            const float B = b1 * b2;
            const float S = (a1 * a2) / B;
            const float dA = 2.0f * my * (a2 - a1);
            const float dB = 2.0f * mx * (b2 - b1);
            dmap[3 * p + c] = (dA - S * dB) / B;      // dS/dmu_x
            dmap[3 * p + 3 + c] = -S / b2;            // dS/dE[x^2]
            dmap[3 * p + 6 + c] = 2.0f * a1 / B;      // dS/dE[xy]
            ssum += (double)S;
            const float* px = s_in + (ou + kSsimR) * kPitchF + (ov + kSsimR) * kInF;
            l1 += fabs((double)px[c] - (double)px[3 + c]);
        }
    }
    for (int d = 32; d >= 1; d >>= 1) {
        ssum += __shfl_xor(ssum, d, kWave);
        l1 += __shfl_xor(l1, d, kWave);
    }
    if (__lane_id() == 0) {
        s_red[0][t / kWave] = ssum;
        s_red[1][t / kWave] = l1;
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

// One workgroup: sums[k] += sum over the nblk partial pairs.
__global__ __launch_bounds__(1024) void k_ssim_sums(const double* __restrict__ partials, int64_t nblk,
                                                    double* __restrict__ sums) {
    __shared__ double s_red[2][1024 / kWave];
    double a = 0.0, b = 0.0;
    for (int64_t i = threadIdx.x; i < nblk; i += 1024) {
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
        for (int k = 0; k < 1024 / kWave; ++k) { ta += s_red[0][k]; tb += s_red[1][k]; }
        sums[0] += ta;
        sums[1] += tb;
    }
}

__global__ __launch_bounds__(256) void k_ssim_backward(const float* __restrict__ x, const float* __restrict__ y,
                                                       int W, int H, SsimWindow win,
                                                       const float* __restrict__ dmap, float w_l1, float w_ssim,
                                                       float* __restrict__ grad) {
    __shared__ float s_in[kSsimIn * kPitchB];      // (column iu, row iv, value) at iu*kPitchB + iv*kInB
    __shared__ float s_v[kSsimIn][kSsimT][9];
    const int t = threadIdx.x;
    int tv, tu;
    ssim_tile((H + kSsimT - 1) / kSsimT, gridDim.x, &tv, &tu);
    const int v0 = tv * kSsimT - kSsimR, u0 = tu * kSsimT - kSsimR;
    for (int k = t; k < kSsimIn * kSsimIn; k += 256) {
        const int iv = k % kSsimIn, iu = k / kSsimIn;
        const int v = v0 + iv, u = u0 + iu;
        const bool in = v >= 0 && v < H && u >= 0 && u < W;
        const int64_t p = 9 * ((int64_t)v + (int64_t)H * u);
        float* d = s_in + iu * kPitchB + iv * kInB;
#pragma unroll
        for (int q = 0; q < 9; ++q) d[q] = in ? dmap[p + q] : 0.0f;
    }
    __syncthreads();
    for (int k = t; k < kSsimIn * kSsimT; k += 256) {
        const int ov = k % kSsimT, iu = k / kSsimT;
        float acc[9];
#pragma unroll
        for (int q = 0; q < 9; ++q) acc[q] = 0.0f;
#pragma unroll
        for (int d = 0; d < 2 * kSsimR + 1; ++d) {
            const float* s = s_in + iu * kPitchB + (ov + d) * kInB;
            const float wd = win.w[d];
#pragma unroll
            for (int q = 0; q < 9; ++q) acc[q] = fmaf(wd, s[q], acc[q]);
        }
#pragma unroll
        for (int q = 0; q < 9; ++q) s_v[iu][ov][q] = acc[q];
    }
    __syncthreads();
    const int ov = t % kSsimT, ou = t / kSsimT;
    const int v = v0 + kSsimR + ov, u = u0 + kSsimR + ou;
    if (v >= H || u >= W) return;
    float f[9];
#pragma unroll
    for (int q = 0; q < 9; ++q) f[q] = 0.0f;
#pragma unroll
    for (int d = 0; d < 2 * kSsimR + 1; ++d) {
        const float wd = win.w[d];
#pragma unroll
        for (int q = 0; q < 9; ++q) f[q] = fmaf(wd, s_v[ou + d][ov][q], f[q]);
    }
    const int64_t p = 3 * ((int64_t)v + (int64_t)H * u);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float xv = x[p + c], yv = y[p + c];
        const float dssim = -(f[c] + 2.0f * xv * f[3 + c] + yv * f[6 + c]);
        const float s = xv > yv ? w_l1 : -w_l1;
        grad[p + c] = fmaf(w_ssim, dssim, s);
    }
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

// Scratch: the 9 SSIM partial-derivative maps, then one (|x - y|, S) sum pair per workgroup.
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
    k_ssim_sums<<<1, 1024, 0, s>>>(partials, loss_blocks(width, height), sums_dev);
    TDGS_LAUNCHED();
    const float w_l1 = (1.0f - dssim_weight) / (float)count;
    const float w_ssim = dssim_weight / (float)count;
    k_ssim_backward<<<grid, 256, 0, s>>>(rendered, gt, width, height, win, (const float*)temp, w_l1, w_ssim,
                                         grad_out);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

}  // extern "C"
