// image.hip — rendered images to the viewer's UInt8 RGB layout (the GUI's convert_*_to_gl_img
// kernels, src/gui.jl:958-1067).
//
// The render outputs are column-major 3 x h x w (rgb) and h x w (T, depth): consecutive
// addresses run down a pixel column. The viewer wants 3 x w x h bytes: consecutive addresses
// run along a pixel row. The kernel therefore transposes through LDS: a workgroup converts a
// 32 x 32 pixel block reading along columns and writes it out along rows, so both the float
// reads and the byte writes are contiguous (the reference's kernel leaves this as a TODO and
// reads with a stride of h).
#include "internal.hpp"

namespace tdgs {

constexpr int kImgBlock = 32;

__device__ __forceinline__ uint8_t to_u8(float x) {   // round(UInt8, x) for x in [0, 255]
    return (uint8_t)(int)rintf(x);
}

__global__ __launch_bounds__(256) void k_image_to_rgb8(int kind, const float* __restrict__ src, int32_t W,
                                                       int32_t H, float dmin, float dmax,
                                                       uint8_t* __restrict__ dst) {
    __shared__ uint8_t s[kImgBlock][3 * kImgBlock + 4];   // [row in block][3 * column + channel]
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8 threads
    const int u0 = blockIdx.x * kImgBlock, v0 = blockIdx.y * kImgBlock;
    // read: lanes along a column (v), rows of the block in turn
    for (int r = ty; r < kImgBlock; r += 8) {
        const int u = u0 + r, v = v0 + tx;
        if (u < W && v < H) {
            const int64_t px = (int64_t)v + (int64_t)H * u;
            uint8_t c0, c1, c2;
            if (kind == TDGS_IMAGE_RGB) {
                const float* p = src + 3 * px;
                const float f0 = p[0], f1 = p[1], f2 = p[2];
                c0 = f0 <= 1.0f ? to_u8(f0 * 255.0f) : (uint8_t)255;
                c1 = f1 <= 1.0f ? to_u8(f1 * 255.0f) : (uint8_t)255;
                c2 = f2 <= 1.0f ? to_u8(f2 * 255.0f) : (uint8_t)255;
            } else if (kind == TDGS_IMAGE_TRANSMITTANCE) {
                c0 = c1 = c2 = to_u8(src[px] * 255.0f);
            } else {
                float q = (src[px] - dmin) / (dmax - dmin);
                q = q < 0.0f ? 0.0f : (q > 1.0f ? 1.0f : q);
                c0 = c1 = c2 = to_u8((1.0f - q) * 255.0f);
            }
            s[tx][3 * r] = c0;
            s[tx][3 * r + 1] = c1;
            s[tx][3 * r + 2] = c2;
        }
    }
    __syncthreads();
    // write: lanes along a row (u), the 96 bytes of each block row
    for (int r = ty; r < kImgBlock; r += 8) {
        const int v = v0 + r;
        if (v >= H) continue;
        const int nu = W - u0 < kImgBlock ? W - u0 : kImgBlock;
        uint8_t* row = dst + 3 * ((int64_t)u0 + (int64_t)W * v);
        for (int b = tx; b < 3 * nu; b += 32) row[b] = s[r][b];
    }
}

}  // namespace tdgs

using namespace tdgs;

extern "C" {

int tdgs_image_to_rgb8(void* stream, int32_t kind, const float* src, int32_t width, int32_t height,
                       float min_depth, float max_depth, uint8_t* dst) {
    TDGS_REQUIRE(kind == TDGS_IMAGE_RGB || kind == TDGS_IMAGE_TRANSMITTANCE || kind == TDGS_IMAGE_DEPTH,
                 "unknown image kind %d", kind);
    TDGS_REQUIRE(width >= 0 && height >= 0, "negative image size %d x %d", width, height);
    if (width == 0 || height == 0) return TDGS_OK;
    TDGS_REQUIRE(src && dst, "null image");
    TDGS_REQUIRE(kind != TDGS_IMAGE_DEPTH || min_depth < max_depth,
                 "depth range needs min_depth < max_depth (got %g, %g)", (double)min_depth, (double)max_depth);
    const dim3 grid((unsigned)ceil_div(width, kImgBlock), (unsigned)ceil_div(height, kImgBlock));
    k_image_to_rgb8<<<grid, 256, 0, (hipStream_t)stream>>>(kind, src, width, height, min_depth, max_depth, dst);
    TDGS_LAUNCHED();
    return TDGS_OK;
}

}  // extern "C"
