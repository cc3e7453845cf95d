// internal.hpp — pieces shared between the translation units of libtdgs.
#pragma once

#include <cmath>

#include "common.hpp"

struct tdgs_ctx {
    int device;
    int64_t* d_counters;   // device scratch for counts reported to the host (+ the monitor state)
    int64_t* h_counters;   // pinned host mirror of d_counters
    int64_t* h_monitor;    // pinned, coherent host memory the device writes the frame monitor to
    int64_t* h_monitor_dev;   // its device address
};

namespace tdgs {

constexpr int kCounters = 12;
// Frame monitor of device-count renders: [frames, largest M, frames whose keys did not fit,
// last M, the device error flags pending when the last frame blended], kept on the device
// after the counters (d_counters + kCounters) and copied to the host (h_monitor) by every
// such frame.
constexpr int kMonitor = 5;
// Slot of ctx->d_counters holding the sticky device error flags (low 32 bits): kernels OR
// kErr* bits into it; every host synchronisation through read_counters reports and clears it.
constexpr int kErrSlot = 7;
constexpr uint32_t kErrSortCounts = 1u;   // radix-sort counts disagreed with the keys

inline uint32_t* ctx_error_word(tdgs_ctx* ctx) { return reinterpret_cast<uint32_t*>(ctx->d_counters + kErrSlot); }

// Other slots of ctx->d_counters: 0 filtered count N_f, 1 key count M, 2 ADC count, 4 count of
// non-empty Gaussians, 8 entries of the coarse blocks' lists (with M: see kLow32); in a render with
// TDGS_FLAG_DEVICE_COUNTS, 5 the key count the frame uses (M, or 0 when M does not fit the key
// arrays), 6 the frame status and 9 the coarse entries used (0 with 5).
constexpr int kCntKeysUsed = 5, kCntStatus = 6, kCntCoarse = 8, kCntCoarseUsed = 9;
// Slot kCntCoarse holds (M << 32) | coarse entries (one scan of packed counts).
constexpr int64_t kLow32 = 0xffffffffll;
// Frame status: the keys fit, M > key_capacity, M >= 2^31.
constexpr int64_t kFrameOk = 0, kFrameKeyCapacity = 1, kFrameKeyRange = 2;
// A device-count render leaves [N_f, M, non-empty count, status] in the first four int64 of
// the render buffers' temp, for the entry points that read the counts on the device.
inline int64_t* frame_counts(const tdgs_render_buffers* buf) { return reinterpret_cast<int64_t*>(buf->temp); }

// Copy the device counters to the host and wait for the stream; returns TDGS_ERR_DEVICE (and
// clears the flags) when a kernel has raised an error flag since the last check.
int read_counters(tdgs_ctx* ctx, hipStream_t stream);

// Stage profiler: records a start/stop HIP event pair around a stage when enabled.
void profile_mark(int stage, bool start, hipStream_t stream);

struct StageScope {
    int stage;
    hipStream_t stream;
    StageScope(int st, hipStream_t s) : stage(st), stream(s) { profile_mark(stage, true, stream); }
    ~StageScope() { profile_mark(stage, false, stream); }
};

// Exponent below which blending can skip an entry: for e < exponent_cut(min_alpha),
// exp_f(e) (relative error a few 1e-7) is below min_alpha, so alpha < min_alpha. A margin of
// 1e-3 in the exponent covers the rounding; no cut without a positive min_alpha.
inline float exponent_cut(float min_alpha) {
    if (!(min_alpha > 0.0f)) return -__builtin_inff();
    return std::nextafter((float)(std::log((double)min_alpha) - 1e-3), -__builtin_inff());
}

// Pixel of thread t inside a TW x TH tile (1-based). With both sides multiples of 8 each
// wavefront covers an 8x8 block (blocks column-major, lanes column-major inside), which
// keeps a Gaussian's footprint inside as few wavefronts as possible; otherwise wavefront
// t/64 covers 64 consecutive pixels of the column-major tile.
__device__ __forceinline__ void tile_pixel(int t, int TW, int TH, int* u_in, int* v_in) {
    if ((TW & 7) == 0 && (TH & 7) == 0) {
        const int w = t >> 6, l = t & 63, bpc = TH >> 3;
        *v_in = (w % bpc) * 8 + (l & 7) + 1;
        *u_in = (w / bpc) * 8 + (l >> 3) + 1;
    } else {
        *v_in = t % TH + 1;
        *u_in = t / TH + 1;
    }
}

// The 2D gradients of a tdgs_gradients in either layout: component k (0-8: dmu_x, dmu_y, da,
// dM11, dM21, dM22, dr, dg, db) of filtered Gaussian f (0-based) is base[k][stride[k] * f].
struct Grads2D {
    float* base[9];
    int32_t stride[9];
    __device__ __forceinline__ float* at(int k, int64_t f) const { return base[k] + (int64_t)stride[k] * f; }
    // the same for a k that differs between lanes (selects instead of an indexed argument)
    __device__ __forceinline__ float* at_dynamic(int k, int64_t f) const {
        float* b = base[0];
        int32_t st = stride[0];
#pragma unroll
        for (int i = 1; i < 9; ++i) {
            if (k == i) {
                b = base[i];
                st = stride[i];
            }
        }
        return b + (int64_t)st * f;
    }
};

// Host: the view of grads' 2D gradients; TDGS_ERR_INVALID when the arrays of neither layout are
// given.
inline int grads2d_view(const tdgs_gradients* g, Grads2D* v) {
    TDGS_REQUIRE(g != nullptr, "null gradients");
    if (g->grads2d) {
        for (int k = 0; k < 9; ++k) {
            v->base[k] = g->grads2d + k;
            v->stride[k] = 9;
        }
        return TDGS_OK;
    }
    TDGS_REQUIRE(g->mean2d_grads && g->opacity_grads && g->licov2d_grads && g->color_grads,
                 "2D gradients: neither grads2d nor all of mean2d_grads, opacity_grads, licov2d_grads and "
                 "color_grads given");
    float* const arr[4] = {g->mean2d_grads, g->opacity_grads, g->licov2d_grads, g->color_grads};
    const int comps[4] = {2, 1, 3, 3};
    int k = 0;
    for (int a = 0; a < 4; ++a)
        for (int c = 0; c < comps[a]; ++c, ++k) {
            v->base[k] = arr[a] + c;
            v->stride[k] = comps[a];
        }
    return TDGS_OK;
}

inline int check_gaussians(const tdgs_gaussians* g, bool trainable_only) {
    TDGS_REQUIRE(g != nullptr, "gaussians is null");
    TDGS_REQUIRE(g->n >= 0, "negative Gaussian count %d", g->n);
    TDGS_REQUIRE(g->sh_degree >= 0 && g->sh_degree <= 3, "unsupported SH degree %d", g->sh_degree);
    TDGS_REQUIRE(g->kind == TDGS_TRAINABLE || g->kind == TDGS_RENDER_ONLY, "unknown Gaussian kind %d", g->kind);
    if (trainable_only) TDGS_REQUIRE(g->kind == TDGS_TRAINABLE, "operation needs trainable Gaussians");
    if (g->n > 0) {
        TDGS_REQUIRE(g->means_opacity && g->sh, "null Gaussian arrays");
        if (g->kind == TDGS_TRAINABLE) TDGS_REQUIRE(g->scaling && g->rotation, "null scaling/rotation");
        else TDGS_REQUIRE(g->covariances, "null covariances");
    }
    return TDGS_OK;
}

inline int check_tiling(const tdgs_tiling* t, const tdgs_camera* cam) {
    TDGS_REQUIRE(t && cam, "null tiling or camera");
    TDGS_REQUIRE(t->tile_width > 0 && t->tile_height > 0, "bad tile size");
    // any tile shape the reference's Tiling accepts (forward_structs.jl:340-424) whose pixels fit
    // one workgroup: the kernels run one thread per pixel (one per four in the backward pass)
    const int64_t nt = (int64_t)t->tile_width * t->tile_height;
    TDGS_REQUIRE(nt <= 1024, "tile of %lld pixels: at most 1024 are supported", (long long)nt);
    TDGS_REQUIRE(cam->width > 0 && cam->height > 0, "bad image size");
    TDGS_REQUIRE(t->nb_tiles_x == (cam->width + t->tile_width - 1) / t->tile_width &&
                     t->nb_tiles_y == (cam->height + t->tile_height - 1) / t->tile_height,
                 "tiling does not match the image size");
    return TDGS_OK;
}

// The blending kernels compare against these thresholds with selects that equal fminf only
// for non-NaN operands.
inline int check_thresholds(const tdgs_render_options* o) {
    TDGS_REQUIRE(o != nullptr, "null options");
    TDGS_REQUIRE(o->min_alpha == o->min_alpha && o->max_alpha == o->max_alpha &&
                     o->min_transmittance == o->min_transmittance,
                 "NaN alpha or transmittance threshold");
    return TDGS_OK;
}

inline int check_options(const tdgs_render_options* o, int data_degree) {
    TDGS_REQUIRE(o != nullptr, "null options");
    TDGS_REQUIRE(o->sh_degree >= 0 && o->sh_degree <= data_degree,
                 "render SH degree %d exceeds the data's %d", o->sh_degree, data_degree);
    TDGS_REQUIRE(o->clip_mode == TDGS_CLIP_CLAMP || o->clip_mode == TDGS_CLIP_FILTER, "bad clip mode");
    return check_thresholds(o);
    return TDGS_OK;
}

}  // namespace tdgs
