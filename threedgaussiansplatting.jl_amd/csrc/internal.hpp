// internal.hpp — pieces shared between the translation units of libtdgs.
#pragma once

#include <cmath>

#include "common.hpp"

struct tdgs_ctx {
    int device;
    int64_t* d_counters;   // device scratch for counts reported to the host
    int64_t* h_counters;   // pinned host mirror of d_counters
};

namespace tdgs {

constexpr int kCounters = 8;

// Copy the first count device counters to the host and wait for the stream.
int read_counters(tdgs_ctx* ctx, hipStream_t stream, int count);

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
    const int nt = t->tile_width * t->tile_height;
    TDGS_REQUIRE(nt <= 1024 && nt % 64 == 0, "tile of %d pixels: need a multiple of 64 up to 1024", nt);
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
