// tdgs_oracle.cpp — CPU restatement of the reference render/train core.
//
// TEST INFRASTRUCTURE ONLY. This file is the checker the GPU path is compared against;
// only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it. Nothing
// in the product library links or calls it.
//
// It restates the reference algorithms sequentially, in the reference's order (one
// filtered Gaussian, key, pixel at a time), with the per-element mathematics shared with
// the kernels (threedgaussiansplatting.jl_amd/csrc/tdgs_math.hpp). The comments give the
// reference file:line each function follows. Pinning of each function against the
// reference's own golden vectors, closed forms, brute force and an independent float64
// restatement differentiated by torch autograd is in tests/ (see the module docstrings
// there: test_oracle_goldens, test_oracle_pins, test_oracle_closed_forms,
// test_oracle_float64, test_oracle_training). Parity unpinned: the individual split draws of
// oracle_adc_apply (the reference samples them with device randn; their distribution
// R (z * s), z ~ N(0, I), is pinned by a sample-covariance closed form).
//
// Built by oracle/build.py into oracle/liboracle.so (g++ -O2 -ffp-contract=off).

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <numeric>
#include <thread>
#include <vector>

#include "../threedgaussiansplatting.jl_amd/csrc/tdgs_math.hpp"

using namespace tdgs;

namespace {

inline int h_of(int degree) { return (degree + 1) * (degree + 1); }

// Gather the per-Gaussian projection parameters (log-scales + quaternion, or covariance).
inline void gaussian_params(const tdgs_gaussians& g, int64_t gi, float params[7]) {
    if (g.kind == TDGS_TRAINABLE) {
        for (int k = 0; k < 3; ++k) params[k] = g.scaling[3 * gi + k];
        for (int k = 0; k < 4; ++k) params[3 + k] = g.rotation[4 * gi + k];
    } else {
        for (int k = 0; k < 6; ++k) params[k] = g.covariances[6 * gi + k];
    }
}

// Threads for the per-tile loops (oracle_set_threads). Tiles are independent in the forward
// pass, so any thread count gives the same images bit for bit; the backward pass sums each
// thread's contributions in double precision and adds the per-thread sums in thread order.
int g_threads = 1;

// Runs body(ty) for every tile row ty in [1, nty], tile rows dealt round-robin to threads.
template <class F>
void for_tile_rows(int nty, F body) {
    const int nt = std::max(1, std::min(g_threads, nty));
    if (nt == 1) {
        for (int ty = 1; ty <= nty; ++ty) body(ty, 0);
        return;
    }
    std::vector<std::thread> pool;
    for (int k = 0; k < nt; ++k)
        pool.emplace_back([&, k]() {
            for (int ty = 1 + k; ty <= nty; ty += nt) body(ty, k);
        });
    for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

void oracle_set_threads(int32_t threads) { g_threads = threads > 0 ? threads : 1; }

// fill_keep_gaussians_kernel! (forward_core.jl:326-355).
void oracle_fill_keep(const tdgs_gaussians* g, const tdgs_camera* cam,
                      const tdgs_render_options* opt, uint8_t* keep) {
    for (int64_t i = 0; i < g->n; ++i) {
        const float* mo = g->means_opacity + 4 * i;
        const float a = opacity_of(g->kind, mo[3]);
        keep[i] = keep_gaussian(*cam, *opt, mo[0], mo[1], mo[2], a) ? 1 : 0;
    }
}

// accumulate!(+) + fill_fgidx_to_gidx_kernel! (forward_core.jl:231-244, 371-386).
int32_t oracle_fill_fgidx_to_gidx(const uint8_t* keep, int32_t n, int32_t* keep_cs,
                                  int32_t* fgidx_to_gidx) {
    int32_t acc = 0;
    for (int32_t i = 0; i < n; ++i) {
        acc += keep[i] ? 1 : 0;
        if (keep_cs) keep_cs[i] = acc;
        if (keep[i]) fgidx_to_gidx[acc - 1] = i + 1;
    }
    return acc;
}

// project_fgaussians_kernel! (forward_core.jl:411-517). Records of Gaussians with an empty
// bounding box are left untouched, as in the reference.
void oracle_project(const tdgs_gaussians* g, const tdgs_camera* cam, const tdgs_tiling* t,
                    const tdgs_render_options* opt, int32_t nb_f, const int32_t* fgidx_to_gidx,
                    float* depths, float* f2d, int32_t* ranges, int32_t* counts) {
    const int hs = h_of(g->sh_degree);
    for (int32_t f = 0; f < nb_f; ++f) {
        const int64_t gi = fgidx_to_gidx[f] - 1;
        const float* mo = g->means_opacity + 4 * gi;
        const float a = opacity_of(g->kind, mo[3]);
        float params[7];
        gaussian_params(*g, gi, params);
        const Projected pr = project_geometry(*cam, *opt, *t, g->kind, mo[0], mo[1], mo[2], a, params);
        counts[f] = pr.count;
        if (pr.count == 0) continue;
        depths[f] = pr.depth;
        for (int k = 0; k < 4; ++k) ranges[4 * f + k] = pr.rect[k];
        float rgb[3];
        project_color(*cam, opt->sh_degree, g->sh + (int64_t)3 * hs * gi, hs, mo[0], mo[1], mo[2], rgb);
        float* r = f2d + 9 * (int64_t)f;
        r[0] = pr.mux; r[1] = pr.muy; r[2] = pr.a;
        r[3] = pr.m11; r[4] = pr.m21; r[5] = pr.m22;
        r[6] = rgb[0]; r[7] = rgb[1]; r[8] = rgb[2];
    }
}

// accumulate!(+) of overlapped tile counts (forward_core.jl:259-264).
int64_t oracle_scan_counts(const int32_t* counts, int32_t n, int32_t* counts_cs) {
    int64_t acc = 0;
    for (int32_t i = 0; i < n; ++i) {
        acc += counts[i];
        counts_cs[i] = (int32_t)acc;
    }
    return acc;
}

// fill_df2dgs_codes_and_dfgidx_to_fgidx_kernel! (forward_core.jl:531-603).
void oracle_emit_keys(int32_t nb_f, const float* depths, const int32_t* ranges,
                      const int32_t* counts_cs, const tdgs_tiling* t, int64_t* keys,
                      int32_t* values) {
    for (int32_t f = 0; f < nb_f; ++f) {
        int64_t d = f == 0 ? 0 : counts_cs[f - 1];
        if (d >= counts_cs[f]) continue;
        const int32_t* r = ranges + 4 * f;
        for (int32_t ty = r[1]; ty <= r[3]; ++ty) {
            for (int32_t tx = r[0]; tx <= r[2]; ++tx) {
                keys[d] = make_key(tx + (ty - 1) * t->nb_tiles_x, depths[f]);
                values[d] = f + 1;
                ++d;
            }
        }
    }
}

// CUB DeviceRadixSort::SortPairs on bits [0, end_bit) (cub_sort_pairs_wrapper.cu:31-43):
// a stable sort by the masked key; restated as std::stable_sort.
void oracle_sort_pairs(const int64_t* kin, int64_t* kout, const int32_t* vin, int32_t* vout,
                       int64_t n, int32_t end_bit) {
    const uint64_t mask = end_bit >= 64 ? ~0ull : ((1ull << end_bit) - 1ull);
    std::vector<int64_t> idx(n);
    std::iota(idx.begin(), idx.end(), 0);
    std::stable_sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) {
        return ((uint64_t)kin[a] & mask) < ((uint64_t)kin[b] & mask);
    });
    for (int64_t i = 0; i < n; ++i) {
        kout[i] = kin[idx[i]];
        vout[i] = vin[idx[i]];
    }
}

// fill_tiles_end_sdfgidx_kernel! (forward_core.jl:676-734).
void oracle_tile_ranges(int64_t m, const int64_t* sorted_keys, int32_t nb_tiles, int32_t* tiles_end) {
    if (m == 0) return;
    const int32_t first = (int32_t)(sorted_keys[0] >> 32);
    for (int32_t t = 1; t < first; ++t) tiles_end[t - 1] = 0;
    for (int64_t i = 1; i < m; ++i) {
        int32_t cur = (int32_t)(sorted_keys[i - 1] >> 32);
        const int32_t nxt = (int32_t)(sorted_keys[i] >> 32);
        while (cur < nxt) { tiles_end[cur - 1] = (int32_t)i; ++cur; }
    }
    for (int32_t cur = (int32_t)(sorted_keys[m - 1] >> 32); cur <= nb_tiles; ++cur)
        tiles_end[cur - 1] = (int32_t)m;
}

// render_tiles_kernel! (forward_core.jl:756-993) for tile (tx, ty), one pixel at a time:
// entries [beg, end) of the sorted list, entry s being values[s - base].
static void blend_tile(const tdgs_camera* cam, const tdgs_tiling* t, const tdgs_render_options* opt,
                       const float* f2d, const float* depths, const int32_t* values, int64_t base, int64_t beg,
                       int64_t end, int tx, int ty, float* rgb, float* T_img, float* depth_img, int32_t* last_img) {
    const int W = cam->width, H = cam->height, TW = t->tile_width, TH = t->tile_height;
    const float u0 = (float)((tx - 1) * TW), v0 = (float)((ty - 1) * TH);
    for (int pv = 1; pv <= TH; ++pv) {
        for (int pu = 1; pu <= TW; ++pu) {
            const int U = pu + (tx - 1) * TW, Vv = pv + (ty - 1) * TH;
            if (U > W || Vv > H) continue;
            const float cu = (float)pu - 0.5f, cv = (float)pv - 0.5f;
            const float uu = cu * cu, uv = cu * cv, vv = cv * cv;
            float T = 1.0f, C[3] = {0.0f, 0.0f, 0.0f}, D = 0.0f;
            int32_t last = 0;
            for (int64_t s = beg; s < end; ++s) {
                const int64_t f = values[s - base] - 1;
                const float* r = f2d + 9 * f;
                float p[6];
                blend_params(r[0], r[1], r[2], r[3], r[4], r[5], u0, v0, p);
                const float alpha = fminf(opt->max_alpha, exp_f(blend_exponent(p, cu, cv, uu, uv, vv)));
                if (alpha < opt->min_alpha) continue;
                const float Tn = T * (1.0f - alpha);
                if (Tn < opt->min_transmittance) break;
                const float w = T * alpha;
                C[0] = fmaf(w, r[6], C[0]);
                C[1] = fmaf(w, r[7], C[1]);
                C[2] = fmaf(w, r[8], C[2]);
                D = fmaf(w, depths[f], D);
                T = Tn;
                last = (int32_t)(s + 1);
            }
            const int64_t px = (int64_t)(Vv - 1) + (int64_t)H * (U - 1);
            if (rgb) {
                rgb[3 * px + 0] = fmaf(T, opt->background[0], C[0]);
                rgb[3 * px + 1] = fmaf(T, opt->background[1], C[1]);
                rgb[3 * px + 2] = fmaf(T, opt->background[2], C[2]);
            }
            if (T_img) T_img[px] = T;
            if (depth_img) depth_img[px] = D;
            if (last_img) last_img[px] = last;
        }
    }
}

void oracle_render_tiles(const tdgs_camera* cam, const tdgs_tiling* t,
                         const tdgs_render_options* opt, const float* f2d, const float* depths,
                         const int32_t* sorted_values, const int32_t* tiles_end,
                         float* rgb, float* T_img, float* depth_img, int32_t* last_img) {
    for_tile_rows(t->nb_tiles_y, [&](int ty, int) {
        for (int tx = 1; tx <= t->nb_tiles_x; ++tx) {
            const int tile = tx + (ty - 1) * t->nb_tiles_x;
            const int64_t beg = tile == 1 ? 0 : tiles_end[tile - 2];
            const int64_t end = tiles_end[tile - 1];
            blend_tile(cam, t, opt, f2d, depths, sorted_values, 0, beg, end, tx, ty, rgb, T_img, depth_img, last_img);
        }
    });
}

// The same for one tile whose sorted entries [beg, end) are given as list[0 .. end - beg)
// (a slice of a sorted list too large to copy whole); writes only that tile's pixels.
void oracle_blend_tile(const tdgs_camera* cam, const tdgs_tiling* t, const tdgs_render_options* opt,
                       const float* f2d, const float* depths, const int32_t* list, int64_t beg, int64_t end,
                       int32_t tx, int32_t ty, float* rgb, float* T_img, float* depth_img, int32_t* last_img) {
    blend_tile(cam, t, opt, f2d, depths, list, beg, beg, end, tx, ty, rgb, T_img, depth_img, last_img);
}

// render_void! (forward_structs.jl:743-757).
void oracle_render_void(const tdgs_camera* cam, const tdgs_render_options* opt, float* rgb,
                        float* T_img, float* depth_img, int32_t* last_img) {
    const int64_t P = (int64_t)cam->width * cam->height;
    for (int64_t i = 0; i < P; ++i) {
        if (rgb) for (int c = 0; c < 3; ++c) rgb[3 * i + c] = opt->background[c];
        if (T_img) T_img[i] = 1.0f;
        if (depth_img) depth_img[i] = kInf;
        if (last_img) last_img[i] = 0;
    }
}

// render! GPU semantics (forward_core.jl:196-314) run sequentially. Buffers are host
// arrays of the sizes tdgs_render_buffers documents; key arrays must hold the key count
// (query it first with keys == nullptr: then only the counts are produced).
int64_t oracle_render(const tdgs_gaussians* g, const tdgs_camera* cam, const tdgs_tiling* t,
                      const tdgs_render_options* opt, tdgs_render_buffers* b,
                      const tdgs_render_outputs* out, int32_t* nb_f_out) {
    std::vector<uint8_t> keep_local(g->n);
    uint8_t* keep = b->keep ? b->keep : keep_local.data();
    oracle_fill_keep(g, cam, opt, keep);
    const int32_t nb_f = oracle_fill_fgidx_to_gidx(keep, g->n, nullptr, b->fgidx_to_gidx);
    *nb_f_out = nb_f;
    if (nb_f == 0) {
        oracle_render_void(cam, opt, out->rgb, out->T, out->depth, out->last);
        return 0;
    }
    oracle_project(g, cam, t, opt, nb_f, b->fgidx_to_gidx, b->depths, b->f2d, b->tile_ranges, b->counts);
    std::vector<int32_t> cs(nb_f);
    const int64_t m = oracle_scan_counts(b->counts, nb_f, cs.data());
    if (m == 0) {
        oracle_render_void(cam, opt, out->rgb, out->T, out->depth, out->last);
        return 0;
    }
    if (b->keys == nullptr || m > b->key_capacity) return m;
    oracle_emit_keys(nb_f, b->depths, b->tile_ranges, cs.data(), t, b->keys, b->values);
    const int32_t nb_tiles = t->nb_tiles_x * t->nb_tiles_y;
    const int32_t end_bit = 33 + (int32_t)std::floor(std::log2((double)nb_tiles));
    oracle_sort_pairs(b->keys, b->sorted_keys, b->values, b->sorted_values, m, end_bit);
    oracle_tile_ranges(m, b->sorted_keys, nb_tiles, b->tiles_end);
    oracle_render_tiles(cam, t, opt, b->f2d, b->depths, b->sorted_values, b->tiles_end,
                        out->rgb, out->T, out->depth, out->last);
    return m;
}

// backward_render_tiles_kernel! (backward_core.jl:96-293) for tile (tx, ty): each pixel replays
// the tile's list from its last contributor back to the first entry. The list's entries
// first..end (1-based positions in the frame's sorted list) are list[first - base ..
// end - base] (list[0] holds position base). Gradients are accumulated in double precision per
// filtered Gaussian (acc: 9 x nb_f doubles).
static void backward_tile(const tdgs_camera* cam, const tdgs_tiling* t, const tdgs_render_options* opt,
                          const float* f2d, const int32_t* list, int64_t base, int64_t first, int64_t end, int tx,
                          int ty, const float* rgb_grad, const float* T_img, const int32_t* last_img, double* acc) {
    const int W = cam->width, H = cam->height, TW = t->tile_width, TH = t->tile_height;
    for (int pv = 1; pv <= TH; ++pv) {
        for (int pu = 1; pu <= TW; ++pu) {
            const int U = pu + (tx - 1) * TW, Vv = pv + (ty - 1) * TH;
            if (U > W || Vv > H) continue;
            const int64_t px = (int64_t)(Vv - 1) + (int64_t)H * (U - 1);
            float T = T_img[px];
            const int64_t last = last_img[px];
            const float g[3] = {rgb_grad[3 * px], rgb_grad[3 * px + 1], rgb_grad[3 * px + 2]};
            float psi[3] = {T * opt->background[0], T * opt->background[1], T * opt->background[2]};
            const float cu = (float)U - 0.5f, cv = (float)Vv - 0.5f;
            const int64_t start = std::min(last, end);
            for (int64_t s = start; s >= first; --s) {
                const int64_t f = list[s - base] - 1;
                const float* r = f2d + 9 * f;
                float du, dv;
                const float G = backward_gaussian(cu, cv, r[0], r[1], r[3], r[4], r[5], &du, &dv);
                const float alpha = fminf(opt->max_alpha, r[2] * G);
                if (alpha < opt->min_alpha) continue;
                float o[9];
                backward_pair(alpha, 1.0f / (1.0f - alpha), G, du, dv, r[3], r[4], r[5], r + 6, g, &T, psi, o);
                for (int k = 0; k < 9; ++k) acc[9 * f + k] += (double)o[k];
            }
        }
    }
}

// backward_render_tiles_kernel! (backward_core.jl:96-293) over every tile.
void oracle_backward_render_tiles(const tdgs_camera* cam, const tdgs_tiling* t,
                                  const tdgs_render_options* opt, const float* f2d,
                                  const int32_t* sorted_values, const int32_t* tiles_end,
                                  const float* rgb_grad, const float* T_img,
                                  const int32_t* last_img, double* grads2d_acc) {
    // nb_f is not passed: the accumulator covers the largest referenced fgidx
    int64_t nb_f = 0;
    const int64_t m = tiles_end[(int64_t)t->nb_tiles_x * t->nb_tiles_y - 1];
    for (int64_t s = 0; s < m; ++s) nb_f = std::max<int64_t>(nb_f, sorted_values[s]);
    const int nt = std::max(1, std::min(g_threads, t->nb_tiles_y));
    std::vector<std::vector<double>> part(nt > 1 ? nt : 0);
    for (auto& p : part) p.assign(9 * nb_f, 0.0);
    for_tile_rows(t->nb_tiles_y, [&](int ty, int k) {
        double* acc = nt > 1 ? part[k].data() : grads2d_acc;
        for (int tx = 1; tx <= t->nb_tiles_x; ++tx) {
            const int tile = tx + (ty - 1) * t->nb_tiles_x;
            const int64_t first = tile == 1 ? 1 : (int64_t)tiles_end[tile - 2] + 1;
            const int64_t end = tiles_end[tile - 1];
            backward_tile(cam, t, opt, f2d, sorted_values, 1, first, end, tx, ty, rgb_grad, T_img, last_img, acc);
        }
    });
    for (int k = 0; k < (int)part.size(); ++k)
        for (int64_t i = 0; i < 9 * nb_f; ++i) grads2d_acc[i] += part[k][i];
}

// The same for one tile whose sorted entries beg + 1 .. end (1-based) are list[0 .. end - beg)
// (a replay on a list the GPU sorted); adds into acc (9 x nb_f doubles).
void oracle_backward_tile(const tdgs_camera* cam, const tdgs_tiling* t, const tdgs_render_options* opt,
                          const float* f2d, const int32_t* list, int64_t beg, int64_t end, int32_t tx, int32_t ty,
                          const float* rgb_grad, const float* T_img, const int32_t* last_img, double* acc) {
    backward_tile(cam, t, opt, f2d, list, beg + 1, beg + 1, end, tx, ty, rgb_grad, T_img, last_img, acc);
}

// backward_project_fgaussians_kernel! (backward_core.jl:309-452) + compute_sh_coeffs_grad!
// (:936-964), for a trainable Gaussian vector. grads2d: 9 x nb_f floats.
void oracle_backward_project(const tdgs_gaussians* g, const tdgs_camera* cam,
                             const tdgs_render_options* opt, int32_t nb_f,
                             const int32_t* fgidx_to_gidx, const float* f2d, const int32_t* counts,
                             const float* grads2d, tdgs_gradients* out) {
    const int hs = h_of(g->sh_degree);
    const int hg = h_of(out->sh_degree);
    const int hr = h_of(opt->sh_degree);
    for (int32_t f = 0; f < nb_f; ++f) {
        const int64_t gi = fgidx_to_gidx[f] - 1;
        float* dsh = out->sh + (int64_t)3 * hg * f;
        if (counts[f] == 0) {
            // No key references this Gaussian: every 2D gradient is zero and so is every
            // 3D gradient (the reference evaluates the chain rule on zeros).
            for (int k = 0; k < 3; ++k) out->mean3d[3 * f + k] = 0.0f;
            out->opacity_feature[f] = 0.0f;
            for (int k = 0; k < 3; ++k) out->scaling_features[3 * f + k] = 0.0f;
            for (int k = 0; k < 4; ++k) out->rotation_features[4 * f + k] = 0.0f;
            for (int c = 0; c < 3; ++c) for (int k = 0; k < hr; ++k) dsh[c * hg + k] = 0.0f;
            continue;
        }
        BackwardProjectIn in;
        const float* mo = g->means_opacity + 4 * gi;
        in.m[0] = mo[0]; in.m[1] = mo[1]; in.m[2] = mo[2];
        in.logit = mo[3];
        for (int k = 0; k < 3; ++k) in.logs[k] = g->scaling[3 * gi + k];
        for (int k = 0; k < 4; ++k) in.q[k] = g->rotation[4 * gi + k];
        in.sh = g->sh + (int64_t)3 * hs * gi;
        in.h_storage = hs;
        const float* r = f2d + 9 * (int64_t)f;
        in.mux = r[0]; in.muy = r[1]; in.a = r[2]; in.m11 = r[3]; in.m21 = r[4]; in.m22 = r[5];
        in.rgb[0] = r[6]; in.rgb[1] = r[7]; in.rgb[2] = r[8];
        for (int k = 0; k < 9; ++k) in.g2[k] = grads2d[9 * (int64_t)f + k];
        const BackwardProjectOut o = backward_project(in, *cam, *opt);
        for (int k = 0; k < 3; ++k) out->mean3d[3 * f + k] = o.dm[k];
        out->opacity_feature[f] = o.dlogit;
        for (int k = 0; k < 3; ++k) out->scaling_features[3 * f + k] = o.dlogs[k];
        for (int k = 0; k < 4; ++k) out->rotation_features[4 * f + k] = o.dq[k];
        float b[16];
        sh_grad_basis(*cam, opt->sh_degree, in.m, b);
        for (int c = 0; c < 3; ++c)
            for (int k = 0; k < hr; ++k) dsh[c * hg + k] = in.g2[6 + c] * b[k];
    }
}

// update! (optimizer.jl:964-1009) with scalar_adam_update (:941-953).
void oracle_adam_step(tdgs_gaussians* g, tdgs_adam_state* st, const tdgs_gradients* gr,
                      const int32_t* fgidx_to_gidx, int32_t nb_f, int32_t sh_degree) {
    const double t = (double)st->update_count + 1.0;
    const float bc1 = (float)(1.0 - std::pow((double)st->beta1, t));
    const float bc2 = (float)(1.0 - std::pow((double)st->beta2, t));
    const float b1 = st->beta1, b2 = st->beta2, o1 = 1.0f - b1, o2 = 1.0f - b2, eps = st->epsilon;
    const int hs = h_of(g->sh_degree), hg = h_of(gr->sh_degree), hr = h_of(sh_degree);
    for (int32_t f = 0; f < nb_f; ++f) {
        const int64_t gi = (int64_t)fgidx_to_gidx[f] - 1;
        if (gi < 0) continue;
        for (int k = 0; k < 3; ++k)
            adam_scalar(g->means_opacity[4 * gi + k], gr->mean3d[3 * f + k], st->means_moments[6 * gi + 2 * k],
                        st->means_moments[6 * gi + 2 * k + 1], st->lr_means, b1, b2, o1, o2, bc1, bc2, eps);
        adam_scalar(g->means_opacity[4 * gi + 3], gr->opacity_feature[f], st->opacity_moments[2 * gi],
                    st->opacity_moments[2 * gi + 1], st->lr_opacity, b1, b2, o1, o2, bc1, bc2, eps);
        for (int k = 0; k < 3; ++k)
            adam_scalar(g->scaling[3 * gi + k], gr->scaling_features[3 * f + k], st->scaling_moments[6 * gi + 2 * k],
                        st->scaling_moments[6 * gi + 2 * k + 1], st->lr_scaling, b1, b2, o1, o2, bc1, bc2, eps);
        for (int k = 0; k < 4; ++k)
            adam_scalar(g->rotation[4 * gi + k], gr->rotation_features[4 * f + k], st->rotation_moments[8 * gi + 2 * k],
                        st->rotation_moments[8 * gi + 2 * k + 1], st->lr_rotation, b1, b2, o1, o2, bc1, bc2, eps);
        for (int c = 0; c < 3; ++c) {
            for (int k = 0; k < hr; ++k) {
                const int64_t pi = (int64_t)3 * hs * gi + c * hs + k;
                const int64_t mi = 2 * pi;
                adam_scalar(g->sh[pi], gr->sh[(int64_t)3 * hg * f + c * hg + k], st->sh_moments[mi],
                            st->sh_moments[mi + 1], k == 0 ? st->lr_sh_dc : st->lr_sh_rest, b1, b2, o1, o2,
                            bc1, bc2, eps);
            }
        }
    }
    st->update_count += 1;
}

// update_adc_stats_kernel! (training.jl:472-497); the norm is formed in double precision
// as the reference does ((h^2, w^2) ./ 4 is a Float64 pair there).
void oracle_adc_stats(tdgs_adc_buffers* adc, const float* grads2d, const int32_t* fgidx_to_gidx,
                      int32_t nb_f, int32_t width, int32_t height) {
    const double sw = (double)width * width / 4.0, sh = (double)height * height / 4.0;
    for (int32_t f = 0; f < nb_f; ++f) {
        const float gx = grads2d[9 * (int64_t)f], gy = grads2d[9 * (int64_t)f + 1];
        if (gx != 0.0f || gy != 0.0f) {
            const int64_t gi = fgidx_to_gidx[f] - 1;
            const double nrm = std::sqrt((double)(gx * gx) * sw + (double)(gy * gy) * sh);
            adc->accum_grad_norms[gi] = (float)((double)adc->accum_grad_norms[gi] + nrm);
            adc->contribution_counts[gi] += 1;
        }
    }
}

// Masks, counts, scan and fill_ngidx_to_gidx_kernel! (training.jl:325-397, 557-580).
int32_t oracle_adc_plan(tdgs_adc_buffers* adc, const tdgs_gaussians* g, float prune_logit,
                        int32_t use_max_scale, float log_max_scale, float grad_threshold,
                        float log_size_threshold) {
    int32_t acc = 0;
    for (int32_t i = 0; i < g->n; ++i) {
        const int32_t cnt = adc->contribution_counts[i];
        const float avg = cnt >= 1 ? adc->accum_grad_norms[i] / (float)cnt : 0.0f;
        const float* s = g->scaling + 3 * (int64_t)i;
        const float smax = fmaxf(fmaxf(s[0], s[1]), s[2]);
        bool prune = g->means_opacity[4 * (int64_t)i + 3] < prune_logit;
        if (use_max_scale) prune = prune || smax > log_max_scale;
        const bool dens = !prune && avg >= grad_threshold;
        const bool clone = dens && smax <= log_size_threshold;
        adc->prune[i] = prune; adc->densify[i] = dens; adc->clone[i] = clone;
        acc += (prune ? 0 : 1) + (dens ? 1 : 0);
        adc->new_counts_cs[i] = acc;
    }
    for (int32_t i = 0; i < g->n; ++i) {
        if (adc->prune[i]) continue;
        const int32_t last = adc->new_counts_cs[i];
        if (adc->densify[i] && last <= adc->new_capacity) {
            adc->ngidx_to_gidx[last - 2] = i + 1;
            adc->ngidx_to_gidx[last - 1] = i + 1;
        } else if (last <= adc->new_capacity) {
            adc->ngidx_to_gidx[last - 1] = i + 1;
        }
    }
    return acc;
}

// adaptive_density_control! for parameters (gaussians.jl:1526-1694) and moments
// (optimizer.jl:1304-1378). Split draws use the same counter-based sampler as the kernel.
void oracle_adc_apply(const tdgs_adc_buffers* adc, const tdgs_gaussians* src, tdgs_gaussians* dst,
                      const tdgs_adam_state* sm, tdgs_adam_state* dm, float log_split_factor,
                      uint64_t seed) {
    const int h = h_of(src->sh_degree);
    const int n_new = adc->new_counts_cs[src->n - 1];
    // zero moments of all new Gaussians first
    std::fill(dm->means_moments, dm->means_moments + 6 * (int64_t)n_new, 0.0f);
    std::fill(dm->opacity_moments, dm->opacity_moments + 2 * (int64_t)n_new, 0.0f);
    std::fill(dm->scaling_moments, dm->scaling_moments + 6 * (int64_t)n_new, 0.0f);
    std::fill(dm->rotation_moments, dm->rotation_moments + 8 * (int64_t)n_new, 0.0f);
    std::fill(dm->sh_moments, dm->sh_moments + (int64_t)6 * h * n_new, 0.0f);
    for (int32_t i = 0; i < src->n; ++i) {
        if (adc->prune[i]) continue;
        const int64_t last = adc->new_counts_cs[i] - 1;  // 0-based
        const float* mo = src->means_opacity + 4 * (int64_t)i;
        const float* s = src->scaling + 3 * (int64_t)i;
        auto copy_rest = [&](int64_t ni) {
            for (int k = 0; k < 4; ++k) dst->rotation[4 * ni + k] = src->rotation[4 * (int64_t)i + k];
            for (int k = 0; k < 3 * h; ++k) dst->sh[3 * h * ni + k] = src->sh[3 * h * (int64_t)i + k];
        };
        auto copy_moments = [&](int64_t ni) {
            for (int k = 0; k < 6; ++k) dm->means_moments[6 * ni + k] = sm->means_moments[6 * (int64_t)i + k];
            for (int k = 0; k < 2; ++k) dm->opacity_moments[2 * ni + k] = sm->opacity_moments[2 * (int64_t)i + k];
            for (int k = 0; k < 6; ++k) dm->scaling_moments[6 * ni + k] = sm->scaling_moments[6 * (int64_t)i + k];
            for (int k = 0; k < 8; ++k) dm->rotation_moments[8 * ni + k] = sm->rotation_moments[8 * (int64_t)i + k];
            for (int k = 0; k < 6 * h; ++k) dm->sh_moments[6 * h * ni + k] = sm->sh_moments[6 * h * (int64_t)i + k];
        };
        if (!adc->densify[i]) {
            for (int k = 0; k < 4; ++k) dst->means_opacity[4 * last + k] = mo[k];
            for (int k = 0; k < 3; ++k) dst->scaling[3 * last + k] = s[k];
            copy_rest(last);
            copy_moments(last);
        } else if (adc->clone[i]) {
            for (int64_t ni : {last - 1, last}) {
                for (int k = 0; k < 4; ++k) dst->means_opacity[4 * ni + k] = mo[k];
                for (int k = 0; k < 3; ++k) dst->scaling[3 * ni + k] = s[k];
                copy_rest(ni);
            }
            copy_moments(last - 1);
        } else {
            float R[9];
            const float* q = src->rotation + 4 * (int64_t)i;
            quat_to_rot(q[0], q[1], q[2], q[3], R);
            const float sc[3] = {exp_f(s[0]), exp_f(s[1]), exp_f(s[2])};
            float z[6];
            normal_pair(seed, (uint64_t)i, 0, &z[0], &z[1]);
            normal_pair(seed, (uint64_t)i, 1, &z[2], &z[3]);
            normal_pair(seed, (uint64_t)i, 2, &z[4], &z[5]);
            for (int j = 0; j < 2; ++j) {
                const int64_t ni = last - 1 + j;
                const float w0 = z[3 * j] * sc[0], w1 = z[3 * j + 1] * sc[1], w2 = z[3 * j + 2] * sc[2];
                for (int k = 0; k < 3; ++k)
                    dst->means_opacity[4 * ni + k] = mo[k] + fmaf(R[3 * k + 2], w2, fmaf(R[3 * k + 1], w1, R[3 * k] * w0));
                dst->means_opacity[4 * ni + 3] = mo[3];
                for (int k = 0; k < 3; ++k) dst->scaling[3 * ni + k] = s[k] + log_split_factor;
                copy_rest(ni);
            }
        }
    }
}

// adjust_fgidx_to_gidx_adc_kernel! (training.jl:514-541).
void oracle_adc_remap_fgidx(const tdgs_adc_buffers* adc, int32_t* fgidx_to_gidx, int32_t nb_f) {
    for (int32_t f = 0; f < nb_f; ++f) {
        const int64_t gi = fgidx_to_gidx[f] - 1;
        int32_t ng = 0;
        if (!adc->prune[gi]) {
            if (adc->densify[gi]) {
                if (adc->clone[gi]) ng = adc->new_counts_cs[gi] - 1;
            } else {
                ng = adc->new_counts_cs[gi];
            }
        }
        fgidx_to_gidx[f] = ng;
    }
}

// L1 loss gradient (training.jl:206-215): the pixel weight l1_px_weight = (1 - w) / length
// (:213, l1_weight = 1 - w), +weight where rendered > gt and -weight otherwise (ties included,
// :214-215), plus w times the D-SSIM gradient as a separate product and sum (Julia's broadcast
// `ifelse.(...) .+ weight .* grad` rounds the product, then the sum; no fused multiply-add).
double oracle_l1_loss_grad(const float* rendered, const float* gt, int64_t count, float l1_weight,
                           float dssim_weight, const float* dssim_grad, float* grad_out) {
    const float w = l1_weight / (float)count;
    double acc = 0.0;
    for (int64_t i = 0; i < count; ++i) {
        acc += std::fabs((double)rendered[i] - (double)gt[i]);
        const float base = rendered[i] > gt[i] ? w : -w;
        grad_out[i] = dssim_grad ? base + dssim_weight * dssim_grad[i] : base;
    }
    return acc;
}

// ------------------------------------------------------------------------------------
// The reference's own CPU renderer (render! for CPU arrays, forward_core.jl:25-177):
// no tiles; per kept Gaussian in depth order, the exact pixel span of its alpha = min_alpha
// ellipse; a Gaussian that would drop T below min_T is skipped for that pixel only.
// Used as the CPU baseline. threads > 1 deals the image columns to the threads (thread k
// takes the columns u = k + 1 mod threads), each walking all Gaussians over its own columns:
// per-pixel order is unchanged, so the output equals the single-threaded one bit for bit.
// ------------------------------------------------------------------------------------

namespace {
struct CpuGaussian2D {
    float mux, muy, a, m11, m21, m22, depth, rgb[3];
};

// Splats the Gaussians (in `order`) over the image columns u in [u_lo, u_hi] with
// u = u_first (mod u_step).
void cpu_render_band(const std::vector<CpuGaussian2D>& gs, const std::vector<int64_t>& order,
                     const tdgs_camera& cam, const tdgs_render_options& o, int u_lo, int u_hi, int u_first,
                     int u_step, float* rgb, float* T_img) {
    const int W = cam.width, H = cam.height;
    for (int64_t oi : order) {
        const CpuGaussian2D& g = gs[oi];
        const float idet = fmaf(g.m11, g.m22, -(g.m21 * g.m21));
        const float gamma = 2.0f * log_f(g.a / o.min_alpha) / idet;
        const float q = g.m21, r = g.m22;
        const float x_radius = sqrtf(r * gamma);
        if (!(x_radius >= 0.0f)) continue;
        const float us = ceilf(g.mux - x_radius + 0.5f);
        const float ue = rintf(g.mux + x_radius);
        if (!(us == us) || !(ue == ue)) continue;
        int u_start = std::max(u_lo, (int)clampf(us, 1.0f, (float)W + 1.0f));
        const int u_end = std::min(u_hi, (int)clampf(ue, 0.0f, (float)W));
        u_start += ((u_first - u_start) % u_step + u_step) % u_step;   // next column of the stride
        const float ir = 1.0f / r;
        for (int u = u_start; u <= u_end; u += u_step) {
            const float du = ((float)u - 0.5f) - g.mux;
            const float disc = fmaf(r, gamma, -(du * du));
            const float sq = disc <= 0.0f ? 0.0f : sqrtf(idet * disc);
            const float qdu = q * du;
            const float top = g.muy + (-qdu - sq) * ir;
            const float bottom = g.muy + (-qdu + sq) * ir;
            const float vs = ceilf(top + 0.5f), ve = rintf(bottom);
            if (!(vs == vs) || !(ve == ve)) continue;
            const int v_start = (int)clampf(vs, 1.0f, (float)H + 1.0f);
            const int v_stop = (int)clampf(ve, 0.0f, (float)H);
            for (int v = v_start; v <= v_stop; ++v) {
                const float dv = ((float)v - 0.5f) - g.muy;
                const float G = exp_f(fmaf(-0.5f, fmaf(g.m11 * du, du, g.m22 * dv * dv), -(g.m21 * du) * dv));
                const float alpha = fminf(o.max_alpha, g.a * G);
                const int64_t px = (int64_t)(v - 1) + (int64_t)H * (u - 1);
                const float cur = T_img[px];
                const float nxt = cur * (1.0f - alpha);
                if (nxt < o.min_transmittance) continue;
                const float w = alpha * cur;
                rgb[3 * px] = fmaf(w, g.rgb[0], rgb[3 * px]);
                rgb[3 * px + 1] = fmaf(w, g.rgb[1], rgb[3 * px + 1]);
                rgb[3 * px + 2] = fmaf(w, g.rgb[2], rgb[3 * px + 2]);
                T_img[px] = nxt;
            }
        }
    }
}
}  // namespace

namespace {
// The per-Gaussian part of the reference CPU renderer: cull, project and colour every
// Gaussian, then a stable sort by depth (forward_core.jl:25-116).
void cpu_reference_prepare(const tdgs_gaussians* g, const tdgs_camera* cam, const tdgs_render_options* opt,
                           std::vector<CpuGaussian2D>& gs, std::vector<int64_t>& order) {
    const int hs = h_of(g->sh_degree);
    gs.clear();
    gs.reserve(g->n);
    tdgs_tiling unit{1, 1, cam->width, cam->height};
    for (int64_t i = 0; i < g->n; ++i) {
        const float* mo = g->means_opacity + 4 * i;
        const float a = opacity_of(g->kind, mo[3]);
        if (!(a >= opt->min_alpha)) continue;
        float mux, muy, depth;
        project_point(cam->P, mo[0], mo[1], mo[2], &mux, &muy, &depth);
        if (!(cam->near_z < depth && depth <= cam->far_z)) continue;
        if (opt->clip_mode == TDGS_CLIP_FILTER && !on_extended_screen(*opt, mux, muy)) continue;
        float params[7];
        gaussian_params(*g, i, params);
        const Projected pr = project_geometry(*cam, *opt, unit, g->kind, mo[0], mo[1], mo[2], a, params);
        CpuGaussian2D c;
        c.mux = pr.mux; c.muy = pr.muy; c.a = pr.a; c.m11 = pr.m11; c.m21 = pr.m21; c.m22 = pr.m22;
        c.depth = pr.depth;
        project_color(*cam, opt->sh_degree, g->sh + (int64_t)3 * hs * i, hs, mo[0], mo[1], mo[2], c.rgb);
        gs.push_back(c);
    }
    order.resize(gs.size());
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return gs[a].depth < gs[b].depth; });
}

// Splat the sorted Gaussians over the image columns u = u_first (mod u_step) with `threads`
// threads, thread k taking every threads-th of those columns.
void cpu_reference_splat(const std::vector<CpuGaussian2D>& gs, const std::vector<int64_t>& order,
                         const tdgs_camera* cam, const tdgs_render_options* opt, int32_t threads, int u_first,
                         int u_step, float* rgb, float* T_img) {
    const int W = cam->width;
    if (threads <= 1) {
        cpu_render_band(gs, order, *cam, *opt, 1, W, u_first, u_step, rgb, T_img);
        return;
    }
    std::vector<std::thread> pool;
    for (int k = 0; k < threads; ++k)
        pool.emplace_back(cpu_render_band, std::cref(gs), std::cref(order), std::cref(*cam), std::cref(*opt), 1, W,
                          u_first + k * u_step, u_step * threads, rgb, T_img);
    for (auto& th : pool) th.join();
}
}  // namespace

void cpu_render_reference(const tdgs_gaussians* g, const tdgs_camera* cam,
                          const tdgs_render_options* opt, int32_t threads, float* rgb,
                          float* T_img) {
    const int64_t P = (int64_t)cam->width * cam->height;
    std::fill(rgb, rgb + 3 * P, 0.0f);
    std::fill(T_img, T_img + P, 1.0f);
    std::vector<CpuGaussian2D> gs;
    std::vector<int64_t> order;
    cpu_reference_prepare(g, cam, opt, gs, order);
    cpu_reference_splat(gs, order, cam, opt, threads, 1, 1, rgb, T_img);
    for (int64_t i = 0; i < P; ++i)
        for (int c = 0; c < 3; ++c) rgb[3 * i + c] = fmaf(T_img[i], opt->background[c], rgb[3 * i + c]);
}

// Timing of the reference CPU renderer (std::chrono::steady_clock): seconds_out[0] = the
// per-Gaussian part (cull, projection, colour, depth sort), seconds_out[1] = the splatting of
// the image columns u = u_first (mod u_step) with `threads` threads. The images receive those
// columns only.
void cpu_render_reference_timed(const tdgs_gaussians* g, const tdgs_camera* cam, const tdgs_render_options* opt,
                                int32_t threads, int32_t u_first, int32_t u_step, float* rgb, float* T_img,
                                double* seconds_out) {
    const int64_t P = (int64_t)cam->width * cam->height;
    std::fill(rgb, rgb + 3 * P, 0.0f);
    std::fill(T_img, T_img + P, 1.0f);
    std::vector<CpuGaussian2D> gs;
    std::vector<int64_t> order;
    const auto t0 = std::chrono::steady_clock::now();
    cpu_reference_prepare(g, cam, opt, gs, order);
    const auto t1 = std::chrono::steady_clock::now();
    cpu_reference_splat(gs, order, cam, opt, threads, u_first, u_step, rgb, T_img);
    const auto t2 = std::chrono::steady_clock::now();
    seconds_out[0] = std::chrono::duration<double>(t1 - t0).count();
    seconds_out[1] = std::chrono::duration<double>(t2 - t1).count();
}

// Scalar helpers exposed for closed-form checks of the shared mathematics.
float oracle_exp(float x) { return exp_f(x); }
float oracle_log(float x) { return log_f(x); }
void oracle_exp_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = exp_f(x[i]);
}
void oracle_log_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = log_f(x[i]);
}
float oracle_sigmoid(float x) { return sigmoid_f(x); }
void oracle_quat_to_rot(const float* q, float* R) { quat_to_rot(q[0], q[1], q[2], q[3], R); }
void oracle_normal_pair(uint64_t seed, uint64_t stream, uint32_t pair, float* out) {
    normal_pair(seed, stream, pair, &out[0], &out[1]);
}

}  // extern "C"
