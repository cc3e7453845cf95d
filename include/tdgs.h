/*
 * tdgs.h — C-ABI of libtdgs, the MI355X (gfx950) render/train core for 3D Gaussian
 * Splatting. Every entry point takes plain pointers and sizes; device buffers are owned by
 * the caller; every call is asynchronous on the given HIP stream unless stated otherwise.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   render!                        src/forward_core.jl:196-314
 *   fill_keep_gaussians_kernel!    src/forward_core.jl:326-355
 *   fill_fgidx_to_gidx_kernel!     src/forward_core.jl:371-386   (+ accumulate! at :231)
 *   project_fgaussians_kernel!     src/forward_core.jl:411-517
 *   fill_df2dgs_codes_..._kernel!  src/forward_core.jl:531-603   (+ accumulate! at :259)
 *   sort_pairs / determine_sort_pairs_temp_storage
 *                                  deps/cub_sort_pairs/cub_sort_pairs_wrapper.cu:31-61,
 *                                  called from src/forward_core.jl:618-660
 *   fill_tiles_end_sdfgidx_kernel! src/forward_core.jl:676-734
 *   render_tiles_kernel!           src/forward_core.jl:756-993
 *   render_void!                   src/forward_structs.jl:743-757
 *   backward!                      src/backward_core.jl:37-72
 *   update! (Adam)                 src/optimizer.jl:964-1009, 1084-1127, 1165-1248
 *   adaptive_density_control!      src/gaussians.jl:1526-1694, src/optimizer.jl:1304-1378
 *   maybe_densify_and_prune!       src/training.jl:313-444, 472-580
 *
 * Conventions (identical to the reference so results compare bit for bit):
 *   - Arrays use the reference's Julia column-major layouts: "k x n" means k contiguous
 *     values per element. Images are 3 x h x w (rgb) and h x w (T, depth, last); pixel
 *     (row v, column u), 1-based, sits at offset (v-1) + h*(u-1).
 *   - Index values stored in buffers are 1-based (fgidx_to_gidx, sorted values, tiles_end,
 *     last contributor; 0 means "none").
 *   - Keys are (int64(tile) << 32) | int32 bits of the float32 depth; tile = tx + (ty-1)*ntx.
 *   - Return value: TDGS_OK or an error code; tdgs_last_error() gives the message of the
 *     last failure on the calling host thread. No exception crosses the ABI.
 *   - Calls that report a count back to the host (number of filtered Gaussians, number of
 *     duplicated keys, number of Gaussians after densification) synchronise their stream.
 *   - A context (tdgs_ctx_create) holds the device counters of the frame in progress: frames
 *     rendered concurrently on several streams each need their own context, render buffers
 *     and outputs (the Gaussians may be shared); calls on one context are ordered on one
 *     stream.
 */
#ifndef TDGS_H
#define TDGS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TDGS_ABI_VERSION 2

enum {
    TDGS_OK = 0,
    TDGS_ERR_INVALID = 1,     /* bad argument: null pointer, size, degree, tile shape */
    TDGS_ERR_CAPACITY = 2,    /* a caller buffer is too small; the *_out count says how big */
    TDGS_ERR_HIP = 3,         /* a HIP runtime call failed */
    TDGS_ERR_UNSUPPORTED = 4, /* option combination not implemented */
    TDGS_ERR_DEVICE = 5       /* a kernel detected inconsistent data (reported at a sync point) */
};

enum { TDGS_TRAINABLE = 0, TDGS_RENDER_ONLY = 1 };
enum { TDGS_CLIP_CLAMP = 0, TDGS_CLIP_FILTER = 1 };  /* CovarianceBoundaryClamp / BoundaryFilter */

/* tdgs_render_options.flags */
#define TDGS_FLAG_EXACT_SH_JACOBIAN 0x1  /* use basis coefficient 16 where src/sh.jl:249 uses 15 */
/* With antialiasing the forward pass scales the opacity by f = max(aa_min, sqrt(det0 / det))
 * (forward_core.jl:450-462), but the reference's backward pass adds a0 * dL/da * d(det0/det)/dSigma
 * to the covariance gradient (backward_core.jl:480-490, derived for f = det0/det in
 * docs/src/math.md:194-197): the derivative of f^2, not of f. That is reproduced by default; this
 * flag uses the derivative of f instead (d(f^2)/dSigma / (2 f), zero where f is clamped to aa_min). */
#define TDGS_FLAG_EXACT_AA_GRADIENT 0x2
/* tdgs_render without host synchronisation (no counterpart in the reference, which reads the
 * filtered and key counts on the host every frame, forward_core.jl:231-233, 259-264): the
 * launches after the count scan are sized by buf->key_capacity and read the counts on the
 * device; *nb_fgaussians_out and *nb_keys_out are set to -1 and the frame's counts stay in
 * device memory (tdgs_render_counts reads them; the entry points below that take
 * nb_fgaussians accept -1 with the render buffers and read them there). A key count above
 * buf->key_capacity renders the frame as render_void! would and sets the frame status to
 * TDGS_FRAME_KEY_CAPACITY (nb_keys still says how many keys are needed); the fused backward
 * projection + Adam then leaves the parameters untouched. Needs at most 65535 tiles. */
#define TDGS_FLAG_DEVICE_COUNTS 0x4

/* PinholeCamera (src/cameras.jl:50-106): P = K [R^T | -R^T t] cached as 3x4, row-major here. */
typedef struct tdgs_camera {
    int32_t width;
    int32_t height;
    float P[12];        /* row-major 3x4 projection matrix */
    float near_z;       /* exclusive */
    float far_z;        /* inclusive (may be +inf) */
    float position[3];  /* camera centre (camera-to-world translation) */
} tdgs_camera;

/* RenderOptions (src/forward_structs.jl:579-665); clip bounds already in pixel units. */
typedef struct tdgs_render_options {
    float background[3];
    float aa_min_factor;
    float min_alpha;
    float max_alpha;
    float min_transmittance;
    float dilation_x;
    float dilation_y;
    float clip_x_min, clip_x_max, clip_y_min, clip_y_max;
    int32_t sh_degree;   /* degree used for colour; <= the Gaussians' storage degree */
    int32_t clip_mode;   /* TDGS_CLIP_CLAMP or TDGS_CLIP_FILTER */
    int32_t antialiasing;
    int32_t flags;
} tdgs_render_options;

/* Tiling (src/forward_structs.jl:340-380): ntx = cld(w, tw), nty = cld(h, th). */
typedef struct tdgs_tiling {
    int32_t tile_width;
    int32_t tile_height;
    int32_t nb_tiles_x;
    int32_t nb_tiles_y;
} tdgs_tiling;

/* TrainableGaussiansVector (src/gaussians.jl:29-98) or RenderOnlyGaussiansVector (:342-392). */
typedef struct tdgs_gaussians {
    int32_t kind;           /* TDGS_TRAINABLE or TDGS_RENDER_ONLY */
    int32_t n;
    int32_t sh_degree;      /* storage degree: (sh_degree+1)^2 coefficients per channel */
    int32_t reserved;
    float* means_opacity;   /* 4 x n: [x, y, z, opacity logit] or [x, y, z, opacity] */
    float* scaling;         /* 3 x n log-scales (trainable) */
    float* rotation;        /* 4 x n unnormalised quaternions [r, x, y, z] (trainable) */
    float* covariances;     /* 6 x n lower [V11, V21, V31, V22, V32, V33] (render-only) */
    float* sh;              /* h x 3 x n, coefficient fastest */
} tdgs_gaussians;

/* RenderBuffers (src/forward_structs.jl:1541-1677) + Filtered2DGaussiansVector (:762-833). */
typedef struct tdgs_render_buffers {
    int32_t capacity;        /* per-Gaussian arrays hold this many entries (>= n) */
    int32_t reserved;
    int64_t key_capacity;    /* per-key arrays hold this many entries */
    uint8_t* keep;           /* capacity; keep flags (written when non-null) */
    int32_t* fgidx_to_gidx;  /* capacity; 1-based */
    float* depths;           /* capacity */
    float* f2d;              /* 9 x capacity: [mu_x, mu_y, a, M11, M21, M22, r, g, b]; 16-byte aligned */
    int32_t* tile_ranges;    /* 4 x capacity: [tx_min, ty_min, tx_max, ty_max] */
    int32_t* counts;         /* capacity; overlapped tiles per filtered Gaussian */
    int64_t* keys;           /* key_capacity; scratch of the tile sort */
    int32_t* values;         /* key_capacity; scratch of the tile sort */
    int64_t* sorted_keys;    /* key_capacity */
    int32_t* sorted_values;  /* key_capacity; sdfgidx_to_fgidx, 1-based */
    int32_t* tiles_end;      /* nb_tiles; tiles_end_sdfgidx */
    void* temp;              /* scratch of tdgs_render_temp_bytes() bytes */
    size_t temp_bytes;
} tdgs_render_buffers;

/* RenderOutputs (src/forward_structs.jl:1-129); each pointer may be null (not requested). */
typedef struct tdgs_render_outputs {
    float* rgb;      /* 3 x h x w */
    float* T;        /* h x w transmittance */
    float* depth;    /* h x w */
    int32_t* last;   /* h x w last contributing sorted index (1-based, 0 = none) */
} tdgs_render_outputs;

/* FilteredGaussiansGradientsVector (src/backward_structs.jl:1-93). The 2D gradients come in
 * either of two layouts:
 *   - the reference's four arrays (grads2d null): mean2d_grads 2 x capacity, opacity_grads
 *     capacity, licov2d_grads (lower [M11, M21, M22]) 3 x capacity, color_grads 3 x capacity,
 *     exactly as backward_structs.jl:17-22 holds them, so a Julia caller passes its arrays;
 *   - one interleaved 9 x capacity array (grads2d non-null, the four pointers ignored):
 *     [dmu_x, dmu_y, da, dM11, dM21, dM22, dr, dg, db] per filtered Gaussian, so the nine
 *     accumulations of one Gaussian hit one or two cache lines (the faster layout).
 * The 3D gradient arrays keep the reference layout. */
typedef struct tdgs_gradients {
    int32_t capacity;
    int32_t sh_degree;          /* storage degree of sh */
    float* grads2d;             /* 9 x capacity, or null for the four arrays below */
    float* mean2d_grads;        /* 2 x capacity (used when grads2d is null) */
    float* opacity_grads;       /* capacity */
    float* licov2d_grads;       /* 3 x capacity */
    float* color_grads;         /* 3 x capacity */
    float* mean3d;              /* 3 x capacity */
    float* opacity_feature;     /* capacity */
    float* scaling_features;    /* 3 x capacity */
    float* rotation_features;   /* 4 x capacity */
    float* sh;                  /* h x 3 x capacity */
} tdgs_gradients;

/* GaussianAdamMomentsLearningRatesVector + AdamOptimizer (src/optimizer.jl:9-195, 761-854). */
typedef struct tdgs_adam_state {
    float* means_moments;       /* 2 x 3 x n (m1, m2 interleaved) */
    float* opacity_moments;     /* 2 x n */
    float* scaling_moments;     /* 2 x 3 x n */
    float* rotation_moments;    /* 2 x 4 x n */
    float* sh_moments;          /* 2 x h x 3 x n */
    float lr_means, lr_opacity, lr_scaling, lr_rotation, lr_sh_dc, lr_sh_rest;
    float beta1, beta2, epsilon;
    int32_t update_count;       /* incremented by tdgs_adam_step */
} tdgs_adam_state;

/* AdaptiveDensityControlBuffers (src/training_structs.jl:265-331). */
typedef struct tdgs_adc_buffers {
    int32_t capacity;           /* per-Gaussian arrays (>= n) */
    int32_t new_capacity;       /* ngidx_to_gidx capacity */
    float* accum_grad_norms;    /* capacity; accumulated mean2d grad norms (NDC) */
    int32_t* contribution_counts; /* capacity */
    uint8_t* prune;             /* capacity */
    uint8_t* densify;           /* capacity */
    uint8_t* clone;             /* capacity */
    int32_t* new_counts_cs;     /* capacity; inclusive scan of (!prune + densify) */
    int32_t* ngidx_to_gidx;     /* new_capacity; 1-based */
    void* temp;                 /* scratch of tdgs_scan_temp_bytes(capacity) bytes */
    size_t temp_bytes;
} tdgs_adc_buffers;

typedef struct tdgs_ctx tdgs_ctx;

/* Stages timed by the optional profiler (tdgs_profile_begin/end). */
enum {
    TDGS_STAGE_CULL_COMPACT = 0,   /* keep flags + compaction (scan) */
    TDGS_STAGE_PROJECT = 1,        /* projection, SH colour, tile rectangles */
    TDGS_STAGE_DEPTH_SORT = 2,     /* radix sort of the Gaussians by depth */
    TDGS_STAGE_COUNT_SCAN = 3,     /* scan of overlapped-tile counts */
    TDGS_STAGE_EMIT = 4,           /* key duplication */
    TDGS_STAGE_TILE_SORT = 5,      /* radix sort of the keys by tile */
    TDGS_STAGE_TILE_RANGES = 6,
    TDGS_STAGE_BLEND = 7,          /* forward per-tile blending */
    TDGS_STAGE_BACKWARD_BLEND = 8,
    TDGS_STAGE_BACKWARD_PROJECT = 9,
    TDGS_STAGE_ADAM = 10,
    TDGS_STAGE_ADC = 11,
    TDGS_STAGE_LOSS = 12,
    TDGS_STAGE_COUNT = 13
};

/* ---- context, errors, device memory plumbing --------------------------------------- */
int tdgs_abi_version(void);
const char* tdgs_last_error(void);
/* Both work on the context's device and leave the caller's current device unchanged;
 * tdgs_ctx_destroy first waits for that device's work to finish. */
int tdgs_ctx_create(int device, tdgs_ctx** ctx_out);
int tdgs_ctx_destroy(tdgs_ctx* ctx);
int tdgs_malloc(void** ptr_out, size_t bytes);
int tdgs_free(void* ptr);
int tdgs_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int tdgs_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int tdgs_memset(void* dst, int value, size_t bytes, void* stream);
int tdgs_stream_synchronize(void* stream);

/* Streams, events and pinned host memory, so that a caller without a GPU runtime of its own
 * can order work as training_step! does with CUDA.jl's task-local stream (training.jl:173-244)
 * and overlap the ground-truth upload (the copyto! of training.jl:196-201) with kernels: a copy
 * stream uploads from pinned host memory, an event records the copy, the compute stream waits
 * on it. Streams are created at the default priority. The reference's CUB call has no stream
 * argument (cub_sort_pairs_wrapper.cu:37-42); every call here takes one. */
int tdgs_stream_create(void** stream_out);
int tdgs_stream_destroy(void* stream);
int tdgs_event_create(void** event_out);
int tdgs_event_destroy(void* event);
int tdgs_event_record(void* event, void* stream);
int tdgs_stream_wait_event(void* stream, void* event);
int tdgs_event_synchronize(void* event);
/* Milliseconds between two recorded events (both complete). */
int tdgs_event_elapsed_ms(void* start, void* stop, float* ms_out);
int tdgs_host_malloc(void** ptr_out, size_t bytes);   /* pinned (page-locked) host memory */
int tdgs_host_free(void* ptr);

/* Synchronises the stream and reports an inconsistency a kernel of an earlier call on this
 * context detected after that call returned (for example radix-sort counts that disagree
 * with the keys, which leaves sorted lists incomplete): TDGS_ERR_DEVICE with a message, and
 * the condition is cleared. Every call of the library that synchronises (tdgs_render,
 * tdgs_project, tdgs_fill_fgidx_to_gidx, tdgs_scan_counts, tdgs_adc_plan) checks it too. */
int tdgs_ctx_check(tdgs_ctx* ctx, void* stream);

/* Stage profiler (calling host thread): while enabled, library calls record a pair of HIP
 * events around each stage on the stream they run on (no extra synchronisation). At most
 * max_records stage executions are recorded. tdgs_profile_end waits for the recorded
 * events and returns, per stage, the summed milliseconds and the number of executions
 * (arrays of TDGS_STAGE_COUNT entries), then disables recording. */
int tdgs_profile_begin(int32_t max_records);
int tdgs_profile_end(double* ms_out, int64_t* executions_out);

/* ---- forward building blocks (each replaces one reference kernel) ------------------- */

/* The first half of render! (forward_core.jl:222-254): fill_keep_gaussians_kernel! (:326-355),
 * accumulate! + fill_fgidx_to_gidx_kernel! (:231-244, 371-386) and project_fgaussians_kernel!
 * (:411-517), fused. Writes buf->fgidx_to_gidx (1-based, ascending), and for every filtered
 * Gaussian with a non-empty bounding box its depth, f2d record, tile rectangle; counts gets
 * every filtered Gaussian's overlapped-tile count (0 for an empty box; such a Gaussian's f2d
 * record is written as zeros, its depth and rectangle are left unwritten as in the reference).
 * buf->keep is written when non-null.
 * Scratch: buf->temp (tdgs_render_temp_bytes). Synchronises to return N_f. */
int tdgs_project(tdgs_ctx* ctx, void* stream, const tdgs_gaussians* g, const tdgs_camera* cam,
                 const tdgs_tiling* tiling, const tdgs_render_options* opt,
                 tdgs_render_buffers* buf, int32_t* nb_fgaussians_out);

/* fill_keep_gaussians_kernel! (forward_core.jl:326-355): keep[g] = culling test. */
int tdgs_fill_keep(void* stream, const tdgs_gaussians* g, const tdgs_camera* cam,
                   const tdgs_render_options* opt, uint8_t* keep);

/* Scratch bytes for the device-wide scans used by the calls below (n elements). */
size_t tdgs_scan_temp_bytes(int64_t n);

/* accumulate!(+) + fill_fgidx_to_gidx_kernel! (forward_core.jl:231-244, 371-386):
 * keep_cs = inclusive scan of keep; fgidx_to_gidx[keep_cs[g]] = g for kept g (1-based).
 * keep_cs may be null. Synchronises to return the number of kept Gaussians. */
int tdgs_fill_fgidx_to_gidx(tdgs_ctx* ctx, void* stream, const uint8_t* keep, int32_t n,
                            int32_t* keep_cs, int32_t* fgidx_to_gidx, void* temp,
                            size_t temp_bytes, int32_t* nb_fgaussians_out);

/* accumulate!(+) of overlapped-tile counts (forward_core.jl:259-264): inclusive scan.
 * Synchronises to return the total (M); fails with TDGS_ERR_CAPACITY if M >= 2^31. */
int tdgs_scan_counts(tdgs_ctx* ctx, void* stream, const int32_t* counts, int32_t n,
                     int32_t* counts_cs, void* temp, size_t temp_bytes, int64_t* total_out);

/* No counterpart in the reference: tdgs_scan_counts for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). It
 * calls no allocating routine and needs no context or scratch argument: the per-tile partial
 * sums live in a fixed static device array of 64 KiB (per GPU, held until the process ends),
 * so n may be at most TDGS_SCAN_NOALLOC_MAX_ITEMS (TDGS_ERR_INVALID beyond). It does not
 * synchronise: the total is written to total_dev (device memory, one int64). Unlike
 * tdgs_scan_counts it cannot fail on a total of 2^31 or more (it does not look at the total
 * on the host): counts_cs[i] then holds the inclusive sum modulo 2^32 as an int32, so a caller
 * must check *total_dev < 2^31 before using counts_cs. Calls that overlap on one GPU
 * (different streams or host threads) share that array and race. */
#define TDGS_SCAN_NOALLOC_MAX_ITEMS 16777216
int tdgs_scan_counts_noalloc(void* stream, const int32_t* counts, int32_t n, int32_t* counts_cs,
                             int64_t* total_dev);

/* fill_df2dgs_codes_and_dfgidx_to_fgidx_kernel! (forward_core.jl:531-603). */
int tdgs_emit_keys(void* stream, int32_t nb_fgaussians, const float* depths,
                   const int32_t* tile_ranges, const int32_t* counts_cs,
                   const tdgs_tiling* tiling, int64_t* keys, int32_t* values);

/* determine_sort_pairs_temp_storage / sort_pairs (cub_sort_pairs_wrapper.cu:31-61):
 * stable LSD radix sort of (int64 key, int32 value) pairs on key bits [0, end_bit).
 * Same argument order as the CUB wrapper, plus a stream. */
size_t tdgs_sort_pairs_temp_bytes(int32_t n, int32_t end_bit);
int tdgs_sort_pairs(void* temp, size_t temp_bytes, const int64_t* keys_in, int64_t* keys_out,
                    const int32_t* values_in, int32_t* values_out, int32_t n, int32_t end_bit,
                    void* stream);

/* fill_tiles_end_sdfgidx_kernel! (forward_core.jl:676-734). */
int tdgs_tile_ranges(void* stream, int64_t nb_keys, const int64_t* sorted_keys,
                     int32_t nb_tiles, int32_t* tiles_end);

/* render_tiles_kernel! (forward_core.jl:756-993) on already sorted lists; render_void!
 * semantics are not applied here. */
int tdgs_render_tiles(void* stream, const tdgs_camera* cam, const tdgs_tiling* tiling,
                      const tdgs_render_options* opt, const tdgs_render_buffers* buf,
                      const tdgs_render_outputs* out);

/* Instrumentation: replays the blending of the last tdgs_render (same buffers, nb_keys keys)
 * without writing images and adds to evaluations_dev[0..2] (device) the number of (pixel,
 * sorted entry) evaluations made before each pixel's early exit, how many of them passed
 * the exponent cut (exponential evaluated), and how many contributed. No reference
 * counterpart: it sizes the FLOP count of the blending kernel for roofline reporting. */
int tdgs_blend_evaluations(void* stream, const tdgs_camera* cam, const tdgs_tiling* tiling,
                           const tdgs_render_options* opt, const tdgs_render_buffers* buf,
                           int64_t nb_keys, uint64_t* evaluations_dev);

/* ---- forward: render! --------------------------------------------------------------- */

/* Scratch for tdgs_render with the given capacities. */
size_t tdgs_render_temp_bytes(int32_t capacity, int64_t key_capacity, const tdgs_tiling* tiling);

/* render! GPU (forward_core.jl:196-314): cull, compact, project, duplicate, sort, ranges,
 * raster. Synchronises once to learn the filtered count and the key count. When the key
 * count exceeds buf->key_capacity it returns TDGS_ERR_CAPACITY with *nb_keys_out set and
 * leaves the outputs untouched; grow the key arrays (and temp) and call again.
 * With at most 65535 tiles the keys are not materialised: the tile lists (sorted_values,
 * tiles_end) are built by binning the depth-ordered Gaussians to coarse blocks of tiles (the
 * blocks' lists go through buf->keys and buf->values), with the same result as the sort, and
 * buf->sorted_keys is not written: tdgs_render_sorted_keys assembles it on request. */
int tdgs_render(tdgs_ctx* ctx, void* stream, const tdgs_gaussians* g, const tdgs_camera* cam,
                const tdgs_tiling* tiling, const tdgs_render_options* opt,
                tdgs_render_buffers* buf, const tdgs_render_outputs* out,
                int32_t* nb_fgaussians_out, int64_t* nb_keys_out);

/* Frame status of a render with TDGS_FLAG_DEVICE_COUNTS. */
enum { TDGS_FRAME_OK = 0, TDGS_FRAME_KEY_CAPACITY = 1, TDGS_FRAME_KEY_RANGE = 2 /* M >= 2^31 */ };

/* The counts of the last tdgs_render with TDGS_FLAG_DEVICE_COUNTS into these buffers:
 * counts_out[0..3] = nb_fgaussians, nb_keys, non-empty Gaussians, frame status. Synchronises
 * the stream. (They live in the first 32 bytes of buf->temp.) No reference counterpart. */
int tdgs_render_counts(void* stream, const tdgs_render_buffers* buf, int64_t* counts_out);

/* Frame monitor of the context's TDGS_FLAG_DEVICE_COUNTS renders, in pinned host memory that
 * the device updates at every such frame (when its blending starts): [frames, largest key
 * count, frames whose keys did not fit the key arrays, last key count, device error flags
 * pending at the last frame (non-zero: tdgs_ctx_check reports TDGS_ERR_DEVICE)]. Readable at
 * any time without synchronisation (the frames still in flight are not counted yet); lets a
 * training loop grow its key arrays ahead of need and re-run a frame whose keys did not fit.
 * No reference counterpart. */
int tdgs_ctx_frame_monitor(tdgs_ctx* ctx, const int64_t** monitor_out);

/* The sorted keys of the last tdgs_render with these buffers and tiling (nb_keys keys), as
 * the reference's RenderBuffers hold them after sort_keys_and_sdfgidx!
 * (forward_core.jl:641-659): (tile << 32) | depth bits, ascending, into buf->sorted_keys.
 * Nothing to do when the render sorted 64-bit keys (more than 65535 tiles). */
int tdgs_render_sorted_keys(void* stream, const tdgs_tiling* tiling, const tdgs_render_buffers* buf,
                            int64_t nb_keys);

/* ---- backward: backward! -------------------------------------------------------------- */

/* backward! (backward_core.jl:37-72): zero the 2D gradients, replay the tiles back to
 * front, then the backward projection to 3D gradients. Uses the buffers of the preceding
 * tdgs_render call with the same arguments; out must hold T and last. nb_fgaussians < 0
 * (here and in tdgs_backward_project / tdgs_backward_project_adam) takes the filtered count
 * of a TDGS_FLAG_DEVICE_COUNTS render from buf on the device (grads->capacity must then be at
 * least buf->capacity; the 2D gradients are zeroed over the whole capacity). */
int tdgs_backward(void* stream, tdgs_gradients* grads, const float* rgb_grad,
                  const tdgs_render_outputs* out, const tdgs_gaussians* g,
                  const tdgs_camera* cam, const tdgs_tiling* tiling,
                  const tdgs_render_options* opt, const tdgs_render_buffers* buf,
                  int32_t nb_fgaussians);

/* The two halves of tdgs_backward (backward_core.jl:96-293 and :309-452). The first
 * accumulates into grads->grads2d without zeroing it. */
int tdgs_backward_render_tiles(void* stream, tdgs_gradients* grads, const float* rgb_grad,
                               const tdgs_render_outputs* out, const tdgs_camera* cam,
                               const tdgs_tiling* tiling, const tdgs_render_options* opt,
                               const tdgs_render_buffers* buf);
int tdgs_backward_project(void* stream, tdgs_gradients* grads, const tdgs_gaussians* g,
                          const tdgs_camera* cam, const tdgs_render_options* opt,
                          const tdgs_render_buffers* buf, int32_t nb_fgaussians);

/* backward_project_fgaussians_kernel! (backward_core.jl:309-452) fused with update!
 * (optimizer.jl:964-1009, sh_degree = opt->sh_degree): the 3D gradients of each filtered
 * Gaussian are applied to its parameters and moments at once instead of being written to
 * grads (whose 3D arrays are left untouched; grads2d is read). The result equals
 * tdgs_backward_project followed by tdgs_adam_step bit for bit; increments st->update_count.
 * No reference counterpart as one call: for trainers that run no density control between the
 * backward pass and the optimiser step (training.jl:221-236 does so every adc_interval
 * iterations; call the two functions separately then). */
int tdgs_backward_project_adam(void* stream, const tdgs_gradients* grads, tdgs_gaussians* g,
                               tdgs_adam_state* st, const tdgs_camera* cam,
                               const tdgs_render_options* opt, const tdgs_render_buffers* buf,
                               int32_t nb_fgaussians);

/* tdgs_backward_project_adam with update_adc_stats_kernel! (training.jl:472-497) folded in:
 * adc's accumulated 2D mean-gradient norms and contribution counts are updated from grads2d
 * as tdgs_adc_stats / tdgs_adc_stats_frame (width and height from cam) would, bit for bit,
 * in the same launch. No reference counterpart as one call: for trainers whose step between
 * the backward pass and update! is only the statistics (training.jl:221-236, whose
 * maybe_densify_and_prune! runs the statistics kernel at :313-318 and density control only
 * every adc_interval iterations). adc->capacity must be at least g->n. */
int tdgs_backward_project_adam_adc(void* stream, const tdgs_gradients* grads, tdgs_gaussians* g,
                                   tdgs_adam_state* st, const tdgs_camera* cam,
                                   const tdgs_render_options* opt, const tdgs_render_buffers* buf,
                                   int32_t nb_fgaussians, tdgs_adc_buffers* adc);

/* ---- optimiser: update! -------------------------------------------------------------- */

/* update!(opt, fgradients, Val(sh_degree)) (optimizer.jl:964-1009): sparse Adam over the
 * filtered Gaussians (fgidx_to_gidx[f] <= 0 is skipped), all components in one launch;
 * increments st->update_count. */
int tdgs_adam_step(void* stream, tdgs_gaussians* g, tdgs_adam_state* st,
                   const tdgs_gradients* grads, const int32_t* fgidx_to_gidx,
                   int32_t nb_fgaussians, int32_t sh_degree);

/* ---- adaptive density control -------------------------------------------------------- */

/* update_adc_stats_kernel! (training.jl:472-497). */
int tdgs_adc_stats(void* stream, tdgs_adc_buffers* adc, const tdgs_gradients* grads,
                   const int32_t* fgidx_to_gidx, int32_t nb_fgaussians, int32_t width,
                   int32_t height);

/* tdgs_adc_stats for a render with TDGS_FLAG_DEVICE_COUNTS: fgidx_to_gidx from the render
 * buffers and the filtered count from the frame counts on the device (nothing for a frame
 * whose keys did not fit). */
int tdgs_adc_stats_frame(void* stream, tdgs_adc_buffers* adc, const tdgs_gradients* grads,
                         const tdgs_render_buffers* buf, int32_t width, int32_t height);

/* Masks, counts, scan and ngidx_to_gidx (training.jl:325-397). Thresholds are in feature
 * space: prune if logit < prune_logit or (use_max_scale and max log-scale > log_max_scale);
 * densify if not pruned and average grad >= grad_threshold; clone if densify and max
 * log-scale <= log_size_threshold. Synchronises to return the new Gaussian count. Fails
 * with TDGS_ERR_CAPACITY (count in *n_new_out) if adc->new_capacity is too small. */
int tdgs_adc_plan(tdgs_ctx* ctx, void* stream, tdgs_adc_buffers* adc, const tdgs_gaussians* g,
                  float prune_logit, int32_t use_max_scale, float log_max_scale,
                  float grad_threshold, float log_size_threshold, int32_t* n_new_out);

/* adaptive_density_control! for parameters (gaussians.jl:1526-1694) and Adam moments
 * (optimizer.jl:1304-1378): fills dst and dst_m (n_new Gaussians, every slot written: moments
 * copied for carried-over Gaussians and first clones, zero for second clones and splits).
 * Split means use a counter-based normal generator keyed by (seed, old index, draw). */
int tdgs_adc_apply(void* stream, const tdgs_adc_buffers* adc, const tdgs_gaussians* src,
                   tdgs_gaussians* dst, const tdgs_adam_state* src_m, tdgs_adam_state* dst_m,
                   float log_split_factor, uint64_t seed);

/* adjust_fgidx_to_gidx_adc_kernel! (training.jl:514-541). */
int tdgs_adc_remap_fgidx(void* stream, const tdgs_adc_buffers* adc, int32_t* fgidx_to_gidx,
                         int32_t nb_fgaussians);

/* Reset the ADC statistics (set_nb_gaussians!, training_structs.jl). */
int tdgs_adc_reset_stats(void* stream, tdgs_adc_buffers* adc, int32_t n);

/* ---- training helpers ------------------------------------------------------------------ */

/* L1 part of the loss and its gradient (training.jl:206-215):
 * grad = (rendered > gt ? w : -w) + dssim_weight * dssim_grad (dssim_grad may be null),
 * w = l1_weight / count; a tie (rendered == gt) takes -w as the reference's ifelse does, and
 * the product is rounded before the sum (no fused multiply-add), as the reference's broadcast.
 * Adds sum |rendered - gt| to *l1_sum_dev (device double, may be null; the caller zeroes it).
 * The trainer uses it when the D-SSIM weight is 0. */
int tdgs_l1_loss_grad(void* stream, const float* rendered, const float* gt, int64_t count,
                      float l1_weight, float dssim_weight, const float* dssim_grad,
                      float* grad_out, double* l1_sum_dev);

/* Training loss of training_step! (training.jl:196-217) fused with its gradient:
 * L = (1 - w) mean|K - I| + w DSSIM(K, I), DSSIM = 1 - SSIM (docs/src/math.md:125-126),
 * SSIM with an 11 x 11 Gaussian window (sigma 1.5), C1 = 0.01^2, C2 = 0.03^2, zero padding,
 * averaged over pixels and channels (replaces FastCUDASSIM.dssim_with_gradient!).
 * Images are 3 x h x w. grad_out = dL/dK. sums_dev (device, 2 doubles, zeroed by the
 * caller) receives sum|K - I| and the sum of the SSIM map: L = (1-w) s0/N + w (1 - s1/N)
 * with N = 3 w h. temp holds tdgs_loss_temp_bytes(width, height) bytes. */
size_t tdgs_loss_temp_bytes(int32_t width, int32_t height);
int tdgs_loss_grad(void* stream, const float* rendered, const float* gt, int32_t width,
                   int32_t height, float dssim_weight, float* grad_out, double* sums_dev,
                   void* temp, size_t temp_bytes);

/* reset_opacities! (gaussians.jl:1093-1101) + zero opacity moments (optimizer.jl:754-756). */
int tdgs_opacity_reset(void* stream, tdgs_gaussians* g, float max_logit,
                       float* opacity_moments);

/* resize_array for a spherical-harmonics degree change (misc.jl:100-125, used by
 * set_sh_degree! in gaussians.jl:1070-1080 and optimizer.jl:737-747): copies the first
 * min(h_src, h_dst) coefficients of every (channel, element) from src (interleave x h_src x
 * 3 x n) to dst (interleave x h_dst x 3 x n) and zero-fills the rest. interleave is 1 for
 * coefficients and gradients, 2 for Adam moments. */
int tdgs_sh_resize(void* stream, const float* src, int32_t h_src, float* dst, int32_t h_dst,
                   int64_t n, int32_t interleave);

/* ---- viewer output ---------------------------------------------------------------------- */

enum { TDGS_IMAGE_RGB = 0, TDGS_IMAGE_TRANSMITTANCE = 1, TDGS_IMAGE_DEPTH = 2 };

/* One rendered image to the UInt8 3 x width x height (channel fastest, then x, then y)
 * buffer an OpenGL RGB texture takes, as convert_rgb_to_gl_img_kernel!,
 * convert_transmittance_to_gl_img_kernel! and convert_depth_to_gl_img_kernel!
 * (gui.jl:958-1067) write it into the viewer's pixel buffer:
 *   RGB (3 x h x w, values >= 0):  v <= 1 ? round(v * 255) : 255 per channel;
 *   transmittance (h x w, [0, 1]): round(T * 255) in all three channels;
 *   depth (h x w):                 round((1 - clamp01((d - min_depth) / (max_depth -
 *                                   min_depth))) * 255) in all three channels
 * (round = to nearest, ties to even; products in float). dst holds 3 * width * height bytes;
 * min_depth < max_depth is required for TDGS_IMAGE_DEPTH. */
int tdgs_image_to_rgb8(void* stream, int32_t kind, const float* src, int32_t width, int32_t height,
                       float min_depth, float max_depth, uint8_t* dst);

#ifdef __cplusplus
}
#endif

#endif /* TDGS_H */
