/*
 * vsplat.h -- C ABI of the MI355X (gfx950) Gaussian-splat rasterizer.
 *
 * This is the drop-in boundary for the reference's render / sort / scan call
 * surface (voyager-so/vauss).  Every entry point names the reference
 * interface it replaces.  Paths are relative to the reference repository.
 *
 * Conventions
 *  - All array arguments are device pointers (HIP global memory) unless the
 *    comment says "host".  Inputs are contiguous, row-major, fp32/u32.
 *  - Outputs are caller-owned; intermediate state is library-owned and lives
 *    in a `vs_fwd_state` until vs_fwd_state_free().
 *  - Work is enqueued on the context's HIP stream.  Calls that must learn a
 *    device-side count before sizing a buffer (the forward render after
 *    projection, unless lagged counts apply) synchronise that stream once;
 *    everything else is stream-ordered and returns without waiting.
 *  - No C++ exception crosses this boundary.  Every call returns a
 *    vs_status; vs_last_error() gives a human-readable message for the
 *    calling thread.
 *  - One context per host thread.  Contexts are independent.
 */
#ifndef VSPLAT_H
#define VSPLAT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum vs_status {
    VS_OK = 0,
    VS_ERR_INVALID = 1,      /* bad argument (shape, size, null pointer, mode) */
    VS_ERR_HIP = 2,          /* a HIP runtime call failed */
    VS_ERR_OOM = 3,          /* device allocation failed */
    VS_ERR_UNSUPPORTED = 4,  /* a mode the reference has that is not built here */
    VS_ERR_CAPACITY = 5,     /* intersection count exceeds the u32 limit or the cap */
    VS_ERR_NONFINITE = 6,    /* validation found NaN/Inf in an input */
} vs_status;

typedef struct vs_ctx vs_ctx;
typedef struct vs_fwd_state vs_fwd_state;

/* Camera models: crates/splat-train-render/src/kernels/camera_model/mod.rs:30-37.
 * Distortion parameters: KB4 k1..k4 in kb4[]; RT8 (OpenCV rational +
 * tangential) k1..k6, p1, p2 in dist[0..7]; thin-prism fisheye (COLMAP
 * THIN_PRISM_FISHEYE) its KB4 part in kb4[] and p1, p2, sx1, sy1 in
 * dist[0..3]. */
typedef enum vs_camera_model {
    VS_CAMERA_PINHOLE = 0, VS_CAMERA_KB4 = 1, VS_CAMERA_RT8 = 2, VS_CAMERA_TPF = 3
} vs_camera_model;

/* Device-side projection uniforms, the fields of ProjectUniforms
 * (crates/splat-train-render/src/kernels/types.rs:53-82) other than sizes.
 * Built on the host by vs_camera_uniforms() exactly as render.rs:478-503
 * builds them, or filled by the caller. */
typedef struct vs_camera {
    int32_t model;                  /* vs_camera_model */
    float fx, fy, cx, cy;           /* PinholeParams */
    float kb4[4];                   /* KannalaBrandt4Params k1..k4 */
    float viewmat[12];              /* world->camera 3x4, column-major (col0,col1,col2,translation) */
    float cam_pos[3];               /* view-direction origin for SH */
    float half_max_render_fov;      /* fisheye angular cull */
    float lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y, lim_r; /* JacobianClampLimits */
    float dist[8];                  /* RT8 / thin-prism parameters (see vs_camera_model) */
} vs_camera;

/* Host camera description, crates/splat-train-render/src/camera.rs:11-23. */
typedef struct vs_pose {
    double fov_x, fov_y;            /* radians */
    float center_uv[2];             /* principal point as a fraction of the image */
    float position[3];              /* camera centre, world */
    float rotation[4];              /* camera-to-world rotation quaternion, (x, y, z, w) */
    int32_t model;                  /* vs_camera_model */
    float kb4[4];
    float dist[8];                  /* RT8 / thin-prism parameters */
} vs_pose;

/* Element type of the SH coefficients (render.rs:683-687: f32 or f16; the
 * trainer's SH step keeps them in f16).  Gradients are always f32. */
typedef enum vs_sh_dtype { VS_SH_F32 = 0, VS_SH_F16 = 1 } vs_sh_dtype;

/* Parameters of N splats, crates/splat-train-render/src/gaussian_splats.rs:127-153. */
typedef struct vs_splats {
    const float* transforms;        /* [N,10]: mean xyz, quat w x y z, log-scale xyz */
    const void* sh_coeffs;          /* [N,(d+1)^2,3] f32, or IEEE binary16 when sh_dtype = VS_SH_F16 */
    const float* raw_opacities;     /* [N] logits */
    uint32_t num_splats;
    uint32_t sh_degree;             /* 0..4 */
    float log_scale_offset;         /* added to every log-scale (render.rs:325) */
    uint32_t sh_dtype;              /* vs_sh_dtype */
    const float* min_scale;         /* [N] scale floor (the Mip-Splatting 3D filter,
                                       kernels/helpers.rs:497-553) or NULL for none
                                       (render's min_scale / has_min_scale) */
    const float* decoder;           /* [816] compact neural appearance (kernels/neural.rs,
                                       SplatOps::render_neural, render.rs:352-397) or NULL
                                       for SH colour.  With a decoder, sh_coeffs holds
                                       [N,4,3] rows (base colour as a DC coefficient, an
                                       8-value latent, a pad) and sh_degree is the
                                       decoder's direction band, 0..3. */
} vs_splats;

/* RasterPass, crates/splat-train-render/src/gaussian_splats.rs:32-107.
 * Every pass but FORWARD writes a float image and keeps backward state.
 * Training passes (BACKWARD, BACKWARD_DENSE, EXPOSURE, BACKWARD_FUSED_UPDATE)
 * use lagged counts when the context enables them (vs_ctx_set_lagged_counts).
 * BACKWARD_DENSE and EXPOSURE carry the reference's `slot` (RasterPass::
 * BackwardDense { slot }, Exposure { slot }) in bits 8..15 of the value,
 * written VS_PASS_SLOT(pass, slot): a render settles the lagged counts of the
 * previous render at its (width, height, slot), so a step's several renders
 * at one size keep their capacity hints and pending counts apart
 * (render.rs:741-747).  Other passes take slot 0. */
typedef enum vs_pass {
    VS_PASS_FORWARD = 0,            /* packed RGBA8 image [H,W] u32, no backward state */
    VS_PASS_BACKWARD = 1,           /* float RGBA [H,W,4] + backward state (training) */
    VS_PASS_FLOAT = 2,              /* float RGBA [H,W,4], exact counts, not differentiated */
    VS_PASS_BACKWARD_SMOOTH_CUTOFF = 3, /* Backward with the C^1 alpha cutoff (gradient checks) */
    VS_PASS_GEOMETRY = 4,           /* float [H,W,12]: RGBA, sum(w z), median z, normal, distortion, median id */
    VS_PASS_BACKWARD_DENSE = 5,     /* Backward whose dense gradients several renders of a step sum (training, slot) */
    VS_PASS_EXPOSURE = 6,           /* a training-time forward with no gradient, e.g. exposure sub-renders (slot) */
    VS_PASS_BACKWARD_FUSED_UPDATE = 7, /* Backward whose vs_render_backward stops at v_combined for vs_project_update */
    VS_PASS_GEOMETRY_TRAIN_DEPTH = 8,  /* GEOMETRY with the training median (T > 1/2) for surfels too */
    VS_PASS_SLOT_MASK = 0xFF00      /* bits of the count slot (BACKWARD_DENSE, EXPOSURE) */
} vs_pass;
#define VS_PASS_SLOT(pass, slot) ((vs_pass)((uint32_t)(pass) | (((uint32_t)(slot) & 0xFFu) << 8)))

/* SplatRenderMode, gaussian_splats.rs:19-26: DEFAULT (+0.3 2-D blur), MIP
 * (+0.1 blur with opacity compensation, kernels/helpers.rs:227-245) and
 * SURFEL (2DGS: each splat is the disk of its first two scaled axes, covered
 * by the pixel ray's intersection with its plane and a screen-space low-pass,
 * kernels/helpers.rs:316-423, kernels/rasterize.rs:267-301).  Surfels are
 * pinhole-only (a lens camera renders as the pinhole with its focal length)
 * and take SH colour; every pass but FORWARD writes the 12 geometry channels
 * (RGBA, sum(w z), median z, normal, distortion moments, median id; the
 * median by the surface criterion except in training passes and
 * VS_PASS_GEOMETRY_TRAIN_DEPTH, gaussian_splats.rs:100-106), and the
 * backward's v_combined rows have 17 components [M rows (9), normal (3),
 * rgb (3), alpha, refine]. */
typedef enum vs_render_mode { VS_MODE_DEFAULT = 0, VS_MODE_MIP = 1, VS_MODE_SURFEL = 2 } vs_render_mode;

/* Forward outputs (RenderAux, crates/splat-train-render/src/render_aux.rs:74-100).
 * Device arrays may be NULL when not wanted. */
typedef struct vs_fwd_out {
    void* out_img;                  /* [H,W,C] f32 (C = 4 or 12) or [H,W] u32 packed (FORWARD) */
    float* visible;                 /* [N] 1 if the splat was blended into any pixel (bwd passes) */
    float* max_radius;              /* [N] max(ex/W, ey/H), 0 if culled */
    float* opacities;               /* [N] sigmoid(raw) for splats past the first culls, else 0 */
    uint32_t* tile_offsets;         /* [ty,tx,2] start/end per tile (end shrunk on bwd passes) */
    uint32_t num_visible;           /* host: splats that survived culling */
    uint32_t num_intersections;     /* host: (tile, splat) pairs */
} vs_fwd_out;

/* Dense gradients per global splat (the reference's compact rows gathered
 * through compact_from_global, bwd/burn_glue.rs:355-430). NULL skips one. */
typedef struct vs_grads {
    float* v_transforms;            /* [N,10] d/d(mean, quat wxyz, log-scale) */
    float* v_sh_coeffs;             /* [N,(d+1)^2,3], or the neural rows [N,4,3] */
    float* v_raw_opacities;         /* [N] */
    float* v_refine_weight;         /* [N] screen-space refine weight, clamped [0,1e32] */
    float* v_combined;              /* [N,10] raster gradient rows (xy, conic, rgb, alpha, refine); surfels [N,17] */
    float* v_decoder;               /* [816] neural appearance: decoder gradient summed over splats */
    float* v_coeffs_sq;             /* [N] neural appearance: mean square of each row's gradient */
} vs_grads;

/* ---- context --------------------------------------------------------------- */

/* Create a context on `device` enqueueing on `hip_stream` (NULL: the null
 * stream).  No reference counterpart: the reference's CubeCL client owns the
 * device queue (crates/splat-train-cube/src/host.rs:12-38). */
vs_status vs_ctx_create(int device, void* hip_stream, vs_ctx** out);
void vs_ctx_destroy(vs_ctx* ctx);
/* Switch the stream later work is enqueued on. */
vs_status vs_ctx_set_stream(vs_ctx* ctx, void* hip_stream);
/* Message of the last failing call on this host thread. */
const char* vs_last_error(void);
/* Library version string. */
const char* vs_version(void);

/* Per-stage HIP event timing (replaces the reference's tracing spans,
 * render.rs:520-886).  `stages` is a bitmask of the stages to bracket with
 * events on the context's stream (bit i = field i of vs_stage_times, in
 * order; VS_TIME_ALL for every stage, 0 to stop); vs_ctx_stage_times()
 * synchronises the stream once and returns the milliseconds summed over all
 * calls since the previous query.  Each bracket costs a few microseconds of
 * stream time, so timing only the stage of interest keeps the rest of a
 * render's timeline as it runs untimed. */
typedef struct vs_stage_times {
    float project_ms, emit_ms, sort_ms, ranges_ms, raster_fwd_ms;
    float raster_bwd_ms, project_bwd_ms, other_ms;
} vs_stage_times;
enum {
    VS_TIME_PROJECT = 1u << 0, VS_TIME_EMIT = 1u << 1, VS_TIME_SORT = 1u << 2, VS_TIME_RANGES = 1u << 3,
    VS_TIME_RASTER_FWD = 1u << 4, VS_TIME_RASTER_BWD = 1u << 5, VS_TIME_PROJECT_BWD = 1u << 6,
    VS_TIME_OTHER = 1u << 7, VS_TIME_ALL = 0xFFu
};
vs_status vs_ctx_enable_timing(vs_ctx* ctx, uint32_t stages);
vs_status vs_ctx_stage_times(vs_ctx* ctx, vs_stage_times* out);

/* Lagged counts for training renders (render.rs:38-304, 741-768, 887-915).
 * With `enable` set, a training-pass forward (VS_PASS_BACKWARD,
 * _BACKWARD_DENSE, _EXPOSURE, _BACKWARD_FUSED_UPDATE) at an image size and
 * count slot this context has already rendered sizes its intersection arena
 * from a capacity hint kept per (width, height, slot) and runs every stage
 * after projection on device-resident counts: it never waits for the GPU.
 * Its vs_fwd_out counts are then the previous lagged render's at that key
 * (0, 0 for the first), and its own are read by the next one.  A render needing more intersections than the hint
 * keeps the first `capacity` of the depth-ordered list (the farthest splats'
 * tiles are dropped), logs to stderr and grows the hint.  The hint follows
 * the reference's policy: 200-render windows sized to the p99 intersections
 * per splat with 25% headroom, never below the window's largest render + 5%,
 * 1.5x growth before the first full window.  Other passes, and every render
 * with `enable` clear (the default), stay exact and refine the hint.  The
 * reference enables this for every training render; it is opt-in here. */
vs_status vs_ctx_set_lagged_counts(vs_ctx* ctx, int enable);
/* Wait for every pending lagged render's counts, fold them into the hints
 * and return the number of lagged renders settled so far and how many of
 * them overflowed their capacity (either pointer may be NULL). */
vs_status vs_ctx_settle_lagged_counts(vs_ctx* ctx, uint64_t* renders, uint64_t* overflows);

/* Bound on a one-sweep radix pass's wait for its predecessors' digit counts
 * (the decoupled look-back), and on the render's slot scan's wait for its
 * predecessors' sums: after `polls` polls of an unpublished predecessor the
 * pass gives up, its output is wrong, and the call that ran it returns
 * VS_ERR_HIP (vs_radix_argsort_*, exact renders; a lagged render's are
 * reported by the next lagged render at its size or by
 * vs_ctx_settle_lagged_counts).  0xFFFFFFFF restores the default (2^18).  The
 * reference's sort has no bounded wait (crates/splat-train-sort/src/lib.rs);
 * a small limit lets tests drive the give-up path with every kernel exiting. */
vs_status vs_ctx_set_sort_spin_limit(vs_ctx* ctx, uint32_t polls);

/* Validation readbacks (crates/splat-train-render/src/validation.rs:1-140;
 * Splats::validate_values / bwd_validate, gaussian_splats.rs:417-509).  With
 * `enable` set, vs_render_forward first scans the splat parameters (means,
 * rotations, log-scales, SH coefficients, raw opacities, the floor and the
 * decoder when given) and vs_render_backward the gradients it wrote; a NaN or
 * Inf fails the call with VS_ERR_NONFINITE naming the tensor and its first
 * bad element (the reference panics), values outside the reference's ranges
 * (log-scales [-10, 10], SH [-5, 5], raw opacity [-20, 20]) are logged to
 * stderr.  Each scan synchronises the stream.  Off by default, as in the
 * reference's release builds; without it, non-finite splats are culled. */
vs_status vs_ctx_set_validation(vs_ctx* ctx, int enable);

/* Depth cutoff for renders whose tiles are listed far more splats than
 * their pixels can blend (no reference counterpart: the reference lists and
 * sorts every intersection).  From the opacity each splat lays over the
 * whole of a tile (its core at half its opacity), a tile's list
 * stops at the depth bin (64 bins over the frame's depth range) by which
 * every pixel of the tile has provably reached the raster's stopping
 * transmittance; the splats it drops are never evaluated there, so images,
 * consumed ranges and gradients are those of the full list.  Gaussian modes
 * only.  VS_CUTOFF_OFF (the default) lists every intersection, as the
 * reference does; ON applies the cutoff to every gaussian render, AUTO when a
 * render lists at least 2048 intersections per tile on average (the exact
 * count, or a lagged render's capacity).  Opt in knowing what it changes:
 * outputs that index the intersection list then index the shortened one.
 * vs_fwd_out.tile_offsets (RenderAux.tile_offsets, render_aux.rs:84,100)
 * holds for each tile a range of the same length over the same pairs as the
 * full list's shrunk range, but starting at the tile's offset in the
 * shortened list, and the geometry render's median-id channel is an index
 * into that list (the same position within its tile's list).
 * num_intersections still reports every intersection; the state view gives
 * the listed ones. */
typedef enum vs_cutoff_mode { VS_CUTOFF_AUTO = 0, VS_CUTOFF_OFF = 1, VS_CUTOFF_ON = 2 } vs_cutoff_mode;
vs_status vs_ctx_set_depth_cutoff(vs_ctx* ctx, vs_cutoff_mode mode);

/* Fill every buffer the library allocates for this context with the f32
 * pattern of -12345.0 before first use, as the reference's test builds
 * initialise fresh tensors (crates/splat-train-cube/src/host.rs:23-36), so a
 * kernel reading a slot it never wrote shows up as a wrong result.  A debug
 * aid; also switched on for new contexts by the environment variable
 * VSPLAT_POISON=1. */
vs_status vs_ctx_set_poison(vs_ctx* ctx, int enable);

/* ---- camera host math --------------------------------------------------------- */

/* camera.rs:99-116 fov_to_focal / :118-134 focal_to_fov (host, f64).
 * `params` holds 12 floats: kb4 k1..k4 then dist[8] (NULL for pinhole). */
double vs_fov_to_focal(double fov, uint32_t pixels, int32_t model, const float* params);
double vs_focal_to_fov(double focal, uint32_t pixels, int32_t model, const float* params);
/* camera.rs:166-172 max_render_theta (the KB4 / thin-prism fold angle, pi otherwise). */
double vs_max_render_theta(int32_t model, const float* params);
/* render.rs:478-503 + camera.rs:55-96,305-374: uniforms of a pose at W x H (host). */
vs_status vs_camera_uniforms(const vs_pose* pose, uint32_t img_w, uint32_t img_h, vs_camera* out);

/* ---- render ------------------------------------------------------------------- */

/* SplatOps::render (crates/splat-train-render/src/lib.rs:53-90; implementation
 * render.rs:401-979).  Writes the image and aux outputs; for every pass but
 * FORWARD also returns the state the backward needs in *state (free with
 * vs_fwd_state_free).  `background` is host memory. */
vs_status vs_render_forward(vs_ctx* ctx, const vs_camera* cam, const vs_splats* splats,
                            uint32_t img_w, uint32_t img_h, const float background[3],
                            vs_pass pass, vs_render_mode mode,
                            vs_fwd_out* out, vs_fwd_state** state);

/* vs_render_forward followed by vs_l1_cotangent_packed of its image, with the
 * cotangent written by the raster pass itself (no second read of the image;
 * one launch fewer): for a pass with a float RGBA image (every pass but
 * VS_PASS_FORWARD and the geometry passes; not surfels).  gt_packed
 * [H,W] RGBA8 as the reference's loss reads it (crates/splat-train-loss/src/
 * lib.rs:93,1042-1044), the circle mask as vs_l1_cotangent's, v_out [H,W,4]
 * f32, 16-byte aligned: bit for bit what vs_l1_cotangent_packed writes for
 * the same image.  No counterpart in the reference, whose loss is a separate
 * pass (lib.rs:786-811). */
vs_status vs_render_forward_l1(vs_ctx* ctx, const vs_camera* cam, const vs_splats* splats,
                               uint32_t img_w, uint32_t img_h, const float background[3],
                               vs_pass pass, vs_render_mode mode,
                               const uint32_t* gt_packed, float mask_cx, float mask_cy, float mask_radius,
                               float* v_out, vs_fwd_out* out, vs_fwd_state** state);

/* SplatBwdOps::rasterize_bwd + project_bwd (bwd/burn_glue.rs:70-111;
 * bwd/render_bwd.rs:27-155 and 295-447).  `out_img` is the image the
 * forward wrote (f32, C channels), `v_out` its cotangent [H,W,C].  The
 * splat parameters must be the ones the forward saw; splats->log_scale_offset
 * is not read: the forward's is used, as the reference's ProjectUniforms
 * carry it from the forward to project_bwd.  When every dense
 * output of `grads` is NULL the call stops at the raster gradients
 * (grads->v_combined), as the reference's BackwardFusedUpdate pass does
 * (gaussian_splats.rs:95); vs_project_update then consumes them. */
vs_status vs_render_backward(vs_ctx* ctx, vs_fwd_state* state, const vs_splats* splats,
                             const float* out_img, const float* v_out, vs_grads* grads);

void vs_fwd_state_free(vs_fwd_state* state);

/* Read-only view of the forward's intermediate buffers (device pointers owned
 * by the state), for parity checks of each stage against the reference
 * semantics.  Projected rows are indexed by global splat id.  The render does
 * not keep the sorted tile ids (its tile sort derives the ranges instead):
 * the first view of a state rebuilds them from the ranges on the context's
 * stream and waits for that. */
#define VS_PROJ_ROW_FLOATS 16u   /* stride of the projected rows, in floats */
typedef struct vs_state_view {
    uint32_t num_splats, num_visible, num_intersections, num_tiles, tile_bw, tile_bh;
    const uint32_t* isect_tiles;    /* [I] sorted tile ids (T = sentinel, sorts last) */
    const uint32_t* isect_gids;     /* [I] sorted global splat ids */
    const uint32_t* intersect_counts; /* [N] */
    const uint32_t* depth_bits;     /* [N] raw f32 bits of view z (the depth key) */
    const uint32_t* compact_from_global; /* [N] g + 1 for splats past every cull, 0 if culled
                                       (RenderOutput state, render_aux.rs:36-41: the rows of
                                       vs_project_update's color_dir) */
    /* The projected rows: N rows of VS_PROJ_ROW_FLOATS floats (64 bytes), valid
       for visible splats; the three pointers below point into row 0. */
    const float* proj_xy_conic;     /* x, y, c00, c01 (floats 0-3 of each row) */
    const float* proj_c11_opac_rg;  /* c11, opacity, r, g (floats 4-7) */
    const float* proj_b;            /* b (float 8; float 9 holds logf(255 opacity)) */
    const float* proj_aux;          /* [N,4] z, nx, ny, nz (GEOMETRY) or NULL */
    const uint32_t* tile_ranges;    /* [T,2] before the forward shrank the ends */
    const float* proj_surf;         /* [N,16] surfels: M rows (9), low-pass centre (2), normal (3),
                                       the raster's footprint bound on sigma, 1 pad;
                                       else NULL */
    uint32_t listed_intersections;  /* length of isect_tiles / isect_gids: num_intersections, or
                                       under the depth cutoff the pairs each tile's list keeps */
    uint32_t depth_cutoff;          /* 1: every tile's list is the front of its full list */
    const uint32_t* listed_counts;  /* [N] pairs of each splat in the lists (intersect_counts
                                       without the depth cutoff) */
} vs_state_view;
vs_status vs_fwd_state_view(const vs_fwd_state* state, vs_state_view* out);

/* ---- fused projection backward + Adam ------------------------------------------- */

/* FusedAdam (bwd/project_update.rs:232-250): the Adam step shared by the
 * transforms and raw opacities. */
typedef struct vs_adam_step {
    float beta1, beta2;             /* moment decays */
    float inv1, inv2;               /* 1 / (1 - beta1^t), 1 / (1 - beta2^t) */
    float epsilon;                  /* Adam epsilon, also the moment codec's scale */
    float lr_opac;                  /* raw-opacity learning rate */
    float opac_reg;                 /* opacity regulariser gradient weight (w / N), 0 = off */
    uint32_t round_seed;            /* stochastic-rounding stream (the step count) */
} vs_adam_step;

/* ProjectUpdateOut minus the stepped tensors (bwd/project_update.rs:25-40).
 * NULL skips an output. */
typedef struct vs_update_out {
    float* color_dir;               /* [N+1,6]: row compact_from_global[g] = colour gradient, view
                                       direction; row 0, rows without gradient and the rows g + 1
                                       of culled splats zero */
    float* v_refine_weight;         /* [N] clamped to [0,1e32], 0 for culled splats */
    float* coeffs_grad_sq;          /* [N] mean square of the SH gradient row, from its DC entries */
} vs_update_out;

/* SplatBwdOps::pose_bwd (bwd/render_bwd.rs:224-288, kernel
 * bwd/kernels/pose_backwards.rs:88-191): the camera gradient.  The camera is
 * perturbed by x_c' = (I + A) x_c + b after the world-to-camera transform, A
 * pivoting on the camera centre (which b moves by -M^-1 b, all the SH view
 * direction sees); v_pose [12] (device) receives d loss / d [A row-major,
 * b], summed over the splats with position, conic or colour gradients in
 * `v_combined` [N,10] (vs_render_backward's raster rows for `state`).  A
 * rigid twist [rho, w] is A = [w]x, b = rho.  `splats` must be the forward's
 * (same floor); the log-scale offset is the forward's, as in
 * vs_render_backward.  Stream-ordered; the sum is deterministic. */
vs_status vs_pose_backward(vs_ctx* ctx, vs_fwd_state* state, const vs_splats* splats, const float* v_combined,
                           float* v_pose);

/* ProjectUpdateOps::project_update (bwd/project_update.rs:80-220; kernel
 * bwd/kernels/project_update.rs:40-178): the projection VJP of a backward
 * pass's raster gradients `v_combined` [N,10] fused with one Adam step of
 * `transforms` [N,10] and `raw_opacities` [N], both updated in place, whose
 * moments are packed one u32 per value in `w_t` [N,10] and `w_o` [N]
 * (geo_moments.rs codec; zero words are reset moments).  `lr_scale` is the
 * per-column transforms learning rate [10] (device).  The parameters must be
 * the pre-step values the forward of `state` saw (`sh_coeffs` in the
 * forward's dtype; the render mode and the forward's `min_scale` array, which
 * must still hold the same floors, apply).  Every splat steps: culled ones decay their moments with a
 * zero gradient plus the opacity regulariser. */
vs_status vs_project_update(vs_ctx* ctx, vs_fwd_state* state, float* transforms, const void* sh_coeffs,
                            float* raw_opacities, const float* v_combined, uint32_t* w_t,
                            const float* lr_scale, uint32_t* w_o, const vs_adam_step* adam,
                            vs_update_out* out);

/* GeoMomentOps (bwd/geo_moments.rs:25-60, kernels geo_moments.rs:104-137):
 * pack f32 (m, v) pairs into words rounding to nearest, unpack words, and
 * zero `row_width` words of each listed row (a reset moment; rows past
 * num_words are ignored). */
vs_status vs_geo_encode(vs_ctx* ctx, const float* m, const float* v, uint32_t n, float epsilon, uint32_t* words);
vs_status vs_geo_decode(vs_ctx* ctx, const uint32_t* words, uint32_t n, float epsilon, float* m, float* v);
vs_status vs_geo_zero_rows(vs_ctx* ctx, uint32_t* words, uint64_t num_words, const uint32_t* rows,
                           uint32_t num_rows, uint32_t row_width);

/* Block-scaled 8-bit moment (BlockMoment, crates/splat-train/src/quant.rs:30-160;
 * kernels quant_kernels.rs:438-498, 911-925).  n values in blocks of 128: block
 * b has scales[b] = absmax / 127 and codes round(clamp(v / scale, -127, 127)) +
 * 128 (128 for a zero scale), four per u32 word, value 4w+j in byte j of word
 * w; `codes` holds ceil(n/128)*32 words, `scales` ceil(n/128) floats.  All-zero
 * codes and scales are a fresh moment (BlockMoment::zeros).  zero_rows sets the
 * codes of each listed row of `row_width` values to 128 (values past n are
 * ignored); growing the moment for new rows (BlockMoment::reset_rows' extra
 * blocks) is the caller's allocation: new words 0x80808080, new scales 0. */
vs_status vs_block8_encode(vs_ctx* ctx, const float* values, uint32_t n, uint32_t* codes, float* scales);
vs_status vs_block8_decode(vs_ctx* ctx, const uint32_t* codes, const float* scales, uint32_t n, float* values);
vs_status vs_block8_zero_rows(vs_ctx* ctx, uint32_t* codes, uint32_t n, const uint32_t* rows, uint32_t num_rows,
                              uint32_t row_width);

/* Step constants of the SH step (MomentUpdate, quant.rs:19-28, with beta2). */
typedef struct vs_sh_step_params {
    float beta1, beta2;
    float inv1, inv2;               /* 1 / (1 - beta1^t), 1 / (1 - beta2^t) */
    float epsilon, lr;              /* lr = the DC learning rate; lr_scale scales it per column */
    uint32_t round_seed;            /* the step count t: seeds the stochastic f16 rounding */
    uint32_t first;                 /* 1 on the first step (no moments yet) */
} vs_sh_step_params;

/* AdamScaled::step_sh_color (crates/splat-train/src/optim.rs:391-498;
 * BlockMoment::step quant.rs:121-161; step_kernel_w4 quant_kernels.rs:582-727).
 * One lazy Adam step of the f16 SH coefficients `sh_coeffs` [N,K,3] (IEEE
 * binary16, in place) from vs_project_update's `color_dir` [rows,6]: the
 * coefficient gradient Y_k(dir) colour_c is rebuilt per value.  `grad_rows`
 * [N] is the forward's compact_from_global (row of color_dir, 0 = culled),
 * `grad_sq` [N] vs_project_update's coeffs_grad_sq.  The second moment
 * `variance` [N] first becomes v beta2 + grad_sq (1 - beta2) for splats with a
 * row (grad_sq (1 - beta2) for every splat when p->first); then each value of
 * a splat with a row steps m = m beta1 + g (1 - beta1), c -= (m inv1 /
 * (sqrt(v inv2) + eps)) lr_scale[col] lr, rounded stochastically to f16;
 * values of culled splats keep coefficient and moment; blocks holding a
 * value of a splat with a row are re-packed, others are left as they are.
 * `lr_scale` [K*3] (device). */
vs_status vs_sh_step(vs_ctx* ctx, uint16_t* sh_coeffs, uint32_t num_splats, uint32_t sh_degree,
                     const float* color_dir, const uint32_t* grad_rows, const float* grad_sq, float* variance,
                     uint32_t* codes, float* scales, const float* lr_scale, const vs_sh_step_params* p);

/* ---- sort / scan ---------------------------------------------------------------- */

/* radix_argsort_skip_low_with_count (crates/splat-train-sort/src/lib.rs:40-189):
 * stable LSD sort of (key, value) pairs by key bits [skip, skip+8*ceil(bits/8)).
 * `n_dev` (device, may be NULL) holds the active count <= n; entries past it
 * are not read or written.  Outputs must not alias inputs.  The call waits
 * for the sort to finish, so that a pass that gave up (see
 * vs_ctx_set_sort_spin_limit) is reported here. */
vs_status vs_radix_argsort_u32(vs_ctx* ctx, const uint32_t* keys, const uint32_t* vals, uint32_t n,
                               const uint32_t* n_dev, uint32_t skip_bits, uint32_t sorting_bits,
                               uint32_t* out_keys, uint32_t* out_vals);
/* vs_radix_argsort_u32 without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Its scratch is one device array of 40 MiB per GPU, held by the library
 * until the process ends, so n <= VS_NOALLOC_SORT_MAX_KEYS (else
 * VS_ERR_CAPACITY).  Every call on a GPU uses that GPU's one array: calls on
 * one stream are ordered by it, and a call on another stream than the array's
 * last user first makes its stream wait for that user's sort (an event, no
 * allocation), so calls from several contexts or streams serialise on the
 * GPU.  Host threads are serialised by a lock while they enqueue.  If the
 * array's address could not be taken when the device's first context was
 * created, this call returns VS_ERR_INVALID (the context itself is usable).
 * Stream-ordered and does not wait: a one-sweep pass that gave up (vs_ctx_set_sort_spin_limit)
 * is reported by the context's next synchronising call (vs_radix_argsort_u32,
 * an exact render, vs_ctx_settle_lagged_counts).  Same arguments and result
 * as vs_radix_argsort_u32. */
#define VS_NOALLOC_SORT_MAX_KEYS 4194304u
vs_status vs_radix_argsort_u32_noalloc(vs_ctx* ctx, const uint32_t* keys, const uint32_t* vals, uint32_t n,
                                       const uint32_t* n_dev, uint32_t skip_bits, uint32_t sorting_bits,
                                       uint32_t* out_keys, uint32_t* out_vals);
/* The same sort on 64-bit keys, bits [0, sorting_bits) with sorting_bits <= 64
 * (e.g. a packed (tile, depth) key).  No reference counterpart: the
 * reference's sort crate takes u32 keys only. */
vs_status vs_radix_argsort_u64(vs_ctx* ctx, const uint64_t* keys, const uint32_t* vals, uint32_t n,
                               uint32_t sorting_bits, uint64_t* out_keys, uint32_t* out_vals);
/* prefix_sum (crates/splat-train-scan/src/lib.rs:24-83): inclusive scan. */
vs_status vs_prefix_sum_u32(vs_ctx* ctx, const uint32_t* in, uint32_t* out, uint32_t n);
/* scan_in_place (crates/splat-train-scan/src/lib.rs:85-96). */
vs_status vs_scan_in_place_u32(vs_ctx* ctx, uint32_t* data, uint32_t n);

/* ---- loss cotangent ------------------------------------------------------------- */

/* L1 image-loss cotangent used by the training step after the render
 * (crates/splat-train-loss/src/lib.rs:786-811 sign, :1297-1300 weights):
 * v[h,w,c] = sign(pred - gt) / (3 * count) for c < 3, 0 for alpha and for
 * masked pixels; `count` is H*W, or the number of unmasked pixels when a
 * circular mask of `mask_radius` > 0 px about (mask_cx, mask_cy) is given.
 * pred is [H,W,C] f32, gt [H,W,3] f32. */
vs_status vs_l1_cotangent(vs_ctx* ctx, const float* pred, uint32_t channels, const float* gt,
                          uint32_t img_w, uint32_t img_h, float mask_cx, float mask_cy,
                          float mask_radius, float* v_out);
/* vs_l1_cotangent with the ground truth as the reference's training loss
 * takes it (crates/splat-train-loss/src/lib.rs, header and :93,1042-1044):
 * gt_packed [H,W] u32 RGBA8, r in the low byte, each channel byte x (1/255)
 * in f32. */
vs_status vs_l1_cotangent_packed(vs_ctx* ctx, const float* pred, uint32_t channels, const uint32_t* gt_packed,
                                 uint32_t img_w, uint32_t img_h, float mask_cx, float mask_cy,
                                 float mask_radius, float* v_out);

/* ---- image loss: L1 + SSIM ------------------------------------------------------- */

/* ImageLossConfig (crates/splat-train-loss/src/lib.rs:1227-1260).  The
 * per-pixel loss is l1_weight |pred - gt| + ssim_weight SSIM(pred, gt) per
 * colour channel (ssim_weight multiplies SSIM itself: a training loss passes
 * it negative, e.g. l1_dssim(w) = {1 - w, -w}), times gt.a when `mask`, with
 * gt composited over `bg` (gt + (1 - gt.a) bg) when `composite`; an
 * alpha-match term alpha_weight |pred.a - gt.a| joins with a 4-channel pred. */
typedef struct vs_loss_cfg {
    float l1_weight, ssim_weight, alpha_weight;
    int32_t composite;
    float bg[3];
    int32_t mask;
} vs_loss_cfg;

/* LossOps::image_loss_forward / image_loss_forward_train (lib.rs:1312-1380;
 * kernel :238-478) over pred [H,W,C] f32 (C = 3 or 4) and gt_packed [H,W]
 * u32 RGBA8 (r in the low byte).  Writes (NULL skips each): the weighted
 * 16x16-tile partial sums [planes, tiles] (planes 3, or 4 with alpha
 * matching; tiles row-major) whose sum is the loss, the SSIM coefficients
 * [3][3][H,W] the backward blurs, the per-pixel loss map [H,W,C], and the
 * loss `total` [1] (needs `partials`). */
vs_status vs_image_loss_forward(vs_ctx* ctx, const float* pred, uint32_t channels, const uint32_t* gt_packed,
                                uint32_t img_w, uint32_t img_h, const vs_loss_cfg* cfg, float* partials,
                                float* coeffs, float* loss_map, float* total);
/* LossOps::image_loss_backward / image_loss_backward_coeffs (lib.rs:1335-1380;
 * kernels :481-1020): dL/dpred [H,W,C] (16-byte aligned when C = 4) from
 * dl_dpartials, the [1] gradient of the total (dl_count 1) or one per
 * partial (dl_count = planes x tiles).  `coeffs` from the forward, or NULL to
 * recompute them (same values). */
vs_status vs_image_loss_backward(vs_ctx* ctx, const float* pred, uint32_t channels, const uint32_t* gt_packed,
                                 uint32_t img_w, uint32_t img_h, const vs_loss_cfg* cfg,
                                 const float* dl_dpartials, uint32_t dl_count, const float* coeffs,
                                 float* dl_dpred);

/* ---- measurement aid ------------------------------------------------------------ */

/* Streaming kernels of known memory traffic, for calibrating the memory
 * counters that turn a profiled kernel's requests into HBM bytes (bench.py
 * --copy-calib).  No counterpart in the reference.  Reads (VS_PROBE_READ*)
 * or writes (VS_PROBE_WRITE*) each byte of `buf` [bytes] exactly once, in
 * fully coalesced 16- or 4-byte words per lane; `buf` aligned to the word
 * width and `bytes` a multiple of it.  Stream-ordered; written contents are
 * a fixed pattern. */
typedef enum vs_probe_mode {
    VS_PROBE_READ16 = 0, VS_PROBE_WRITE16 = 1, VS_PROBE_READ4 = 2, VS_PROBE_WRITE4 = 3
} vs_probe_mode;
vs_status vs_stream_probe(vs_ctx* ctx, void* buf, uint64_t bytes, int32_t mode);

/* The compositing kernels' 2^x (the G = 2^(-sigma log2 e) of every forward
 * and backward raster pass, the hardware's exp2 instruction), for checking:
 * out[i] = G(x) for the f32 x whose bit pattern is first_bits + i, i < count.
 * No counterpart in the reference, whose compositing exp is its shader's.
 * VS_ERR_INVALID when the range passes bit pattern 0xFFFFFFFF.  Stream-ordered. */
vs_status vs_compositing_exp2(vs_ctx* ctx, uint32_t first_bits, uint64_t count, float* out);

/* The raster kernels' refined quotient a / b, which must round as the
 * division does (the surfel backward replays the forward's ray-plane sample
 * with its 1 / q.z: a reciprocal refined in six instructions for
 * 2^-100 <= |b| <= 2^100, the division for other b), for checking.  No counterpart in the reference.
 * vs_raster_division: out[i] = the quotient for the f32 b whose bit pattern is
 * bits[i], i < count (device arrays).  vs_raster_division_mismatches:
 * *mismatches (device memory, one u64) = the number of the 2^32 bit patterns b
 * at which the quotient and the IEEE division a / b differ (two NaNs agree).
 * Stream-ordered. */
vs_status vs_raster_division(vs_ctx* ctx, float a, const uint32_t* bits, uint64_t count, float* out);
vs_status vs_raster_division_mismatches(vs_ctx* ctx, float a, uint64_t* mismatches);

#ifdef __cplusplus
}
#endif
#endif
