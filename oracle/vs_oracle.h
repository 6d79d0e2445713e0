/*
 * vs_oracle.h -- C ABI of the CPU oracle.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is a scalar/OpenMP CPU restatement
 * of the reference Gaussian-splat render path (voyager-so/vauss,
 * crates/splat-train-render, splat-train-sort, splat-train-scan).  It is
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg only, as the checker.  Nothing in the product links or calls it.
 *
 * The camera struct below has the same field order and sizes as
 * `vs_camera` in include/vsplat.h so one ctypes struct feeds both sides; it
 * is declared here independently on purpose.
 */
#ifndef VS_ORACLE_H
#define VS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_MODEL_PINHOLE = 0, OR_MODEL_KB4 = 1, OR_MODEL_RT8 = 2, OR_MODEL_TPF = 3 };

/* Device-side ProjectUniforms of the reference
 * (crates/splat-train-render/src/kernels/types.rs:53-82) minus the sizes. */
typedef struct or_camera {
    int32_t model;
    float fx, fy, cx, cy;
    float kb4[4];
    float viewmat[12];          /* 3x4 column-major: col0, col1, col2, translation */
    float cam_pos[3];
    float half_max_render_fov;
    float lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y, lim_r;
    float dist[8];              /* RT8: k1..k6, p1, p2; thin-prism: p1, p2, sx1, sy1 */
} or_camera;

/* Render flags (RasterPass semantics, gaussian_splats.rs:32-107). */
enum {
    OR_FLAG_BWD_INFO = 1,       /* float RGBA image + visible marks + shrunk tile ends */
    OR_FLAG_GEOMETRY = 2,       /* 12-channel output with depth/normal/distortion */
    OR_FLAG_SMOOTH_CUTOFF = 4,  /* C^1 alpha cutoff (BackwardSmoothCutoff) */
    OR_FLAG_BRUTE_FORCE = 8,    /* composite every pixel over the whole depth-sorted
                                   visible list instead of its tile's list (checks binning) */
    OR_FLAG_MIP = 16,           /* SplatRenderMode::Mip: 0.1 blur with opacity compensation */
    OR_FLAG_SURFEL = 32,        /* SplatRenderMode::Surfel (2DGS, pinhole): ray-plane coverage; with
                                   BWD_INFO the image carries the 12 geometry channels */
    OR_FLAG_SURFACE = 64,       /* surfels outside training: median by the surface criterion */
};

typedef struct or_fwd or_fwd;

/* Forward render.  `threads` <= 0 uses every OpenMP thread. */
int or_render_forward(const or_camera* cam, uint32_t img_w, uint32_t img_h,
                      const float* transforms, const float* sh_coeffs, uint32_t sh_degree,
                      const float* raw_opacities, uint32_t num_splats, float log_scale_offset,
                      const float* min_scale /* [N] scale floor or NULL */,
                      const float* decoder /* [816] neural appearance or NULL */,
                      const float background[3], int flags, int threads, or_fwd** out);

/* Sizes of the result arrays. */
typedef struct or_fwd_info {
    uint32_t num_splats, num_visible, num_intersections, num_tiles;
    uint32_t tile_bw, tile_bh, img_w, img_h, out_channels;
    uint64_t num_evaluations;   /* pixel-splat evaluations actually performed */
} or_fwd_info;
void or_fwd_get_info(const or_fwd* f, or_fwd_info* info);

/* Copy one result array out.  Fields: */
enum {
    OR_F_INTERSECT_COUNTS = 0,  /* u32 [N]   tiles hit per global splat (0 if culled) */
    OR_F_MAX_RADIUS = 1,        /* f32 [N] */
    OR_F_OPACITIES = 2,         /* f32 [N] */
    OR_F_GLOBAL_FROM_COMPACT = 3, /* u32 [V] visible splats in compaction order */
    OR_F_DEPTHS = 4,            /* f32 [V] view-space z, compaction order */
    OR_F_PROJECTED = 5,         /* f32 [V,9] x,y,c00,c01,c11,opac,r,g,b */
    OR_F_AUX = 6,               /* f32 [V,4] z,nx,ny,nz (geometry) */
    OR_F_ISECT_TILE = 7,        /* u32 [I] tile id per sorted intersection */
    OR_F_ISECT_GID = 8,         /* u32 [I] global splat id per sorted intersection */
    OR_F_TILE_OFFSETS = 9,      /* u32 [T,2] before the raster shrinks the ends */
    OR_F_TILE_OFFSETS_SHRUNK = 10, /* u32 [T,2] after it */
    OR_F_VISIBLE = 11,          /* f32 [N] */
    OR_F_OUT_IMG = 12,          /* f32 [H,W,C] (C=4 or 12) or u32 [H,W] packed */
    OR_F_SURFEL_AUX = 13,       /* f32 [V,14] surfels: M rows (9), low-pass centre (2), normal (3) */
};
int or_fwd_get(const or_fwd* f, int field, void* dst);
void or_fwd_free(or_fwd* f);

/* Backward of the same render: v_out is [H,W,C] (C as the forward image).
 * All outputs dense per global splat; pass NULL to skip one. */
int or_render_backward(const or_fwd* f, const float* v_out, int threads,
                       float* v_combined /* [N,10] */, float* v_transforms /* [N,10] */,
                       float* v_sh /* [N,K,3] */, float* v_raw_opac /* [N] */,
                       float* v_refine /* [N] */);

/* The projection VJP alone (bwd/kernels/project_backwards.rs:132-424) applied
 * to a given v_combined [N,10]: checks a projection backward on the exact
 * raster gradients it was fed. */
int or_project_backward(const or_fwd* f, const float* v_combined, int threads,
                        float* v_transforms, float* v_sh, float* v_raw_opac, float* v_refine);

/* Neural appearance backward (bwd/kernels/neural_backwards.rs, bwd/render_bwd.rs:
 * 390-435) of a forward rendered with a decoder: per-splat row gradients
 * [N,12] (base in DC units, latents, 0), their mean squares [N], the decoder
 * gradient [816] (f64 sum), and each row's view-direction term added to
 * v_transforms [N,10] (in/out, as or_render_backward wrote it; NULL skips). */
int or_neural_backward(const or_fwd* f, const float* v_combined, int threads, float* v_transforms,
                       float* v_rows, float* v_rows_sq, float* v_decoder,
                       double* v_decoder_abs /* [816] sum of |products| (a bound for summation error) or NULL */);

/* Shared transcendentals and the neural colour, for the oracle's own tests. */
void or_sincosf_n(const float* x, float* s, float* c, uint64_t n);
void or_tanhf_n(const float* x, float* y, uint64_t n);
void or_neural_color(const float row[12], const float decoder[816], const float dir[3], uint32_t degree,
                     float out[3]);

/* The camera gradient (bwd/render_bwd.rs:224-288, bwd/kernels/pose_backwards.rs):
 * d loss / d [A (row-major 3x3), b] of the camera-space perturbation
 * x_c' = (I + A) x_c + b, summed in f64 over the visible splats; `rows`
 * [N,12] (may be NULL) receives each splat's row (zero for culled splats and
 * rows without position, conic or colour gradients). */
int or_pose_backward(const or_fwd* f, const float* v_combined, int threads, double* v_pose /* [12] */,
                     float* rows /* [N,12] */);

/* FusedAdam (bwd/project_update.rs:232-250). */
typedef struct or_adam {
    float beta1, beta2, inv1, inv2, epsilon, lr_opac, opac_reg;
    uint32_t round_seed;
} or_adam;

/* project_update (bwd/kernels/project_update.rs:40-178) on host arrays: the
 * projection VJP of `v_combined` [N,10] fused with one Adam step of
 * `transforms` [N,10] and `raw_opac` [N] (updated in place, and read as the
 * pre-step values the forward saw), packed moments `w_t` [N,10], `w_o` [N].
 * color_dir is [N+1,6] with row g + 1 for splat g (NULL skips an output). */
int or_project_update(const or_fwd* f, const float* v_combined, float* transforms, float* raw_opac,
                      uint32_t* w_t, const float* lr_scale, uint32_t* w_o, const or_adam* adam,
                      float* color_dir, float* v_refine, float* grad_sq, int threads);

/* The packed-moment codec (bwd/kernels/geo_moments.rs), one value at a time. */
uint32_t or_geo_encode(float m, float v, float epsilon);               /* round to nearest */
void or_geo_decode(uint32_t word, float epsilon, float* m, float* v);
uint32_t or_geo_pack(float m, float v, float epsilon, float round_l, float round_u);
uint32_t or_mix_hash(uint32_t index, uint32_t step);
void or_adam_packed(float* param, uint32_t* word, uint32_t index, float g, float lr, const or_adam* adam,
                    uint32_t seed);

/* IEEE binary16 conversions (round to nearest even) and the SH step's
 * stochastic f16 rounding (crates/splat-train/src/quant_kernels.rs:866-894). */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);
float or_stochastic_half(float value, uint32_t index, uint32_t step);
/* Block-scaled 8-bit moment codec (crates/splat-train/src/quant.rs,
 * quant_kernels.rs:438-498, 911-925): ceil(n/128) scales, ceil(n/128)*32 words. */
void or_block8_encode(const float* values, uint64_t n, uint32_t* codes, float* scales);
void or_block8_decode(const uint32_t* codes, const float* scales, uint64_t n, float* values);
void or_block8_zero_rows(uint32_t* codes, uint64_t n, const uint32_t* rows, uint32_t num_rows, uint32_t row_width);
/* The trainer's SH step (optim.rs:391-498, quant_kernels.rs:582-727) on f16
 * coefficients sh [N,K,3] from color_dir [rows,6]; grad_rows [N] (0 = culled),
 * grad_sq [N]; variance [N], codes and scales updated in place. */
int or_sh_step(uint16_t* sh, uint32_t N, uint32_t degree, const float* color_dir, const uint32_t* grad_rows,
               const float* grad_sq, float* variance, uint32_t* codes, float* scales, const float* lr_scale,
               float beta1, float beta2, float inv1, float inv2, float epsilon, float lr,
               uint32_t round_seed, int first);

/* ImageLossConfig (crates/splat-train-loss/src/lib.rs:1227-1260). ssim_weight
 * multiplies SSIM itself (negative for a training loss). */
typedef struct or_loss_cfg {
    float l1_weight, ssim_weight, alpha_weight;
    int32_t composite;          /* composite gt over bg: gt + (1 - gt.a) bg */
    float bg[3];
    int32_t mask;               /* multiply each loss pixel by gt.a */
} or_loss_cfg;

/* image_loss_forward_kernel (lib.rs:238-478) over an [H,W,cn] f32 prediction
 * and [H,W] RGBA8-packed ground truth: per-16x16-tile weighted partial sums
 * [planes, tiles] (planes = 3, or 4 with the alpha-match term), the SSIM
 * coefficients [3][3][H,W] and the per-pixel loss map [H,W,cn]; NULL skips. */
int or_image_loss_forward(const float* pred, uint32_t cn, const uint32_t* gt, uint32_t w, uint32_t h,
                          const or_loss_cfg* cfg, float* partials, float* coeffs, float* loss_map);
/* image_loss_backward_coeffs_kernel (lib.rs:821-1020): dL/dpred [H,W,cn]. */
int or_image_loss_backward(const float* pred, uint32_t cn, const uint32_t* gt, uint32_t w, uint32_t h,
                           const or_loss_cfg* cfg, const float* dl_dpartials, int scalar_grad,
                           const float* coeffs, float* dl_dpred);

/* Stable LSD radix argsort restated (splat-train-sort/src/lib.rs:40-189):
 * sorts by key bits [skip, skip + 8*ceil(bits/8)). */
void or_radix_argsort_u32(const uint32_t* keys, const uint32_t* vals, uint32_t n,
                          uint32_t skip_bits, uint32_t sorting_bits,
                          uint32_t* out_keys, uint32_t* out_vals);
/* Inclusive prefix sum (splat-train-scan/src/lib.rs:24-83). */
void or_prefix_sum_u32(const uint32_t* in, uint32_t* out, uint32_t n);

/* Arithmetic contract transcendentals, exported for the tests. */
float or_expf(float x);
float or_logf(float x);
float or_atan2f(float y, float x);
void or_expf_n(const float* x, float* y, uint64_t n);
/* The compositing loops' default 2^x (exp2n). */
void or_exp2n_n(const float* x, float* y, uint64_t n);
/* The compositing loops' 2^x taken from a table: tab[i] is G for the f32 x
 * whose bit pattern is first_bits + i (i < count); other x keep exp2n.  The
 * table is not copied and must outlive its use; tab = NULL restores exp2n. */
void or_set_comp_exp2_table(const float* tab, uint32_t first_bits, uint64_t count);
void or_logf_n(const float* x, float* y, uint64_t n);
void or_atan2f_n(const float* y, const float* x, float* r, uint64_t n);

/* SH basis values Y_k(v) for degree <= 4 (kernels/sh.rs:51-140), for tests. */
void or_sh_basis(uint32_t degree, const float v[3], float* out /* [(d+1)^2] */);

/* Camera host math restated from camera.rs (f64). model: 0 pinhole, 1 KB4. */
double or_fov_to_focal(double fov, uint32_t pixels, int model, const float kb4[4]);
double or_focal_to_fov(double focal, uint32_t pixels, int model, const float kb4[4]);
double or_max_render_theta(int model, const float kb4[4]);
double or_kb4_d(double theta, const float kb4[4]);
double or_kb4_dd_dtheta(double theta, const float kb4[4]);
double or_kb4_invert_d(double target, const float kb4[4]);

int or_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
