/* CPU oracle for the gaussian-splat render path — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
 * only as the checker (or as the timed CPU baseline). The product path (libsplat_hip.so) never
 * links, loads or calls it.
 *
 * Each function restates one reference kernel of amacati/splax (file:line cited in the .c file).
 * Array conventions follow the reference's Warp FFI callbacks: batched operands arrive flattened
 * into their leading dimension, and an operand is "batched" iff its row count exceeds n
 * (splax/_project/_kernels.py:68-75). All float math follows the arithmetic contract written in
 * splat_oracle.c so that the GPU library can match it bit for bit.
 */
#ifndef SPLAT_ORACLE_H
#define SPLAT_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float oracle_logf(float x);
float oracle_expf(float x);
void oracle_logf_n(const float* x, float* y, int64_t n);
void oracle_expf_n(const float* x, float* y, int64_t n);
void oracle_blend_expf_n(const float* x, float* y, int64_t n);
int oracle_set_threads(int n);

/* Key layout of the packed 32-bit sort key (splax/_rasterize/_sort/_sort.py:51-60).
 * out[0]=tile_bounds_x, out[1]=tile_bounds_y, out[2]=num_tiles, out[3]=tile_n_bits,
 * out[4]=image_n_bits, out[5]=depth_bits. Returns 1 if the packed key fits (depth_bits >= 16). */
int oracle_key_layout(int32_t B, int32_t img_h, int32_t img_w, int32_t* out);

int oracle_project_fwd(const float* means3d, int64_t rows_means, const float* scales,
                       int64_t rows_scales, const float* quats_xyzw, int64_t rows_quats,
                       const float* viewmat, int64_t rows_viewmat, const float* opacities,
                       int64_t rows_opac, const float* transforms, int64_t rows_transforms,
                       const int32_t* transform_ids, int32_t n, int32_t num_transforms,
                       int32_t has_transforms, int64_t total, int32_t img_h, int32_t img_w,
                       float fx, float fy, float cx, float cy, float glob_scale,
                       float clip_thresh, float* xys, float* depths, int32_t* radii,
                       float* conics, int32_t* num_tiles_hit, int32_t* cum_tiles_hit);

/* Force the 64-bit key for every layout (the reference's tests patch _use_32bit_keys,
 * splax/_rasterize/_sort/_sort.py:23-26, the same way). */
void oracle_set_wide_keys(int force);
/* 0: packed 32-bit key; 1: 64-bit key; -2: image + tile bits above 32 (overflow). */
int oracle_key_mode(int32_t B, int32_t img_h, int32_t img_w);

/* 64-bit key path of sort_and_bin: emission-order keys, and sorted keys / ids / bins. */
int64_t oracle_emit_keys_wide(const float* xys, const float* depths, const int32_t* radii,
                              const float* conics, const float* map_opac, int64_t rows_map_opac,
                              const int32_t* cum, int32_t n, int32_t B, int32_t img_h,
                              int32_t img_w, int64_t* keys, int32_t* ids, int64_t cap);
int64_t oracle_sort_and_bin_wide(const float* xys, const float* depths, const int32_t* radii,
                                 const float* conics, const float* map_opac,
                                 int64_t rows_map_opac, const int32_t* cum, int32_t n, int32_t B,
                                 int32_t img_h, int32_t img_w, int64_t* sorted_keys,
                                 int32_t* sorted_ids, int64_t cap, int32_t* tile_bins);

/* Emission order (unsorted) keys and ids, exactly num_tiles_hit per visible item at cum[idx-1].
 * Returns the number of emitted keys, or a negative code (-2: key does not pack). */
int64_t oracle_emit_keys(const float* xys, const float* depths, const int32_t* radii,
                         const float* conics, const float* map_opac, int64_t rows_map_opac,
                         const int32_t* cum, int32_t n, int32_t B, int32_t img_h, int32_t img_w,
                         int32_t* keys, int32_t* ids, int64_t cap, float* depth_mm);

/* Full sort_and_bin: emit, stable sort by key, bin edges. Returns M or a negative code. */
int64_t oracle_sort_and_bin(const float* xys, const float* depths, const int32_t* radii,
                            const float* conics, const float* map_opac, int64_t rows_map_opac,
                            const int32_t* cum, int32_t n, int32_t B, int32_t img_h,
                            int32_t img_w, int32_t* sorted_keys, int32_t* sorted_ids,
                            int64_t cap, int32_t* tile_bins);

/* Forward blend over given sorted ids and tile bins. stats (may be NULL): [Pc, Pr]. With a
 * non-NULL out_depth [B*H*W], also the expected depth from depths [B*n] (depth channel). */
void oracle_blend_fwd(const float* colors, int64_t rows_colors, const float* opacities,
                      int64_t rows_opac, const float* background, int64_t rows_bg,
                      const float* xys, const float* conics, const int32_t* sorted_ids,
                      const int32_t* tile_bins, int32_t B, int32_t img_h, int32_t img_w,
                      float* final_Ts, int32_t* final_idx, float* out_img, int64_t* stats,
                      const float* depths, float* out_depth);

/* rasterize forward = sort_and_bin + blend. Returns M or a negative code. */
int64_t oracle_rasterize_fwd(const float* colors, int64_t rows_colors, const float* opacities,
                             int64_t rows_opac, const float* map_opac, int64_t rows_map_opac,
                             const float* background, int64_t rows_bg, const float* xys,
                             const float* depths, const int32_t* radii, const float* conics,
                             const int32_t* cum, int32_t n, int32_t B, int32_t img_h,
                             int32_t img_w, float* final_Ts, int32_t* final_idx,
                             float* out_img, int64_t* stats, float* out_depth);

/* rasterize backward (recomputes the sort). stats (may be NULL): [Qc, Qr]. With a non-NULL
 * v_depths [B_out*n], the depth-channel backward with cotangent v_out_depth (vdepth_rows rows of
 * width W). */
int64_t oracle_rasterize_bwd(const float* colors, int64_t rows_colors, const float* opacities,
                             int64_t rows_opac, const float* map_opac, int64_t rows_map_opac,
                             const float* background, int64_t rows_bg, const float* xys,
                             const float* depths, const int32_t* radii, const float* conics,
                             const int32_t* cum, const float* final_Ts, const int32_t* final_idx,
                             const float* v_out, int64_t vout_rows, int32_t n, int32_t B_out,
                             int32_t B_geom, int32_t img_h, int32_t img_w, float* v_colors,
                             float* v_opacity, float* v_xy, float* v_conic, int64_t* stats,
                             const float* v_out_depth, int64_t vdepth_rows, float* v_depths);

/* The float64 truth of oracle_rasterize_bwd: the same pairs and accept decisions, every value
 * after them in double; out holds [B_out * n, NG] sums (v_colour 3, v_conic 3, v_xy 2,
 * v_opacity, and v_depth when v_out_depth is given). */
int64_t oracle_rasterize_bwd_f64(const float* colors, int64_t rows_colors, const float* opacities,
                                 int64_t rows_opac, const float* map_opac, int64_t rows_map_opac,
                                 const float* background, int64_t rows_bg, const float* xys,
                                 const float* depths, const int32_t* radii, const float* conics,
                                 const int32_t* cum, const float* final_Ts,
                                 const int32_t* final_idx, const float* v_out_img,
                                 int64_t vout_rows, int32_t n, int32_t B_out, int32_t B_geom,
                                 int32_t img_h, int32_t img_w, const float* v_out_depth,
                                 int64_t vdepth_rows, double* out);

int oracle_project_bwd(const float* means3d, int64_t rows_means, const float* scales,
                       int64_t rows_scales, const float* quats_xyzw, int64_t rows_quats,
                       const float* viewmat, int64_t rows_viewmat, const int32_t* radii,
                       int64_t rows_radii, const float* conics, int64_t rows_conics,
                       const float* v_xy, int64_t rows_vxy, const float* v_depth,
                       int64_t rows_vdepth, const float* v_conic, int64_t rows_vconic,
                       const float* transforms, int64_t rows_transforms,
                       const int32_t* transform_ids, int32_t n, int32_t num_transforms,
                       int32_t has_transforms, int32_t B, float fx, float fy, float glob_scale,
                       float* v_mean3d, float* v_scale, float* v_quat, float* v_viewmat,
                       float* v_transforms);

#ifdef __cplusplus
}
#endif
#endif
