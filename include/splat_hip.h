/* C ABI of libsplat_hip.so — the MI355X (gfx950) gaussian-splat render path.
 *
 * Drop-in boundary for the four FFI callables of amacati/splax's render path plus its host-side
 * sort/bin step and cache control. Plain pointers and sizes only; every device pointer is a
 * gfx950 global-memory address, and all work is enqueued on `stream` (a hipStream_t; NULL is the
 * default stream). Every entry point returns 0 on success or a nonzero status; the message of
 * the last failure on the calling thread is splat_last_error().
 *
 * The library keeps one set of scratch buffers per device, shared by every call on it. A call
 * issued on a different stream than the previous call on that device first waits on the host
 * (hipDeviceSynchronize) for the device's outstanding work, so calls from several streams or
 * threads run one after the other; calls that stay on one stream never wait.
 *
 * Batch convention (splax/_project/_kernels.py:58-75, splax/_rasterize/_kernels.py:56,408-418):
 * operands arrive flattened into their leading dimension; an operand is batched when its row
 * count exceeds num_gaussians (viewmat: exceeds 4 rows, transforms: exceeds num_transforms), and
 * broadcast otherwise. Flat item idx = image * num_gaussians + gaussian.
 *
 * Quaternions are xyzw, as the reference's kernels take them, unless a call selects wxyz (the
 * public API's order, splax/_project/_project.py:74-76). Matrices are row-major float32.
 */
#ifndef SPLAT_HIP_H
#define SPLAT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* splat_stream_t; /* hipStream_t */

/* Replaces _project_warp (splax/_project/_kernels.py:31-107, FFI callable :110-119): projection
 * over total = B * num_gaussians items plus the global inclusive scan of the tile counts.
 * Outputs (total rows each): xys [total,2], depths [total], radii [total] int32, conics [total,3],
 * num_tiles_hit [total] int32, cum_tiles_hit [total] int32 (inclusive, global over the batch).
 * transforms: (rows_transforms, 4, 4); transform_ids: [num_gaussians] (read only when
 * has_transforms != 0). quats_wxyz = 0 reads quats as xyzw, the layout the reference's kernel
 * receives after its roll (splax/_project/_project.py:76), so a binding of the reference passes
 * 0; 1 reads the public API's wxyz directly and saves the roll. */
int splat_project_fwd(splat_stream_t stream, const float* means3d, int64_t rows_means,
                      const float* scales, int64_t rows_scales, const float* quats,
                      int64_t rows_quats, const float* viewmat, int64_t rows_viewmat,
                      const float* opacities, int64_t rows_opac, const float* transforms,
                      int64_t rows_transforms, const int32_t* transform_ids,
                      int32_t num_gaussians, int32_t num_transforms, int32_t has_transforms,
                      int64_t total, int32_t img_h, int32_t img_w, float fx, float fy, float cx,
                      float cy, float glob_scale, float clip_thresh, float* xys, float* depths,
                      int32_t* radii, float* conics, int32_t* num_tiles_hit,
                      int32_t* cum_tiles_hit, int32_t quats_wxyz);

/* No counterpart in the reference: splat_project_fwd for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, validation and outputs as splat_project_fwd, bit for bit; the projection's
 * chunk-total scratch lives in a fixed device array of 65536 entries (256 KiB per device, held
 * until the process ends), so total is at most 65536 * 1024 = 67,108,864 items (status 1
 * beyond). It calls no allocating routine and uses none of the library's per-device scratch.
 * Every call on one device shares that array: calls that overlap on one device (different
 * streams or threads) race on it and must be serialized by the caller. */
int splat_project_fwd_noalloc(splat_stream_t stream, const float* means3d, int64_t rows_means,
                              const float* scales, int64_t rows_scales, const float* quats,
                              int64_t rows_quats, const float* viewmat, int64_t rows_viewmat,
                              const float* opacities, int64_t rows_opac,
                              const float* transforms, int64_t rows_transforms,
                              const int32_t* transform_ids, int32_t num_gaussians,
                              int32_t num_transforms, int32_t has_transforms, int64_t total,
                              int32_t img_h, int32_t img_w, float fx, float fy, float cx,
                              float cy, float glob_scale, float clip_thresh, float* xys,
                              float* depths, int32_t* radii, float* conics,
                              int32_t* num_tiles_hit, int32_t* cum_tiles_hit,
                              int32_t quats_wxyz);

/* Replaces _project_bwd_warp (splax/_project/_kernels.py:257-341, FFI callable :344-353).
 * Outputs: v_mean3d [B*n,3], v_scale [B*n,3], v_quat [B*n,4] (in the quats layout chosen by
 * quats_wxyz, as splat_project_fwd), v_viewmat [4B,4] (may be NULL: no viewmat gradient is
 * formed), v_transforms [B*num_transforms,4,4] (may be NULL when has_transforms == 0). All
 * outputs are fully written (no caller zeroing).
 * fold_shared != 0 (means3d, scales and quats shared, num_gaussians rows each) writes
 * v_mean3d [n,3], v_scale [n,3] and v_quat [n,4] summed over the B images in image order: the
 * cotangent of a shared parameter, which splax forms by summing the batched rows. */
int splat_project_bwd(splat_stream_t stream, const float* means3d, int64_t rows_means,
                      const float* scales, int64_t rows_scales, const float* quats,
                      int64_t rows_quats, const float* viewmat, int64_t rows_viewmat,
                      const int32_t* radii, int64_t rows_radii, const float* conics,
                      int64_t rows_conics, const float* v_xy, int64_t rows_vxy,
                      const float* v_depth, int64_t rows_vdepth, const float* v_conic,
                      int64_t rows_vconic, const float* transforms, int64_t rows_transforms,
                      const int32_t* transform_ids, int32_t num_gaussians,
                      int32_t num_transforms, int32_t has_transforms, int32_t B, float fx,
                      float fy, float glob_scale, float* v_mean3d, float* v_scale,
                      float* v_quat, float* v_viewmat, float* v_transforms,
                      int32_t quats_wxyz, int32_t fold_shared);

/* Replaces _rasterize_warp (splax/_rasterize/_kernels.py:37-87, FFI callable :90-99): sort_and_bin
 * (one pinned device-to-host read of the intersection count) then the forward blend.
 * Geometry inputs have B * num_gaussians rows; colors / opacities / map_opacities may be
 * broadcast (rows == num_gaussians) or batched; background has 1 or B rows.
 * Outputs: final_Ts [B*H, W], final_idx [B*H, W] int32, out_img [B*H, W, 3].
 * num_intersects (may be NULL) receives M. */
int splat_rasterize_fwd(splat_stream_t stream, const float* colors, int64_t rows_colors,
                        const float* opacities, int64_t rows_opac, const float* map_opacities,
                        int64_t rows_map_opac, const float* background, int64_t rows_bg,
                        const float* xys, const float* depths, const int32_t* radii,
                        const float* conics, const int32_t* cum_tiles_hit,
                        int32_t num_gaussians, int32_t B, int32_t img_h, int32_t img_w,
                        float* final_Ts, int32_t* final_idx, float* out_img,
                        int64_t* num_intersects);

/* Replaces _rasterize_depth_warp (splax/_rasterize/_kernels.py:208-262, FFI callable :265-274):
 * splat_rasterize_fwd plus the expected-depth channel out_depth [B*H, W] = sum of depths[g] times
 * the colour blend's weights (no background term); the image, final_Ts and final_idx equal
 * splat_rasterize_fwd's bit for bit. */
int splat_rasterize_depth_fwd(splat_stream_t stream, const float* colors, int64_t rows_colors,
                              const float* opacities, int64_t rows_opac,
                              const float* map_opacities, int64_t rows_map_opac,
                              const float* background, int64_t rows_bg, const float* xys,
                              const float* depths, const int32_t* radii, const float* conics,
                              const int32_t* cum_tiles_hit, int32_t num_gaussians, int32_t B,
                              int32_t img_h, int32_t img_w, float* final_Ts, int32_t* final_idx,
                              float* out_img, float* out_depth, int64_t* num_intersects);

/* Replaces _rasterize_bwd_warp (splax/_rasterize/_kernels.py:386-500, FFI callable :503-512):
 * recomputes sort_and_bin over the B_geom geometry images (deterministic, so it reproduces the
 * forward order) and runs the backward blend over B_out output images. v_out_img has vout_rows
 * rows of width W (B_out*H batched or H broadcast). Outputs (B_out * num_gaussians rows, fully
 * written): v_colors [.,3], v_opacity [.], v_xy [.,2], v_conic [.,3]. No global float atomics:
 * each intersection's sums are stored at its emission position and added per item in a fixed
 * order. */
int splat_rasterize_bwd(splat_stream_t stream, const float* colors, int64_t rows_colors,
                        const float* opacities, int64_t rows_opac, const float* map_opacities,
                        int64_t rows_map_opac, const float* background, int64_t rows_bg,
                        const float* xys, const float* depths, const int32_t* radii,
                        const float* conics, const int32_t* cum_tiles_hit,
                        const float* final_Ts, const int32_t* final_idx, const float* v_out_img,
                        int64_t vout_rows, int32_t num_gaussians, int32_t B_out, int32_t B_geom,
                        int32_t img_h, int32_t img_w, float* v_colors, float* v_opacity,
                        float* v_xy, float* v_conic);

/* Replaces _rasterize_bwd_depth_warp (splax/_rasterize/_kernels.py:797-914, FFI callable
 * :917-926): splat_rasterize_bwd with the depth channel's cotangent v_out_depth
 * (vdepth_rows rows of width W, B_out*H batched or H broadcast) and the extra output v_depths
 * [B_out*num_gaussians] (the cotangent of the projection's depths). */
int splat_rasterize_depth_bwd(splat_stream_t stream, const float* colors, int64_t rows_colors,
                              const float* opacities, int64_t rows_opac,
                              const float* map_opacities, int64_t rows_map_opac,
                              const float* background, int64_t rows_bg, const float* xys,
                              const float* depths, const int32_t* radii, const float* conics,
                              const int32_t* cum_tiles_hit, const float* final_Ts,
                              const int32_t* final_idx, const float* v_out_img,
                              int64_t vout_rows, const float* v_out_depth, int64_t vdepth_rows,
                              int32_t num_gaussians, int32_t B_out, int32_t B_geom,
                              int32_t img_h, int32_t img_w, float* v_colors, float* v_opacity,
                              float* v_xy, float* v_conic, float* v_depths);

/* Forward that keeps the sorted intersection lists resident for the backward (no counterpart in
 * the reference, whose backward re-sorts, splax/_rasterize/_kernels.py:422). The caller passes
 * buffers sorted_ids [capacity], sorted_pos [capacity] and tile_bins [B*num_tiles, 2]; sorted_ids
 * and tile_bins receive exactly what splat_sort_and_bin returns, sorted_pos each sorted
 * intersection's emission position (its index in the cum_tiles_hit-ordered emission sequence).
 * num_intersects receives M. The host does not wait for M before launching the sort and the
 * blend: they are sized by capacity and bounded on the device by the count, and M is read after
 * the last launch. When M > capacity the call returns status 6 with M reported; sorted_ids,
 * sorted_pos, tile_bins, records and the image outputs then hold the results of a list cut at
 * capacity entries (every access inside the buffers), and the caller retries with larger ones.
 * out_depth (may be NULL) selects the depth channel as in splat_rasterize_depth_fwd. records
 * (may be NULL) receives the packed blend record of every geometry item, 16 floats per item
 * ([B*num_gaussians, 16], 16-byte aligned), for splat_rasterize_bwd_sorted; it is written only
 * when capacity > 0. tile_order (may be NULL) receives the order in which the blend dispatched the
 * image tiles ([B*num_tiles] int32, a permutation of the tile indices, heaviest first within each
 * image) for splat_rasterize_bwd_sorted. compensate != 0 selects the antialiased blend of
 * splax.render (splax/_render.py:
 * 105-110): opacities are then the raw opacities, the blend uses opacities * rho(conic) with
 * rho = sqrt(clip(1 - 0.3 (a + c) + 0.09 (a c - b^2), 0, 1)) (splax/_project/_project.py:95-117),
 * and the intersection uses map_opacities as always. Other arguments and outputs as
 * splat_rasterize_fwd. */
int splat_rasterize_fwd_keep(splat_stream_t stream, const float* colors, int64_t rows_colors,
                             const float* opacities, int64_t rows_opac,
                             const float* map_opacities, int64_t rows_map_opac,
                             const float* background, int64_t rows_bg, const float* xys,
                             const float* depths, const int32_t* radii, const float* conics,
                             const int32_t* cum_tiles_hit, int32_t num_gaussians, int32_t B,
                             int32_t img_h, int32_t img_w, int64_t capacity, float* final_Ts,
                             int32_t* final_idx, float* out_img, float* out_depth,
                             int32_t* sorted_ids, int32_t* sorted_pos, int32_t* tile_bins,
                             float* records, int32_t* tile_order, int64_t* num_intersects,
                             int32_t compensate);

/* Backward over the sorted lists kept by splat_rasterize_fwd_keep (no re-sort). Arguments as
 * splat_rasterize_bwd plus sorted_ids / sorted_pos / tile_bins / records / tile_order /
 * num_intersects of the matching forward (records may be NULL: the backward then packs them
 * again from its inputs, which must be the forward's; tile_order may be NULL: the backward then
 * orders the tiles again, as it also does when B_out != B_geom; the order only schedules the
 * tiles, the outputs do not depend on it; these buffers must be the forward's, unchanged: their
 * contents are not validated, except that a tile_order entry out of range skips that tile and a
 * bin range outside [0, num_intersects] is clamped, either setting bit 0 of the device error
 * word, splat_check_device; records must be 16-byte aligned); the
 * outputs equal splat_rasterize_bwd's (same kernels;
 * additions can differ in order only among a tile's four quadrant waves). v_depths (may be NULL)
 * selects the depth channel as in splat_rasterize_depth_bwd (then depths and v_out_depth are
 * read). compensate as in the forward: v_opacity is then the raw opacities' cotangent and
 * v_conic includes the cotangent through rho. fold_shared != 0 (colors and opacities shared,
 * num_gaussians rows) writes v_colors [n,3] and v_opacity [n] summed over the B_out images in
 * image order; v_xy, v_conic and v_depths keep their per-item rows. */
int splat_rasterize_bwd_sorted(splat_stream_t stream, const float* colors, int64_t rows_colors,
                               const float* opacities, int64_t rows_opac,
                               const float* background, int64_t rows_bg, const float* xys,
                               const float* depths, const float* conics,
                               const int32_t* cum_tiles_hit, const int32_t* sorted_ids,
                               const int32_t* sorted_pos, const int32_t* tile_bins,
                               const float* records, const int32_t* tile_order,
                               int64_t num_intersects, const float* final_Ts,
                               const int32_t* final_idx, const float* v_out_img,
                               int64_t vout_rows, const float* v_out_depth, int64_t vdepth_rows,
                               int32_t num_gaussians, int32_t B_out, int32_t B_geom,
                               int32_t img_h, int32_t img_w, float* v_colors, float* v_opacity,
                               float* v_xy, float* v_conic, float* v_depths,
                               int32_t compensate, int32_t fold_shared);

/* Replaces sort_and_bin (splax/_rasterize/_sort/_sort.py:29-171), exposed for callers that keep
 * the sorted lists: writes the M sorted keys (as int64: the packed 32-bit key widened, or the
 * 64-bit key (image << (32 + tile_bits)) | (tile << 32) | raw float depth bits when fewer than 16
 * depth bits remain, _sort.py:56-66,143-170) and gaussian ids (capacity >= M required, else
 * status 6 with *num_intersects = M), and the [B*num_tiles, 2] tile bins. Status 2 when even the
 * 64-bit key overflows (image + tile bits above 32). */
int splat_sort_and_bin(splat_stream_t stream, const float* xys, const float* depths,
                       const int32_t* radii, const float* conics, const float* map_opacities,
                       int64_t rows_map_opac, const int32_t* cum_tiles_hit,
                       int32_t num_gaussians, int32_t B, int32_t img_h, int32_t img_w,
                       int64_t* sorted_keys, int32_t* sorted_ids, int64_t capacity,
                       int32_t* tile_bins, int64_t* num_intersects);

/* Replaces the _use_32bit_keys switch (splax/_rasterize/_sort/_sort.py:23-26), which the
 * reference's tests patch: force != 0 makes every sort take the 64-bit key (process-wide). */
int splat_set_wide_keys(int force);

/* ---------------------------------------------------------------- fused render path
 * splax.render (splax/_render.py:29-115, project then rasterize, each with its custom VJP) as one
 * forward and one backward call: the forward's projection also writes each item's packed blend
 * record and, for the packed key with num_gaussians >= 1024, the per-image depth range of the
 * visible items, so no record pack and no depth-range pass run; the backward keeps the per-item
 * v_xy / v_conic / v_depth rows between the blend backward and the projection VJP in library
 * scratch. Every output equals the two-call path's (splat_project_fwd +
 * splat_rasterize_fwd_keep, then splat_rasterize_bwd_sorted + splat_project_bwd) bit for bit,
 * except that sums the GPU forms with float atomics may add in another order. */

/* Forward. Arguments as splat_project_fwd over total = B * num_gaussians items (its outputs xys
 * .. cum_tiles_hit, every row written) and as splat_rasterize_fwd_keep for colors (rows
 * num_gaussians or B * num_gaussians), background, the kept lists, records (required, [B *
 * num_gaussians, 16], 16-byte aligned) and the image outputs; opacities are the raw ones, which
 * both the projection and, with compensate, the antialiased blend use (splax/_render.py:
 * 105-110). Status 6 when M > capacity, with M reported, as splat_rasterize_fwd_keep (the
 * projection outputs are whole, the lists and image those of a list cut at capacity).
 * sorted_pos, final_Ts and final_idx may be NULL when no backward will follow (a forward-only
 * render): the sort then moves no emission positions and the blend writes only the image (and
 * depth), and the kept lists cannot feed splat_render_bwd.
 * loss_kind 1 (L1) or 2 (MSE) fuses a per-pixel loss into the blend: *loss (one float, device
 * memory) receives the mean over the B * img_h * img_w * 3 colour values of |img - target| or
 * (img - target)^2 against loss_target ([B, img_h, img_w, 3]); the blend leaves each tile's
 * sum (in double, per-pixel terms exact) in library scratch and one more launch adds them in a
 * fixed order. That is the value splat_l1_loss_fwd / splat_mse_loss_fwd give for the same image,
 * up to the order of the double additions. loss_kind 0: no loss (loss_target and loss unused).
 * The reference has no fused loss: its callers apply the loss to the rendered image. */
int splat_render_fwd(splat_stream_t stream, const float* means3d, int64_t rows_means,
                     const float* scales, int64_t rows_scales, const float* quats,
                     int64_t rows_quats, const float* viewmat, int64_t rows_viewmat,
                     const float* opacities, int64_t rows_opac, const float* colors,
                     int64_t rows_colors, const float* background, int64_t rows_bg,
                     const float* transforms, int64_t rows_transforms,
                     const int32_t* transform_ids, int32_t num_gaussians,
                     int32_t num_transforms, int32_t has_transforms, int32_t B, int32_t img_h,
                     int32_t img_w, float fx, float fy, float cx, float cy, float glob_scale,
                     float clip_thresh, int32_t quats_wxyz, int32_t compensate, float* xys,
                     float* depths, int32_t* radii, float* conics, int32_t* num_tiles_hit,
                     int32_t* cum_tiles_hit, int64_t capacity, int32_t* sorted_ids,
                     int32_t* sorted_pos, int32_t* tile_bins, float* records,
                     int32_t* tile_order, float* final_Ts, int32_t* final_idx, float* out_img,
                     float* out_depth, int64_t* num_intersects, const float* loss_target,
                     int32_t loss_kind, float* loss);

/* Backward of splat_render_fwd at the same inputs, given its outputs and kept buffers and the
 * image cotangent (and, with out_depth in the forward, v_out_depth). Outputs: v_means [.,3],
 * v_scales [.,3], v_quats [.,4] (quats layout as quats_wxyz; 16-byte aligned), v_colors [.,3],
 * v_opacities [.] (the raw opacities' cotangent), v_viewmat [4B,4] (may be NULL: not formed),
 * v_transforms [B*num_transforms,4,4] (with has_transforms). Rows: num_gaussians with
 * fold_shared != 0 (means, scales, quats, colors and opacities all shared: the cotangents summed
 * over the B images in image order), else B * num_gaussians. With loss_kind 1 or 2 (the fused
 * loss of the forward) the image cotangent is formed per pixel from out_img (the forward's
 * image), loss_target and the loss cotangent *v_loss (one float, device memory) with the
 * operations of splat_l1_loss_bwd / splat_mse_loss_bwd, so the gradients equal those of the
 * separate loss's cotangent; v_out_img and vout_rows are then unused (may be NULL / 0). */
int splat_render_bwd(splat_stream_t stream, const float* means3d, int64_t rows_means,
                     const float* scales, int64_t rows_scales, const float* quats,
                     int64_t rows_quats, const float* viewmat, int64_t rows_viewmat,
                     const float* opacities, int64_t rows_opac, const float* colors,
                     int64_t rows_colors, const float* background, int64_t rows_bg,
                     const float* transforms, int64_t rows_transforms,
                     const int32_t* transform_ids, int32_t num_gaussians,
                     int32_t num_transforms, int32_t has_transforms, int32_t B, int32_t img_h,
                     int32_t img_w, float fx, float fy, float glob_scale, int32_t quats_wxyz,
                     int32_t compensate, const float* xys, const float* depths,
                     const int32_t* radii, const float* conics, const int32_t* cum_tiles_hit,
                     const int32_t* sorted_ids, const int32_t* sorted_pos,
                     const int32_t* tile_bins, const float* records, const int32_t* tile_order,
                     int64_t num_intersects, const float* final_Ts, const int32_t* final_idx,
                     const float* v_out_img, int64_t vout_rows, const float* v_out_depth,
                     int64_t vdepth_rows, float* v_means, float* v_scales, float* v_quats,
                     float* v_colors, float* v_opacities, float* v_viewmat,
                     float* v_transforms, int32_t fold_shared, const float* loss_target,
                     int32_t loss_kind, const float* out_img, const float* v_loss);

/* ---------------------------------------------------------------- training step
 * The config-4 training step around the render: the per-parameter Adam of the trainers and the
 * MCMC relocation of splax.mcmc. All arrays are contiguous float32 device buffers, updated in
 * place. */

/* One Adam parameter group: params, grads, first and second moments (size elements each) and
 * its learning rate at this step (schedules are evaluated by the caller at the pre-increment
 * count, as optax's scale_by_schedule does). The four buffers of a group must not overlap. */
typedef struct splat_adam_group {
    float* params;
    const float* grads;
    float* mu;
    float* nu;
    int64_t size;
    double lr;
} splat_adam_group;

/* Replaces optax.adam per group under optax.multi_transform (scripts/train_lego.py:203-211;
 * optax 0.2.8 scale_by_adam + scale_by_learning_rate + apply_updates): one launch for up to 8
 * groups. count is the incremented step count (1 on the first update); the bias corrections
 * 1 - b^count are formed in double and rounded to float32. */
int splat_adam_step(splat_stream_t stream, const splat_adam_group* groups, int32_t num_groups,
                    double b1, double b2, double eps, double eps_root, int64_t count);

/* Parameter maps of splat_adam_step_mapped: the group's gradient is the cotangent of the
 * group's value under render_log's map (splax/_render.py:161-164) and the update first applies
 * the map's reverse-mode rule at the parameter before the update, with the float operations of
 * splat_log_params_bwd. */
#define SPLAT_MAP_NONE 0    /* the gradient is the parameter's own */
#define SPLAT_MAP_EXP 1     /* scales = exp(log_scales) */
#define SPLAT_MAP_SIGMOID 2 /* colours / opacities = sigmoid(logits) */
#define SPLAT_MAP_QUAT 3    /* quats / (|quats| + 1e-8), rows of 4 (16-byte aligned) */

/* splat_adam_step with a parameter map per group (maps[num_groups], SPLAT_MAP_*; NULL = none):
 * the reference's render_log backward (splax/_render.py:161-164, here splat_log_params_bwd)
 * followed by the update, in one launch. No counterpart entry point in the reference, whose
 * optax update takes the gradients jax.grad returns for the log / logit parameters; bit for bit
 * equal to splat_log_params_bwd then splat_adam_step. */
int splat_adam_step_mapped(splat_stream_t stream, const splat_adam_group* groups,
                           int32_t num_groups, const int32_t* maps, double b1, double b2,
                           double eps, double eps_root, int64_t count);

/* Replaces _reset_opt_state (scripts/train_lego.py:136-146): zeroes mu and nu of every row
 * whose reset[row] != 0; each group's size must be a multiple of num_rows (its row width). */
int splat_adam_reset_rows(splat_stream_t stream, const splat_adam_group* groups,
                          int32_t num_groups, const uint8_t* reset, int64_t num_rows);

/* Replaces splax.mcmc.relocate (splax/mcmc.py:74-131) in place on the [N,3] means3d, [N,3]
 * log_scales, [N,4] quats (wxyz, copied as is), [N,3] logit_colors and [N] logit_opacities.
 * n_max is the binomial table size of make_binoms (splax/mcmc.py:29-41), at most 62. The
 * source draw uses Philox4x32-10 keyed by seed (the reference uses a JAX PRNG key), with
 * probability exactly proportional to opacity among the alive gaussians. source (may be NULL)
 * receives the reference's `source` (drawn source for dead rows, the row itself otherwise);
 * reset (may be NULL) the rows whose optimizer moments the caller should zero. */
int splat_mcmc_relocate(splat_stream_t stream, float* means3d, float* log_scales, float* quats,
                        float* logit_colors, float* logit_opacities, int64_t num_gaussians,
                        int32_t n_max, float min_opacity, uint64_t seed, int32_t* source,
                        uint8_t* reset);

/* Replaces splax.mcmc.inject_noise (splax/mcmc.py:134-169): out_means [n,3] = means3d +
 * Sigma (z sigmoid(100 (min_opacity - o)) scaler) with Sigma = R diag(exp(log_scales))^2 R^T
 * (R of the normalized wxyz quats [n,4]), o = sigmoid(logit_opacities [n]) and z three standard
 * normals per gaussian, read from noise [n,3] when it is not NULL, else drawn by Box-Muller from
 * Philox4x32-10 keyed by seed (the reference draws with a JAX PRNG key). out_means may be
 * means3d (in place). */
int splat_mcmc_inject_noise(splat_stream_t stream, const float* means3d, const float* log_scales,
                            const float* quats, const float* logit_opacities,
                            int64_t num_gaussians, float scaler, float min_opacity,
                            uint64_t seed, const float* noise, float* out_means);

/* Replaces splax.mcmc.compute_relocation (splax/mcmc.py:44-71): opacities [n], scales [n,3],
 * ratios [n] (rounded, clipped to [1, n_max]) -> new_opacities [n], new_scales [n,3]. Evaluated
 * in double with exact binomial coefficients. */
int splat_mcmc_compute_relocation(splat_stream_t stream, const float* opacities,
                                  const float* scales, const float* ratios, int64_t n,
                                  int32_t n_max, float* new_opacities, float* new_scales);

/* Replaces render_log's parameter map (splax/_render.py:161-164), one pass over n gaussians:
 * scales = exp(log_scales) [n,3], quats_out = quats / (|quats| + 1e-8) [n,4] (any order),
 * colors = sigmoid(logit_colors) [n,3], opacities = sigmoid(logit_opacities) [n]. exp is the
 * library's fixed-sequence exp. */
int splat_log_params_fwd(splat_stream_t stream, const float* log_scales, const float* quats,
                         const float* logit_colors, const float* logit_opacities, int64_t n,
                         float* scales, float* quats_out, float* colors, float* opacities);

/* Reverse mode of splat_log_params_fwd at the same inputs: cotangents of its four outputs (any
 * may be NULL, a zero cotangent) to those of its four inputs. */
int splat_log_params_bwd(splat_stream_t stream, const float* log_scales, const float* quats,
                         const float* logit_colors, const float* logit_opacities, int64_t n,
                         const float* v_scales, const float* v_quats, const float* v_colors,
                         const float* v_opacities, float* v_log_scales, float* v_quats_in,
                         float* v_logit_colors, float* v_logit_opacities);

/* The trainers' L1 loss mean |img - target| over count elements (scripts/train_lego.py:111),
 * summed in double in a fixed order; partials is scratch of ceil(count / 4096) doubles and loss
 * one float, both device memory. */
int splat_l1_loss_fwd(splat_stream_t stream, const float* img, const float* target,
                      int64_t count, double* partials, float* loss);

/* Cotangent of the L1 loss: v_img = sign(img - target) * (*v_loss / count), v_loss a device
 * scalar. */
int splat_l1_loss_bwd(splat_stream_t stream, const float* img, const float* target,
                      int64_t count, const float* v_loss, float* v_img);

/* MSE loss mean (img - target)^2 over count elements, the loss of the benchmark workloads 0-3
 * (no counterpart in the reference library; its callers form the loss in JAX), summed in double
 * in a fixed order; arguments as splat_l1_loss_fwd. One pass each way, where torch's mse_loss
 * takes four kernels and a fill. */
int splat_mse_loss_fwd(splat_stream_t stream, const float* img, const float* target,
                       int64_t count, double* partials, float* loss);

/* Cotangent of the MSE loss: v_img = 2 (img - target) * (*v_loss / count). */
int splat_mse_loss_bwd(splat_stream_t stream, const float* img, const float* target,
                       int64_t count, const float* v_loss, float* v_img);

/* Replaces clear_cache (splax/_cache.py:158-164): frees the per-device scratch. */
void splat_clear_cache(void);

/* Message of the last failed call on this thread ("" if none). */
const char* splat_last_error(void);

/* Stage timing with HIP events on the caller's stream (no counterpart in the reference; used by
 * the benchmark). Stages whose bit is set in stage_mask (0 turns timing off) are bracketed by
 * events at every launch; get_stage_times waits for them and returns, per stage, the summed
 * milliseconds and the number of calls, then resets. Stages: 0 project, 1 minmax, 2 emit,
 * 3 sort, 4 bins, 5 blend_fwd, 6 blend_bwd, 7 project_bwd; 8 and 9 time the forward and backward
 * blend kernels alone, with the events carried by their dispatch (hipExtLaunchKernelGGL), so no
 * marker is enqueued between kernels. */
int splat_set_stage_timing(int stage_mask);
int splat_get_stage_times(double* ms, int64_t* calls, int32_t n);

/* Waits for the current device and returns (then clears) its device error word: 0 when every
 * kernel ran within its invariants; bit 0 (value 1) when splat_rasterize_bwd_sorted or
 * splat_render_bwd met a kept tile order entry or tile-bin range out of range (that tile is then skipped or its range
 * clamped to [0, M], so nothing is read out of bounds, but the call's gradients are not the
 * forward's). No counterpart in the reference. */
int splat_check_device(void);

/* Library ABI version (bumped on any signature or contract change). */
int splat_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
