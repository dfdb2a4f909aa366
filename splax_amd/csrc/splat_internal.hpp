// Internal interfaces of the gfx950 splat library: argument bundles, the per-device scratch
// cache, error codes and device-side scan helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <string>
#include <vector>

namespace splat {

// ------------------------------------------------------------------ error codes
enum : int {
    kOk = 0,
    kErrArgs = 1,         // invalid shapes / arguments (reference raises ValueError)
    kErrKeyOverflow = 2,  // image and tile ids do not fit the 32-bit key
    kErrAlloc = 3,
    kErrLaunch = 4,
    kErrRuntime = 5,
    kErrTooMany = 6,      // intersection count beyond the int32 / 2^31 range
};

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

// ------------------------------------------------------------------ argument bundles
struct ProjectArgs {
    const float* means; int64_t rows_means;
    const float* scales; int64_t rows_scales;
    const float* quats; int64_t rows_quats;
    const float* viewmat; int64_t rows_viewmat;
    const float* opacities; int64_t rows_opac;
    const float* transforms; int64_t rows_transforms;
    const int32_t* transform_ids;
    int32_t n, num_transforms, has_transforms;
    int64_t total;
    int32_t img_h, img_w;
    float fx, fy, cx, cy, glob_scale, clip_thresh;
    float* xys; float* depths; int32_t* radii; float* conics;
    int32_t* num_tiles_hit; int32_t* cum_tiles_hit;
    int32_t quats_wxyz = 0;  // quaternions stored wxyz instead of the kernel's xyzw
};

struct ProjectBwdArgs {
    const float* means; int64_t rows_means;
    const float* scales; int64_t rows_scales;
    const float* quats; int64_t rows_quats;
    const float* viewmat; int64_t rows_viewmat;
    const int32_t* radii; int64_t rows_radii;
    const float* conics; int64_t rows_conics;
    const float* v_xy; int64_t rows_vxy;
    const float* v_depth; int64_t rows_vdepth;
    const float* v_conic; int64_t rows_vconic;
    const float* transforms; int64_t rows_transforms;
    const int32_t* transform_ids;
    int32_t n, num_transforms, has_transforms, B;
    float fx, fy, glob_scale;
    float* v_mean3d; float* v_scale; float* v_quat; float* v_viewmat; float* v_transforms;
    int32_t quats_wxyz = 0;  // quats (and v_quat) stored wxyz instead of xyzw
    int32_t fold = 0;        // v_mean3d / v_scale / v_quat summed over the images (n rows)
};

// Geometry of one sort_and_bin call (splax/_rasterize/_sort/_sort.py:51-60).
// packed: the 32-bit key (at least 16 depth bits left); otherwise the 64-bit key, which
// overflows when image + tile bits exceed 32 (splax/_rasterize/_sort/_sort.py:56-66).
struct KeyLayout {
    int32_t tiles_x, tiles_y, num_tiles, tile_bits, image_bits, depth_bits;
    bool packed, overflow;
};
KeyLayout key_layout(int32_t B, int32_t img_h, int32_t img_w);
// Force the 64-bit key for every layout (the reference's tests patch _use_32bit_keys).
void set_force_wide_keys(bool force);

// Digit passes of the sort: at most 8 bytes of a 64-bit key.
constexpr int kMaxPasses = 8;
constexpr int kSortTileMin = 4096;   // keys per radix-sort partition (smallest size used)
constexpr int64_t kSortBigM = 1 << 20;  // from this many keys on, partitions hold 8192 keys

// Inputs of sort_and_bin and the blends.
struct RasterInputs {
    const float* colors; int64_t rows_colors;
    const float* opac; int64_t rows_opac;
    const float* map_opac; int64_t rows_map_opac;
    const float* background; int64_t rows_bg;
    const float* xys; const float* depths; const int32_t* radii; const float* conics;
    const int32_t* cum;
    int32_t n, B_geom, img_h, img_w;
    // opac holds raw opacities and the blend uses opac * rho(conic), the antialiasing
    // compensation of splax/_project/_project.py:95-117 (kept-list entry points only)
    int32_t compensate = 0;
};

// ------------------------------------------------------------------ device words / scratch
enum : int {
    kCountWord = 62,     // the render path's intersection count (chunk_scan_kernel) in `tickets`
    kDeviceError = 63,   // device error word in `tickets` (bit flags, see kDevErr*)
    kNumTickets = 64,
};
// Bits of the device error word (splat_check_device).
enum : uint32_t {
    kDevErrKeptLists = 1u,  // a kept tile order / tile-bin entry was out of range (bwd_sorted)
};

// Grow-only per-device scratch, the counterpart of splax/_cache.py:52-90. The intersection
// buffers grow with 1.25x headroom; everything is freed by splat_clear_cache().
struct DeviceScratch {
    int device = -1;
    int compute_units = 0;
    std::mutex mu;
    // projection scan
    uint32_t* chunk_sums = nullptr; int64_t chunk_sums_cap = 0;  // projection scan partials
    uint32_t* tickets = nullptr;
    // sort
    int32_t* keys[2] = {nullptr, nullptr};   // packed 32-bit keys (ping-pong)
    uint64_t* wkeys[2] = {nullptr, nullptr};  // 64-bit keys (ping-pong), allocated on first use
    int64_t wide_cap = 0;
    int32_t* vals[2] = {nullptr, nullptr};  // emission positions (ping-pong)
    int32_t* gids[2] = {nullptr, nullptr};  // flat item ids (ping-pong; [0] ends sorted)
    int64_t isect_cap = 0;
    // backward: nine partial gradient sums per (output image, intersection), emission order
    float* rgrad = nullptr; int64_t rgrad_cap = 0;
    // blends: packed per-item records (4 float4 each)
    float4* recs = nullptr; int64_t recs_cap = 0;
    // fused render backward: per-item 2D cotangents (v_xy 2, v_conic 3, v_depth 1 per item)
    float* item_grads = nullptr; int64_t item_grads_cap = 0;
    // blends: workgroup -> (image, tile) dispatch order
    int32_t* tile_order = nullptr; int64_t order_cap = 0;
    // projection backward: 12 viewmat-gradient partials per (image, workgroup)
    float* view_partials = nullptr; int64_t view_partials_cap = 0;
    // fused render loss: one partial sum per blend workgroup (image, tile)
    double* loss_partials = nullptr; int64_t loss_partials_cap = 0;
    uint32_t* part_counts = nullptr; int64_t part_counts_cap = 0;  // 256 * partitions
    uint32_t* hist = nullptr;                                       // 256 digit totals
    int32_t* tile_bins = nullptr; int64_t bins_cap = 0;             // (start, end) pairs
    float* depth_mm = nullptr; int64_t mm_cap = 0;                  // 2 * B
    uint32_t* mm_partial = nullptr; int64_t mm_partial_cap = 0;     // 2 * blocks
    int32_t* pinned_count = nullptr;
    int32_t* pinned_count_dev = nullptr;  // the device's address of pinned_count
    hipEvent_t count_event = nullptr;
    int64_t last_count = -1;  // the last settled deferred count: the sort's partition shape
    // Calls on one device share these buffers: a call on another stream than the last user's
    // first waits on the host for the device's work, so calls from different streams run one
    // after the other.
    hipStream_t last_stream = nullptr;
    bool has_last = false;
    // workload signature (B_geom, n, num_tiles) of the last sort or blend call: a call with
    // another one drops every workload-sized buffer first (splax/_cache.py:61-75)
    int32_t sig_B = -1, sig_n = -1, sig_tiles = -1;

    int ensure_base();
    void workload(int32_t B, int32_t n, int32_t num_tiles);
    void release_sized();
    int order_after_last(hipStream_t s);
    void mark_done(hipStream_t s);
    int grow_chunk_sums(int64_t blocks);
    int ensure_sort(int64_t M, int64_t bins, int32_t B, bool wide);
    int ensure_rgrad(int64_t count);
    int ensure_recs(int64_t items);
    int ensure_item_grads(int64_t items);
    int ensure_order(int64_t blocks);
    int ensure_view_partials(int64_t count);
    int ensure_loss_partials(int64_t count);
    void release();
};

DeviceScratch& scratch_for_current_device();
void release_all_scratch();

// Holds the device's scratch for one entry point: takes its lock, allocates the base buffers,
// orders the call's stream after the previous user's, and on exit records the stream.
struct ScratchUse {
    DeviceScratch& sc;
    hipStream_t stream;
    std::lock_guard<std::mutex> lock;
    int rc;
    ScratchUse(DeviceScratch& d, hipStream_t s) : sc(d), stream(s), lock(d.mu) {
        rc = sc.ensure_base();
        if (!rc) rc = sc.order_after_last(s);
    }
    ~ScratchUse() {
        if (!rc) sc.mark_done(stream);
    }
    ScratchUse(const ScratchUse&) = delete;
    ScratchUse& operator=(const ScratchUse&) = delete;
};

// ------------------------------------------------------------------ stage timing
enum Stage : int {
    kStageProject = 0,
    kStageMinmax,
    kStageEmit,
    kStageSort,
    kStageBins,
    kStageBlendFwd,
    kStageBlendBwd,
    kStageProjectBwd,
    kKernelBlendFwd,  // the blend kernel alone (its dispatch carries the events)
    kKernelBlendBwd,
    kNumStages
};
// When timing is on for a kernel entry, hands out the two events its hipExtLaunchKernelGGL
// dispatch records (start and end of that kernel only) and queues them for splat_get_stage_times.
bool kernel_timer_events(int stage, hipEvent_t* start, hipEvent_t* end);
struct StageTimer {
    hipStream_t stream;
    int stage;
    hipEvent_t start = nullptr;
    StageTimer(hipStream_t s, int st);
    ~StageTimer();
};

// ------------------------------------------------------------------ launchers
// Frees the relocation scratch of every device (train.hip).
void release_train_scratch();

int fill_zero_f32(float* p, int64_t n, hipStream_t stream);
int fill_zero_i32(int32_t* p, int64_t n, hipStream_t stream);
int launch_project_fwd(const ProjectArgs& a, DeviceScratch& sc, hipStream_t stream);
// The projection with its chunk-total scratch (project_fwd_chunks(a.total) uint32) supplied.
int launch_project_fwd_into(const ProjectArgs& a, uint32_t* chunk_sums, hipStream_t stream);
// The fused render forward's projection: also each item's packed blend record (recs, 4 float4
// per item, from colors / compensate as launch_pack_records would write it) and, with depth_mm
// non-null (requires n >= 1024), the per-image depth range of the visible items (mm_partial:
// scratch of 4 uint32 per chunk), as the sort's depth-range kernels would compute it.
struct FusedRecords {
    const float* colors; int64_t rows_colors;
    int32_t compensate;
    float4* recs;
    uint32_t* mm_partial;
    float* depth_mm;
    // non-null: with several chunks the chunk scan writes the intersection count here and the
    // projection leaves cum_tiles_hit chunk-local (chunk_sums then hold the chunks' exclusive
    // prefixes): the emission adds them (SortTargets::chunk_prefix)
    int32_t* count_word = nullptr;
    // non-null (with count_word): the chunk scan also stores the count into this host-visible
    // word (DeviceScratch::pinned_count_dev), so the readback needs no copy
    int32_t* count_host = nullptr;
};
int launch_project_fwd_fused(const ProjectArgs& a, const FusedRecords& f, DeviceScratch& sc,
                             hipStream_t stream);
int launch_project_fwd_impl(const ProjectArgs& a, uint32_t* chunk_sums, const FusedRecords* f,
                            hipStream_t stream);
// Items per chunk of the projection's tile-count scan (one projection workgroup each).
constexpr int64_t kProjChunkItems = 1024;
int64_t project_fwd_chunks(int64_t total);
// Adds chunk c's exclusive prefix to the items of chunk c (1024 items per chunk), c >= 1.
int launch_chunk_offsets(int32_t* cum, int64_t total, const uint32_t* chunk_prefix,
                         hipStream_t stream);
// The projection with no allocation: its chunk totals in a fixed device array of
// kNoAllocMaxChunks entries per device (one per 1024 items).
constexpr int64_t kNoAllocMaxChunks = 65536;
int launch_project_fwd_noalloc(const ProjectArgs& a, hipStream_t stream);
int launch_project_bwd(const ProjectBwdArgs& a, DeviceScratch& sc, hipStream_t stream);

// Optional caller-owned destinations of sort_and_bin: M_known >= 0 skips the count readback
// (it must equal cum[B*n - 1]); ids / pos / bins (when non-null) receive the sorted gaussian ids,
// the sorted emission positions and the tile bins instead of the library scratch. With
// capacity >= 0 (and no M_known) the count is not waited for: the launches are sized by the
// capacity and bounded on the device by the count, and the caller calls settle_count after its
// last launch, which reports a count above the capacity as kErrTooMany (the outputs of that call
// are then those of a truncated list, every access still inside the buffers).
struct SortTargets {
    int64_t M_known = -1;
    int64_t capacity = -1;
    int32_t* ids = nullptr;
    int32_t* pos = nullptr;
    int32_t* bins = nullptr;
    const float* depth_mm = nullptr;  // per-image depth range already formed (fused projection)
    // the fused projection's chunk-local cum_tiles_hit (FusedRecords::count_word): the emission
    // finalizes each item's entry in place (in.cum) from these per-chunk exclusive prefixes, and
    // count_src (else in.cum's last entry) holds the intersection count
    const uint32_t* chunk_prefix = nullptr;
    const int32_t* num_tiles_hit = nullptr;
    const int32_t* count_src = nullptr;
    // the kernel that forms count_src also stores it into the pinned readback word
    // (FusedRecords::count_host): only the readback event is recorded
    bool count_on_host = false;
};

// Where sort_and_bin left its results: sorted keys (int32 when packed, uint64 when wide), ids,
// emission positions (tgt's buffers when given) and bins.
struct SortOutputs {
    const void* keys = nullptr;
    bool wide = false;
    const int32_t* ids = nullptr;
    const int32_t* pos = nullptr;
    const int32_t* bins = nullptr;
    bool count_deferred = false;  // the count is still to be settled (settle_count)
    bool high_keys = false;  // packed keys kept as their 16-bit high halves (image, tile)
};

// sort_and_bin: returns M (>= 0) in *M_out, or -1 with a deferred count, and the result
// locations in *out. full_keys keeps the whole sorted keys (splat_sort_and_bin returns them);
// otherwise packed keys leave the sort as their 16-bit high halves.
int run_sort_and_bin(const RasterInputs& in, DeviceScratch& sc, hipStream_t stream,
                     int64_t* M_out, KeyLayout* lay_out, const SortTargets* tgt,
                     SortOutputs* out, bool full_keys = false);
// Waits for the deferred count's readback (enqueued after the projection, so normally long
// complete), reports it in *M_out and fails with kErrTooMany above the capacity.
int settle_count(DeviceScratch& sc, int64_t capacity, int64_t* M_out);

// Writes the packed blend record (4 float4) of each of the in.B_geom * in.n geometry items.
int launch_pack_records(const RasterInputs& in, float4* recs, hipStream_t stream);

// A per-pixel loss fused into the blends, the mean over every colour value of the images of
// |img - target| (kind kLossL1) or (img - target)^2 (kLossMse). The forward blend leaves one
// double partial sum per workgroup, at its tile's index (image * num_tiles + tile), for
// launch_loss_final; the backward blend forms the image cotangent of each pixel from the image,
// the target and the loss cotangent *v_loss as the loss's own backward does (loss_bwd_kernel).
constexpr int32_t kLossNone = 0, kLossL1 = 1, kLossMse = 2;
struct PixelLoss {
    int32_t kind = kLossNone;
    const float* target = nullptr;  // [images][H][W][3], as the image
    double* partials = nullptr;     // forward: images * num_tiles
    const float* img = nullptr;     // backward: the forward's image
    const float* v_loss = nullptr;  // backward: the loss cotangent (one float, device memory)
    int64_t count = 0;              // images * H * W * 3 (the mean's divisor)
};

// out_depth non-null: also the expected-depth channel (in.depths per geometry item). recs holds
// the records written by launch_pack_records for the same inputs. order (in.B_geom * num_tiles)
// receives the tile dispatch order the blend runs in. loss (may be null): the fused loss's
// per-tile partials.
int launch_blend_fwd(const RasterInputs& in, const KeyLayout& lay, const int32_t* sorted_ids,
                     const int32_t* tile_bins, float* final_Ts, int32_t* final_idx,
                     float* out_img, float* out_depth, const float4* recs, int32_t* order,
                     const PixelLoss* loss, hipStream_t stream);
// The fused loss's value: the blocks partials summed in a fixed order, divided by count (the
// number of colour values), into *loss.
int launch_loss_final(const double* partials, int64_t blocks, int64_t count, float* loss,
                      hipStream_t stream);

// Backward over sorted lists of M intersections: sorted_ids / sorted_pos / tile_bins as produced
// by sort_and_bin; in.cum gives each item's emission range; rgrad is scratch of
// B_out_eff * M * NG floats (B_out_eff = 1 when geometry is batched, else B_out; NG = 9, or 10
// with the depth channel). v_depths non-null selects the depth channel (in.depths, v_out_depth).
struct BlendBwdArgs {
    const float* final_Ts; const int32_t* final_idx;
    const float* v_out; int64_t vout_rows;
    int32_t B_out;
    const int32_t* sorted_pos; int64_t M; float* rgrad;
    float* v_colors; float* v_opacity; float* v_xy; float* v_conic;
    const float* v_out_depth = nullptr; int64_t vdepth_rows = 0; float* v_depths = nullptr;
    const float4* recs = nullptr;  // launch_pack_records output for the same inputs
    int32_t fold = 0;  // v_colors / v_opacity summed over the B_out images (n rows)
    uint32_t* dev_err = nullptr;  // the device's error word (DeviceScratch::tickets)
    PixelLoss loss;  // kind != kLossNone: the image cotangent from the fused loss, v_out unused
};
// order: scratch of B_out * num_tiles for the tile dispatch order; kept_order (may be null) is the
// order a forward over the same bins wrote, used instead when B_out == in.B_geom.
int launch_blend_bwd(const RasterInputs& in, const KeyLayout& lay, const int32_t* sorted_ids,
                     const int32_t* tile_bins, const BlendBwdArgs& a, int32_t* order,
                     const int32_t* kept_order, hipStream_t stream);

// ------------------------------------------------------------------ device helpers

// Records of the per-item gradient gather staged per LDS round (kGatherChunk * NG floats): 512
// keeps a workgroup's LDS at 18 KB, eight per CU (config 4's gather 0.39 -> 0.33 ms against 768).
constexpr int kGatherChunk = 512;

// Sums of the per-item gather kept in double: the conic and xy sums (slots 3..7), whose rounding
// the projection VJP multiplies by up to cond(conic)^2 on needle-thin items. The colour, opacity
// and depth sums (slots 0..2, 8, 9) add a few float rows each and stay in float.
__host__ __device__ constexpr bool gather_in_double(int k) { return k >= 3 && k <= 7; }

// Running per-item sums of rgrad rows: five in double, the others in float (gather_in_double).
template <int NG>
struct GatherSums {
    static constexpr int dslot(int k) { return k >= 3 && k <= 7 ? k - 3 : 0; }
    static constexpr int fslot(int k) { return k < 3 ? k : (k >= 8 ? k - 5 : 0); }
    double d[5];
    float f[NG - 5];
    __device__ __forceinline__ void clear() {
#pragma unroll
        for (int k = 0; k < 5; ++k) d[k] = 0.0;
#pragma unroll
        for (int k = 0; k < NG - 5; ++k) f[k] = 0.0f;
    }
    __device__ __forceinline__ void add_row(const float* r) {
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            if (gather_in_double(k))
                d[dslot(k)] += (double)r[k];
            else
                f[fslot(k)] += r[k];
        }
    }
    __device__ __forceinline__ void out(double* s) const {
#pragma unroll
        for (int k = 0; k < NG; ++k) s[k] = gather_in_double(k) ? d[dslot(k)] : (double)f[fslot(k)];
    }
};

// Per-item sums of NG floats over the item's emission range [my_lo, my_hi) of rgrad rows
// (row e at rgrad + (off + e) * NG), added in emission order (GatherSums). The workgroup's items
// cover one contiguous range [wg_lo, wg_hi) of rows (uniform over the workgroup), which is read
// with coalesced loads into s_buf (kGatherChunk * NG floats of LDS) a round at a time; each
// thread then adds its own rows from LDS. Every thread of the workgroup calls it (an item outside
// the workgroup's range passes my_lo = my_hi).
template <int NG, int kThreads>
__device__ __forceinline__ void block_gather(const float* __restrict__ rgrad, int64_t off,
                                             int64_t wg_lo, int64_t wg_hi, int64_t my_lo,
                                             int64_t my_hi, float* s_buf, double* s) {
    GatherSums<NG> acc;
    acc.clear();
    for (int64_t cs = wg_lo; cs < wg_hi; cs += kGatherChunk) {
        const int64_t ce = cs + kGatherChunk < wg_hi ? cs + kGatherChunk : wg_hi;
        const int nf = (int)((ce - cs) * NG);
        const float* src = rgrad + (off + cs) * NG;
        __syncthreads();  // the previous round's reads of s_buf are done
        for (int i0 = 0; i0 < nf; i0 += 4 * kThreads) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * kThreads + (int)threadIdx.x;
                v[u] = i < nf ? src[i] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * kThreads + (int)threadIdx.x;
                if (i < nf) s_buf[i] = v[u];
            }
        }
        __syncthreads();
        const int64_t a = my_lo > cs ? my_lo : cs, b = my_hi < ce ? my_hi : ce;
        for (int64_t e = a; e < b; ++e) acc.add_row(s_buf + (e - cs) * NG);
    }
    acc.out(s);
}

// Inclusive prefix sum over the 64 lanes (every lane active): DPP row shifts scan each row of 16,
// then row broadcasts add row 0's total into row 1 and row 2's into row 3, and the first two
// rows' total (lane 31) into rows 2 and 3. Lanes without a shift source add 0.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ int32_t dpp_scan_add(int32_t x) {
    return x + __builtin_amdgcn_update_dpp(0, x, kCtrl, kRowMask, 0xf, false);
}
__device__ __forceinline__ int32_t wave_inclusive_scan_i32(int32_t v, int /*lane*/) {
    v = dpp_scan_add<0x111, 0xf>(v);  // row_shr:1
    v = dpp_scan_add<0x112, 0xf>(v);  // row_shr:2
    v = dpp_scan_add<0x114, 0xf>(v);  // row_shr:4
    v = dpp_scan_add<0x118, 0xf>(v);  // row_shr:8
    v = dpp_scan_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_scan_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Block-wide min / max of one int32 per thread; `tmp` is LDS of >= 2 ints. All threads call.
__device__ __forceinline__ int32_t block_min_i32(int32_t v, int32_t* tmp) {
    __syncthreads();
    if (threadIdx.x == 0) tmp[0] = 2147483647;
    __syncthreads();
    atomicMin(tmp, v);
    __syncthreads();
    return tmp[0];
}
__device__ __forceinline__ int32_t block_max_i32(int32_t v, int32_t* tmp) {
    __syncthreads();
    if (threadIdx.x == 0) tmp[1] = (-2147483647 - 1);
    __syncthreads();
    atomicMax(tmp + 1, v);
    __syncthreads();
    return tmp[1];
}

}  // namespace splat
