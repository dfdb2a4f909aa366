// C-ABI entry points of libsplat_hip.so, the per-device scratch cache and stage timing.
//
// Scratch follows splax/_cache.py:52-90 (grow-only, 1.25x headroom, freed by clear_cache) but is
// owned by the library per device and guarded by a mutex (the reference leaned on Warp's FFI
// callback lock, splax/_cache.py:99). The intersection count is read through one pinned
// element and an event per device (splax/_cache.py:130-155). Calls from different host threads
// on one device are serialized; calls that overlap on different streams of one device share the
// scratch and must not run concurrently on the GPU.
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "../../include/splat_hip.h"
#include "splat_common.hpp"
#include "splat_internal.hpp"

namespace splat {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

// ------------------------------------------------------------------ fills

__global__ void fill_zero_f32_kernel(float* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}
__global__ void fill_zero_i32_kernel(int32_t* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

__global__ void widen_i32_kernel(const int32_t* a, int64_t* b, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        b[i] = a[i];
}

static unsigned fill_blocks(int64_t n) {
    int64_t b = (n + 255) / 256;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, 4096));
}

int fill_zero_f32(float* p, int64_t n, hipStream_t stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(fill_zero_f32_kernel, dim3(fill_blocks(n)), dim3(256), 0, stream, p, n);
    return hipGetLastError() == hipSuccess ? 0 : fail(kErrLaunch, "fill launch failed");
}
int fill_zero_i32(int32_t* p, int64_t n, hipStream_t stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(fill_zero_i32_kernel, dim3(fill_blocks(n)), dim3(256), 0, stream, p, n);
    return hipGetLastError() == hipSuccess ? 0 : fail(kErrLaunch, "fill launch failed");
}

// An operand is shared (rows == per) or batched (rows == per * B); the kernels index it as such,
// so any other row count would read outside it (splax/_project/_kernels.py:70-75).
static bool rows_match(int64_t rows, int64_t per, int64_t B) {
    return rows == per || rows == per * B;
}

// ------------------------------------------------------------------ scratch

constexpr int kMaxDevices = 64;
static DeviceScratch g_scratch[kMaxDevices];

template <typename T>
static int dev_alloc(T** p, int64_t count, bool zero) {
    void* q = nullptr;
    size_t bytes = (size_t)std::max<int64_t>(count, 1) * sizeof(T);
    if (hipMalloc(&q, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return fail(kErrAlloc, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    if (zero && hipMemset(q, 0, bytes) != hipSuccess) return fail(kErrAlloc, "hipMemset failed");
    *p = static_cast<T*>(q);
    return 0;
}
template <typename T>
static void dev_free(T** p) {
    if (*p) (void)hipFree(*p);
    *p = nullptr;
}

int DeviceScratch::ensure_base() {
    if (tickets) return 0;
    int rc = dev_alloc(&tickets, kNumTickets, true);
    if (!rc) rc = dev_alloc(&hist, kMaxPasses * 256, true);
    if (!rc) rc = dev_alloc(&chunk_sums, 4096, true);
    if (rc) return rc;
    chunk_sums_cap = 4096;
    void* h = nullptr;
    if (hipHostMalloc(&h, sizeof(int32_t), hipHostMallocDefault) != hipSuccess)
        return fail(kErrAlloc, "pinned readback allocation failed");
    pinned_count = static_cast<int32_t*>(h);
    void* hd = nullptr;
    if (hipHostGetDevicePointer(&hd, h, 0) != hipSuccess || !hd)
        return fail(kErrAlloc, "pinned readback mapping failed");
    pinned_count_dev = static_cast<int32_t*>(hd);
    if (hipEventCreateWithFlags(&count_event, hipEventDisableTiming) != hipSuccess)
        return fail(kErrRuntime, "event creation failed");
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        cus <= 0)
        return fail(kErrRuntime, "compute-unit count query failed");
    compute_units = cus;
    return 0;
}

// A host wait only when the stream changes: an event recorded after every call would put a
// barrier into every single-stream step (1.3% of the config-2 step).
int DeviceScratch::order_after_last(hipStream_t s) {
    if (has_last && s != last_stream && hipDeviceSynchronize() != hipSuccess)
        return fail(kErrRuntime, "device synchronize before a stream change failed");
    return 0;
}

void DeviceScratch::mark_done(hipStream_t s) {
    has_last = true;
    last_stream = s;
}

int DeviceScratch::grow_chunk_sums(int64_t blocks) {
    if (blocks <= chunk_sums_cap) return 0;
    (void)hipDeviceSynchronize();
    dev_free(&chunk_sums);
    int64_t cap = (int64_t)(blocks * 1.25) + 1;
    int rc = dev_alloc(&chunk_sums, cap, true);
    if (rc) {
        chunk_sums_cap = 0;
        return rc;
    }
    chunk_sums_cap = cap;
    return 0;
}

int DeviceScratch::ensure_sort(int64_t M, int64_t bins, int32_t B, bool wide) {
    const int64_t mm_blocks = 2 * (int64_t)B * 4096;  // generous partial capacity bound below
    bool need_sync = true;
    auto sync_once = [&]() {
        if (need_sync) {
            (void)hipDeviceSynchronize();
            need_sync = false;
        }
    };
    int rc = 0;
    if (M > isect_cap) {
        sync_once();
        for (int k = 0; k < 2; ++k) {
            dev_free(&keys[k]);
            dev_free(&vals[k]);
            dev_free(&gids[k]);
        }
        isect_cap = 0;
        int64_t cap = (int64_t)(M * 1.25) + 1;
        for (int k = 0; k < 2 && !rc; ++k) {
            rc = dev_alloc(&keys[k], cap, false);
            if (!rc) rc = dev_alloc(&vals[k], cap, false);
            if (!rc) rc = dev_alloc(&gids[k], cap, false);
        }
        if (rc) return rc;
        isect_cap = cap;
    }
    if (wide && M > wide_cap) {
        sync_once();
        for (int k = 0; k < 2; ++k) dev_free(&wkeys[k]);
        wide_cap = 0;
        const int64_t cap = (int64_t)(M * 1.25) + 1;
        for (int k = 0; k < 2 && !rc; ++k) rc = dev_alloc(&wkeys[k], cap, false);
        if (rc) return rc;
        wide_cap = cap;
    }
    const int64_t parts = (M + kSortTileMin - 1) / kSortTileMin;
    if (parts * 256 > part_counts_cap) {
        sync_once();
        dev_free(&part_counts);
        int64_t cap = (int64_t)(parts * 1.25 + 1) * 256;
        rc = dev_alloc(&part_counts, cap, false);
        if (rc) {
            part_counts_cap = 0;
            return rc;
        }
        part_counts_cap = cap;
    }
    if (2 * bins > bins_cap) {
        sync_once();
        dev_free(&tile_bins);
        rc = dev_alloc(&tile_bins, 2 * bins, true);
        if (rc) {
            bins_cap = 0;
            return rc;
        }
        bins_cap = 2 * bins;
    }
    if (2 * (int64_t)B > mm_cap) {
        sync_once();
        dev_free(&depth_mm);
        rc = dev_alloc(&depth_mm, 2 * (int64_t)B, true);
        if (rc) {
            mm_cap = 0;
            return rc;
        }
        mm_cap = 2 * (int64_t)B;
    }
    (void)mm_blocks;
    return 0;
}

int DeviceScratch::ensure_rgrad(int64_t count) {
    if (count <= rgrad_cap) return 0;
    (void)hipDeviceSynchronize();
    dev_free(&rgrad);
    rgrad_cap = 0;
    const int64_t cap = (int64_t)(count * 1.25) + 9;
    int rc = dev_alloc(&rgrad, cap, false);
    if (rc) return rc;
    rgrad_cap = cap;
    return 0;
}

int DeviceScratch::ensure_item_grads(int64_t items) {
    if (items <= item_grads_cap) return 0;
    (void)hipDeviceSynchronize();
    dev_free(&item_grads);
    item_grads_cap = 0;
    const int64_t cap = (int64_t)(items * 1.25) + 1;
    int rc = dev_alloc(&item_grads, 6 * cap, false);
    if (rc) return rc;
    item_grads_cap = cap;
    return 0;
}

int DeviceScratch::ensure_recs(int64_t items) {
    if (items <= recs_cap) return 0;
    (void)hipDeviceSynchronize();
    dev_free(&recs);
    recs_cap = 0;
    const int64_t cap = (int64_t)(items * 1.25) + 1;
    int rc = dev_alloc(&recs, 4 * cap, false);
    if (rc) return rc;
    recs_cap = cap;
    return 0;
}

int DeviceScratch::ensure_view_partials(int64_t count) {
    if (count <= view_partials_cap) return 0;
    (void)hipDeviceSynchronize();
    dev_free(&view_partials);
    view_partials_cap = 0;
    const int64_t cap = (int64_t)(count * 1.25) + 1;
    int rc = dev_alloc(&view_partials, cap, false);
    if (rc) return rc;
    view_partials_cap = cap;
    return 0;
}

int DeviceScratch::ensure_loss_partials(int64_t count) {
    if (count <= loss_partials_cap) return 0;
    (void)hipDeviceSynchronize();
    dev_free(&loss_partials);
    loss_partials_cap = 0;
    int rc = dev_alloc(&loss_partials, count, false);
    if (rc) return rc;
    loss_partials_cap = count;
    return 0;
}

int DeviceScratch::ensure_order(int64_t blocks) {
    if (blocks <= order_cap) return 0;
    (void)hipDeviceSynchronize();
    dev_free(&tile_order);
    order_cap = 0;
    int rc = dev_alloc(&tile_order, blocks, false);
    if (rc) return rc;
    order_cap = blocks;
    return 0;
}

static int ensure_minmax_partials(DeviceScratch& sc, int64_t count) {
    if (count <= sc.mm_partial_cap) return 0;
    (void)hipDeviceSynchronize();
    dev_free(&sc.mm_partial);
    int64_t cap = (int64_t)(count * 1.25) + 2;
    int rc = dev_alloc(&sc.mm_partial, cap, false);
    if (rc) {
        sc.mm_partial_cap = 0;
        return rc;
    }
    sc.mm_partial_cap = cap;
    return 0;
}

// A new workload signature drops every workload-sized buffer before the call grows what it
// needs, so a large render's buffers do not outlive it (the reference drops its whole scratch
// entry on a signature change, splax/_cache.py:61-75). The base buffers stay.
void DeviceScratch::workload(int32_t B, int32_t n, int32_t num_tiles) {
    if (B == sig_B && n == sig_n && num_tiles == sig_tiles) return;
    if (sig_B >= 0) release_sized();
    sig_B = B;
    sig_n = n;
    sig_tiles = num_tiles;
}

void DeviceScratch::release_sized() {
    (void)hipDeviceSynchronize();
    for (int k = 0; k < 2; ++k) {
        dev_free(&keys[k]);
        dev_free(&vals[k]);
        dev_free(&gids[k]);
        dev_free(&wkeys[k]);
    }
    isect_cap = 0;
    wide_cap = 0;
    dev_free(&rgrad);
    rgrad_cap = 0;
    dev_free(&recs);
    recs_cap = 0;
    dev_free(&item_grads);
    item_grads_cap = 0;
    dev_free(&tile_order);
    order_cap = 0;
    dev_free(&view_partials);
    view_partials_cap = 0;
    dev_free(&loss_partials);
    loss_partials_cap = 0;
    dev_free(&part_counts);
    part_counts_cap = 0;
    dev_free(&tile_bins);
    bins_cap = 0;
    dev_free(&depth_mm);
    mm_cap = 0;
    dev_free(&mm_partial);
    mm_partial_cap = 0;
    dev_free(&chunk_sums);
    chunk_sums_cap = 0;
    last_count = -1;
}

void DeviceScratch::release() {
    if (!tickets && !keys[0] && !tile_bins) return;
    release_sized();
    sig_B = sig_n = sig_tiles = -1;
    dev_free(&tickets);
    dev_free(&hist);
    if (pinned_count) (void)hipHostFree(pinned_count);
    pinned_count = nullptr;
    pinned_count_dev = nullptr;
    if (count_event) (void)hipEventDestroy(count_event);
    count_event = nullptr;
    has_last = false;
    last_stream = nullptr;
}

DeviceScratch& scratch_for_current_device() {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev < 0 || dev >= kMaxDevices) dev = 0;
    g_scratch[dev].device = dev;
    return g_scratch[dev];
}

void release_all_scratch() {
    int cur = 0;
    (void)hipGetDevice(&cur);
    for (int d = 0; d < kMaxDevices; ++d) {
        DeviceScratch& sc = g_scratch[d];
        std::lock_guard<std::mutex> lock(sc.mu);
        if (sc.device < 0) continue;
        if (hipSetDevice(d) != hipSuccess) continue;
        sc.release();
    }
    (void)hipSetDevice(cur);
}

// ------------------------------------------------------------------ stage timing

static std::mutex g_timing_mu;
static uint32_t g_timing_mask = 0;  // bit s set: stage s is bracketed by events
struct TimedSpan {
    int stage;
    hipEvent_t a, b;
};
static std::vector<TimedSpan> g_spans;
static std::vector<hipEvent_t> g_event_pool;

static hipEvent_t take_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);
    return e;
}

bool kernel_timer_events(int stage, hipEvent_t* start, hipEvent_t* end) {
    std::lock_guard<std::mutex> lock(g_timing_mu);
    *start = *end = nullptr;
    if (!((g_timing_mask >> stage) & 1u)) return false;
    *start = take_event();
    *end = take_event();
    g_spans.push_back({stage, *start, *end});
    return true;
}

StageTimer::StageTimer(hipStream_t s, int st) : stream(s), stage(st) {
    std::lock_guard<std::mutex> lock(g_timing_mu);
    if (!((g_timing_mask >> st) & 1u)) return;
    start = take_event();
    (void)hipEventRecord(start, stream);
}

StageTimer::~StageTimer() {
    std::lock_guard<std::mutex> lock(g_timing_mu);
    if (!start) return;
    hipEvent_t end = take_event();
    (void)hipEventRecord(end, stream);
    g_spans.push_back({stage, start, end});
}

}  // namespace splat

using namespace splat;

static double g_stage_ms[kNumStages];
static int64_t g_stage_calls[kNumStages];

extern "C" {

int splat_abi_version(void) { return 17; }

int splat_check_device(void) {
    DeviceScratch& sc = scratch_for_current_device();
    std::lock_guard<std::mutex> lock(sc.mu);
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    if (!sc.tickets) return 0;
    uint32_t word = 0;
    if (hipMemcpy(&word, sc.tickets + kDeviceError, sizeof(word), hipMemcpyDeviceToHost) !=
        hipSuccess)
        return -1;
    if (word) {
        uint32_t zero = 0;
        (void)hipMemcpy(sc.tickets + kDeviceError, &zero, sizeof(zero), hipMemcpyHostToDevice);
    }
    return (int)word;
}

const char* splat_last_error(void) { return g_last_error.c_str(); }

void splat_clear_cache(void) {
    release_all_scratch();
    release_train_scratch();
}

int splat_set_stage_timing(int stage_mask) {
    std::lock_guard<std::mutex> lock(g_timing_mu);
    g_timing_mask = (uint32_t)stage_mask & ((1u << kNumStages) - 1u);
    return 0;
}

int splat_get_stage_times(double* ms, int64_t* calls, int32_t n) {
    std::lock_guard<std::mutex> lock(g_timing_mu);
    for (auto& s : g_spans) {
        if (hipEventSynchronize(s.b) != hipSuccess) return fail(kErrRuntime, "event sync failed");
        float t = 0.f;
        (void)hipEventElapsedTime(&t, s.a, s.b);
        g_stage_ms[s.stage] += t;
        g_stage_calls[s.stage] += 1;
        g_event_pool.push_back(s.a);
        g_event_pool.push_back(s.b);
    }
    g_spans.clear();
    for (int k = 0; k < n && k < kNumStages; ++k) {
        if (ms) ms[k] = g_stage_ms[k];
        if (calls) calls[k] = g_stage_calls[k];
    }
    for (int k = 0; k < kNumStages; ++k) {
        g_stage_ms[k] = 0.0;
        g_stage_calls[k] = 0;
    }
    return 0;
}

}  // extern "C"

// Validates splat_project_fwd's arguments and fills its argument bundle (shared with the
// no-allocation variant).
static int project_fwd_args(const float* means3d, int64_t rows_means, const float* scales,
                            int64_t rows_scales, const float* quats, int64_t rows_quats,
                            const float* viewmat, int64_t rows_viewmat, const float* opacities,
                            int64_t rows_opac, const float* transforms, int64_t rows_transforms,
                            const int32_t* transform_ids, int32_t num_gaussians,
                            int32_t num_transforms, int32_t has_transforms, int64_t total,
                            int32_t img_h, int32_t img_w, float fx, float fy, float cx, float cy,
                            float glob_scale, float clip_thresh, float* xys, float* depths,
                            int32_t* radii, float* conics, int32_t* num_tiles_hit,
                            int32_t* cum_tiles_hit, int32_t quats_wxyz, ProjectArgs* out) {
    if (num_gaussians <= 0 || total < 0 || total % num_gaussians != 0 || img_h <= 0 ||
        img_w <= 0)
        return fail(kErrArgs, "project_fwd: invalid sizes");
    const int64_t B = total / num_gaussians;
    if (!rows_match(rows_means, num_gaussians, B) || !rows_match(rows_scales, num_gaussians, B) ||
        !rows_match(rows_quats, num_gaussians, B) || !rows_match(rows_opac, num_gaussians, B) ||
        !rows_match(rows_viewmat, 4, B))
        return fail(kErrArgs, "project_fwd: operand rows must be num_gaussians (shared) or "
                              "B * num_gaussians (batched); viewmat 4 or 4 * B");
    if (has_transforms && (num_transforms <= 0 || !transforms || !transform_ids ||
                           !rows_match(rows_transforms, num_transforms, B)))
        return fail(kErrArgs, "project_fwd: transforms requested but not given (or rows not "
                              "num_transforms / B * num_transforms)");
    if (total >= ((int64_t)1 << 31))
        return fail(kErrArgs, "project_fwd: more than 2^31 items");
    if (total > 0 && (!means3d || !scales || !quats || !viewmat || !opacities || !xys ||
                      !depths || !radii || !conics || !num_tiles_hit || !cum_tiles_hit))
        return fail(kErrArgs, "project_fwd: missing input or output buffer");
    // xys rows are stored as one 8-byte vector each
    if ((uintptr_t)xys & 7) return fail(kErrArgs, "project_fwd: xys must be 8-byte aligned");
    ProjectArgs& a = *out;
    a.means = means3d; a.rows_means = rows_means;
    a.scales = scales; a.rows_scales = rows_scales;
    a.quats = quats; a.rows_quats = rows_quats;
    a.viewmat = viewmat; a.rows_viewmat = rows_viewmat;
    a.opacities = opacities; a.rows_opac = rows_opac;
    a.transforms = transforms; a.rows_transforms = has_transforms ? rows_transforms : 0;
    a.transform_ids = transform_ids;
    a.n = num_gaussians; a.num_transforms = has_transforms ? num_transforms : 1;
    a.has_transforms = has_transforms;
    a.total = total; a.img_h = img_h; a.img_w = img_w;
    a.fx = fx; a.fy = fy; a.cx = cx; a.cy = cy;
    a.glob_scale = glob_scale; a.clip_thresh = clip_thresh;
    a.xys = xys; a.depths = depths; a.radii = radii; a.conics = conics;
    a.num_tiles_hit = num_tiles_hit; a.cum_tiles_hit = cum_tiles_hit;
    a.quats_wxyz = quats_wxyz != 0;
    return 0;
}

extern "C" {

int splat_project_fwd(splat_stream_t stream, const float* means3d, int64_t rows_means,
                      const float* scales, int64_t rows_scales, const float* quats,
                      int64_t rows_quats, const float* viewmat, int64_t rows_viewmat,
                      const float* opacities, int64_t rows_opac, const float* transforms,
                      int64_t rows_transforms, const int32_t* transform_ids,
                      int32_t num_gaussians, int32_t num_transforms, int32_t has_transforms,
                      int64_t total, int32_t img_h, int32_t img_w, float fx, float fy, float cx,
                      float cy, float glob_scale, float clip_thresh, float* xys, float* depths,
                      int32_t* radii, float* conics, int32_t* num_tiles_hit,
                      int32_t* cum_tiles_hit, int32_t quats_wxyz) {
    ProjectArgs a;
    int rc = project_fwd_args(means3d, rows_means, scales, rows_scales, quats, rows_quats,
                              viewmat, rows_viewmat, opacities, rows_opac, transforms,
                              rows_transforms, transform_ids, num_gaussians, num_transforms,
                              has_transforms, total, img_h, img_w, fx, fy, cx, cy, glob_scale,
                              clip_thresh, xys, depths, radii, conics, num_tiles_hit,
                              cum_tiles_hit, quats_wxyz, &a);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    DeviceScratch& sc = scratch_for_current_device();
    ScratchUse use(sc, s);
    rc = use.rc;
    if (rc) return rc;
    StageTimer tm(s, kStageProject);
    g_last_error.clear();
    rc = launch_project_fwd(a, sc, s);
    if (rc && g_last_error.empty())  // launchers that name their failure set the message
        set_error("project_fwd launch failed");
    return rc;
}

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
                              int32_t quats_wxyz) {
    ProjectArgs a;
    int rc = project_fwd_args(means3d, rows_means, scales, rows_scales, quats, rows_quats,
                              viewmat, rows_viewmat, opacities, rows_opac, transforms,
                              rows_transforms, transform_ids, num_gaussians, num_transforms,
                              has_transforms, total, img_h, img_w, fx, fy, cx, cy, glob_scale,
                              clip_thresh, xys, depths, radii, conics, num_tiles_hit,
                              cum_tiles_hit, quats_wxyz, &a);
    if (rc) return rc;
    if (project_fwd_chunks(total) > kNoAllocMaxChunks)
        return fail(kErrArgs, "project_fwd_noalloc: more than " +
                                  std::to_string(kNoAllocMaxChunks * 1024) +
                                  " items (the size of its fixed scratch)");
    // no library scratch, stage timer or stream bookkeeping: nothing here allocates
    g_last_error.clear();
    rc = launch_project_fwd_noalloc(a, static_cast<hipStream_t>(stream));
    if (rc && g_last_error.empty()) set_error("project_fwd_noalloc launch failed");
    return rc;
}

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
                      int32_t quats_wxyz, int32_t fold_shared) {
    if (num_gaussians <= 0 || B <= 0) return fail(kErrArgs, "project_bwd: invalid sizes");
    if (!rows_match(rows_means, num_gaussians, B) || !rows_match(rows_scales, num_gaussians, B) ||
        !rows_match(rows_quats, num_gaussians, B) || !rows_match(rows_viewmat, 4, B) ||
        !rows_match(rows_radii, num_gaussians, B) || !rows_match(rows_conics, num_gaussians, B) ||
        !rows_match(rows_vxy, num_gaussians, B) || !rows_match(rows_vconic, num_gaussians, B) ||
        (v_depth && !rows_match(rows_vdepth, num_gaussians, B)))
        return fail(kErrArgs, "project_bwd: operand rows must be num_gaussians (shared) or "
                              "B * num_gaussians (batched); viewmat 4 or 4 * B");
    if (has_transforms && (num_transforms <= 0 || !transforms || !transform_ids ||
                           !v_transforms || !rows_match(rows_transforms, num_transforms, B)))
        return fail(kErrArgs, "project_bwd: transforms requested but not given");
    if ((int64_t)B * num_gaussians >= ((int64_t)1 << 31))
        return fail(kErrArgs, "project_bwd: more than 2^31 items");
    if (!means3d || !scales || !quats || !viewmat || !radii || !conics || !v_xy || !v_conic ||
        !v_mean3d || !v_scale || !v_quat)
        return fail(kErrArgs, "project_bwd: missing input or output buffer");
    if (fold_shared && (rows_means != num_gaussians || rows_scales != num_gaussians ||
                        rows_quats != num_gaussians))
        return fail(kErrArgs, "project_bwd: folding needs shared means, scales and quats");
    // v_quat rows are stored as one 16-byte vector each
    if ((uintptr_t)v_quat & 15)
        return fail(kErrArgs, "project_bwd: v_quat must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    ProjectBwdArgs a;
    a.means = means3d; a.rows_means = rows_means;
    a.scales = scales; a.rows_scales = rows_scales;
    a.quats = quats; a.rows_quats = rows_quats;
    a.viewmat = viewmat; a.rows_viewmat = rows_viewmat;
    a.radii = radii; a.rows_radii = rows_radii;
    a.conics = conics; a.rows_conics = rows_conics;
    a.v_xy = v_xy; a.rows_vxy = rows_vxy;
    a.v_depth = v_depth; a.rows_vdepth = rows_vdepth;
    a.v_conic = v_conic; a.rows_vconic = rows_vconic;
    a.transforms = transforms; a.rows_transforms = has_transforms ? rows_transforms : 0;
    a.transform_ids = transform_ids;
    a.n = num_gaussians; a.num_transforms = has_transforms ? num_transforms : 0;
    a.has_transforms = has_transforms; a.B = B;
    a.fx = fx; a.fy = fy; a.glob_scale = glob_scale;
    a.v_mean3d = v_mean3d; a.v_scale = v_scale; a.v_quat = v_quat;
    a.v_viewmat = v_viewmat; a.v_transforms = has_transforms ? v_transforms : nullptr;
    a.quats_wxyz = quats_wxyz != 0;
    a.fold = fold_shared != 0;
    DeviceScratch& sc = scratch_for_current_device();
    ScratchUse use(sc, s);
    int rc = use.rc;
    if (rc) return rc;
    StageTimer tm(s, kStageProjectBwd);
    g_last_error.clear();
    rc = launch_project_bwd(a, sc, s);
    if (rc && g_last_error.empty())  // launchers that name their failure set the message
        set_error("project_bwd launch failed");
    return rc;
}

// blend: the call blends (colours, opacities and background are read), not only sorts.
static int check_raster(const RasterInputs& in, int32_t B_out, bool blend = true) {
    if (in.n <= 0 || in.B_geom <= 0 || in.img_h <= 0 || in.img_w <= 0)
        return fail(kErrArgs, "rasterize: invalid sizes");
    // xys rows are read as one 8-byte vector each
    if ((uintptr_t)in.xys & 7) return fail(kErrArgs, "rasterize: xys must be 8-byte aligned");
    if (in.rows_colors < in.n || in.rows_opac < in.n || in.rows_map_opac < in.n ||
        in.rows_bg < 1)
        return fail(kErrArgs, "rasterize: operand has fewer rows than num_gaussians");
    // the background is indexed per output image when it has more than one row
    if (in.rows_bg > 1 && in.rows_bg < B_out)
        return fail(kErrArgs, "rasterize: background needs 1 or B rows");
    if ((int64_t)in.B_geom * in.n >= ((int64_t)1 << 31))
        return fail(kErrArgs, "rasterize: more than 2^31 items");
    if (!in.map_opac || !in.xys || !in.conics || !in.cum ||
        (blend && (!in.colors || !in.opac || !in.background)))
        return fail(kErrArgs, "rasterize: missing input buffer");
    return 0;
}

int splat_set_wide_keys(int force) {
    set_force_wide_keys(force != 0);
    return 0;
}

int splat_sort_and_bin(splat_stream_t stream, const float* xys, const float* depths,
                       const int32_t* radii, const float* conics, const float* map_opacities,
                       int64_t rows_map_opac, const int32_t* cum_tiles_hit,
                       int32_t num_gaussians, int32_t B, int32_t img_h, int32_t img_w,
                       int64_t* sorted_keys, int32_t* sorted_ids, int64_t capacity,
                       int32_t* tile_bins, int64_t* num_intersects) {
    RasterInputs in{};
    in.colors = nullptr; in.rows_colors = num_gaussians;
    in.opac = nullptr; in.rows_opac = num_gaussians;
    in.map_opac = map_opacities; in.rows_map_opac = rows_map_opac;
    in.background = nullptr; in.rows_bg = 1;
    in.xys = xys; in.depths = depths; in.radii = radii; in.conics = conics;
    in.cum = cum_tiles_hit; in.n = num_gaussians; in.B_geom = B;
    in.img_h = img_h; in.img_w = img_w;
    int rc = check_raster(in, B, false);
    if (rc) return rc;
    if (!depths || !radii || !tile_bins || (capacity > 0 && (!sorted_keys || !sorted_ids)))
        return fail(kErrArgs, "sort_and_bin: missing input or output buffer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    DeviceScratch& sc = scratch_for_current_device();
    ScratchUse use(sc, s);
    rc = use.rc;
    if (!rc) {
        sc.workload(B, num_gaussians, key_layout(B, img_h, img_w).num_tiles);
        const int32_t bpi = (num_gaussians + 4095) / 4096;
        rc = ensure_minmax_partials(sc, 2 * (int64_t)bpi * B);
    }
    if (rc) return rc;
    int64_t M = 0;
    KeyLayout L;
    SortOutputs o;
    rc = run_sort_and_bin(in, sc, s, &M, &L, nullptr, &o, true);
    if (num_intersects) *num_intersects = M;
    if (rc) return rc;
    if (M > capacity) return fail(kErrTooMany, "sort_and_bin: capacity below intersection count");
    const int64_t nb = 2 * (int64_t)B * L.num_tiles;
    if (hipMemcpyAsync(tile_bins, o.bins, nb * sizeof(int32_t), hipMemcpyDeviceToDevice, s) !=
        hipSuccess)
        return fail(kErrRuntime, "bins copy failed");
    if (M > 0) {
        if (o.wide) {
            if (hipMemcpyAsync(sorted_keys, o.keys, M * sizeof(int64_t), hipMemcpyDeviceToDevice,
                               s) != hipSuccess)
                return fail(kErrRuntime, "sorted copy failed");
        } else {
            hipLaunchKernelGGL(widen_i32_kernel, dim3(fill_blocks(M)), dim3(256), 0, s,
                               static_cast<const int32_t*>(o.keys), sorted_keys, M);
            if (hipGetLastError() != hipSuccess) return fail(kErrLaunch, "key copy failed");
        }
        if (hipMemcpyAsync(sorted_ids, o.ids, M * sizeof(int32_t), hipMemcpyDeviceToDevice, s) !=
            hipSuccess)
            return fail(kErrRuntime, "sorted copy failed");
    }
    return 0;
}

static RasterInputs raster_inputs(const float* colors, int64_t rows_colors,
                                  const float* opacities, int64_t rows_opac,
                                  const float* map_opacities, int64_t rows_map_opac,
                                  const float* background, int64_t rows_bg, const float* xys,
                                  const float* depths, const int32_t* radii, const float* conics,
                                  const int32_t* cum, int32_t n, int32_t B_geom, int32_t img_h,
                                  int32_t img_w) {
    RasterInputs in{};
    in.colors = colors; in.rows_colors = rows_colors;
    in.opac = opacities; in.rows_opac = rows_opac;
    in.map_opac = map_opacities; in.rows_map_opac = rows_map_opac;
    in.background = background; in.rows_bg = rows_bg;
    in.xys = xys; in.depths = depths; in.radii = radii; in.conics = conics;
    in.cum = cum; in.n = n; in.B_geom = B_geom;
    in.img_h = img_h; in.img_w = img_w;
    return in;
}

// Forward: sort_and_bin into the library scratch or the caller's kept lists (tgt), then the
// blend; out_depth non-null adds the expected-depth channel.
// records / order: caller buffers for the packed blend records and the tile dispatch order
// (kept for the backward), or null for library scratch.
static int rasterize_fwd_core(hipStream_t s, DeviceScratch& sc, const RasterInputs& in,
                              const SortTargets* tgt, float* final_Ts, int32_t* final_idx,
                              float* out_img, float* out_depth, float* records, int32_t* order,
                              int64_t* num_intersects, bool packed,
                              const PixelLoss* loss = nullptr, float* loss_out = nullptr);

static int rasterize_fwd_impl(hipStream_t s, const RasterInputs& in, const SortTargets* tgt,
                              float* final_Ts, int32_t* final_idx, float* out_img,
                              float* out_depth, float* records, int32_t* order,
                              int64_t* num_intersects) {
    int rc = check_raster(in, in.B_geom);
    if (rc) return rc;
    if (!out_img) return fail(kErrArgs, "rasterize: missing image output");
    if (!in.depths || !in.radii) return fail(kErrArgs, "rasterize: missing input buffer");
    DeviceScratch& sc = scratch_for_current_device();
    ScratchUse use(sc, s);
    rc = use.rc;
    if (rc) return rc;
    return rasterize_fwd_core(s, sc, in, tgt, final_Ts, final_idx, out_img, out_depth, records,
                              order, num_intersects, false);
}

// The forward with the device's scratch held: sort_and_bin (into tgt's buffers when given), the
// record pack (skipped when packed: the fused projection wrote them into records) and the blend.
// With a capacity-bounded tgt the count is settled after the blend's launch (the host waits only
// there, by when the stream is normally well past the count's copy). loss (may be null): a loss
// fused into the blend, its value into *loss_out.
static int rasterize_fwd_core(hipStream_t s, DeviceScratch& sc, const RasterInputs& in,
                              const SortTargets* tgt, float* final_Ts, int32_t* final_idx,
                              float* out_img, float* out_depth, float* records, int32_t* order,
                              int64_t* num_intersects, bool packed, const PixelLoss* loss,
                              float* loss_out) {
    int rc = 0;
    sc.workload(in.B_geom, in.n, key_layout(in.B_geom, in.img_h, in.img_w).num_tiles);
    {
        const int32_t bpi = (in.n + 4095) / 4096;
        rc = ensure_minmax_partials(sc, 2 * (int64_t)bpi * in.B_geom);
    }
    if (rc) return rc;
    int64_t M = 0;
    KeyLayout L;
    SortOutputs o;
    rc = run_sort_and_bin(in, sc, s, &M, &L, tgt, &o);
    if (num_intersects && M >= 0) *num_intersects = M;
    if (rc) return rc;
    // with a deferred count M is its bound (the capacity) until settled
    const bool deferred = o.count_deferred;
    if (deferred) M = tgt->capacity;
    const int32_t* ids = o.ids;
    const int32_t* bins = o.bins;
    float4* recs = reinterpret_cast<float4*>(records);
    if (!recs) {
        rc = sc.ensure_recs((int64_t)in.B_geom * in.n);
        if (rc) return rc;
        recs = sc.recs;
    }
    if (!order) {
        rc = sc.ensure_order((int64_t)in.B_geom * L.num_tiles);
        if (rc) return rc;
        order = sc.tile_order;
    }
    const int64_t blocks = (int64_t)in.B_geom * L.num_tiles;
    PixelLoss lp;
    if (loss) {
        rc = sc.ensure_loss_partials(blocks);
        if (rc) return rc;
        lp = *loss;
        lp.partials = sc.loss_partials;
    }
    {
        StageTimer tm(s, kStageBlendFwd);
        if (M > 0 && !packed) rc = launch_pack_records(in, recs, s);
        if (!rc)
            rc = launch_blend_fwd(in, L, M > 0 ? ids : nullptr, bins, final_Ts, final_idx,
                                  out_img, out_depth, recs, order, loss ? &lp : nullptr, s);
    }
    // the loss's final sum is not part of the blend stage's timing
    if (!rc && loss) rc = launch_loss_final(lp.partials, blocks, loss->count, loss_out, s);
    if (rc) return fail(rc, "blend_fwd launch failed");
    if (deferred) {
        int64_t count = 0;
        rc = settle_count(sc, tgt->capacity, &count);
        if (num_intersects) *num_intersects = count;
        return rc;
    }
    return 0;
}

// Sorted lists (and, when non-null, the packed records and the tile order) kept from the
// forward (splat_rasterize_fwd_keep).
struct KeptLists {
    const int32_t* ids; const int32_t* pos; const int32_t* bins; int64_t M;
    const float* records; const int32_t* order;
};

// Backward over kept sorted lists or, with kept == nullptr, over a fresh sort_and_bin.
// v_depths non-null selects the depth channel.
static int check_raster_bwd(const RasterInputs& in, const BlendBwdArgs& args) {
    int rc = check_raster(in, args.B_out);
    if (rc) return rc;
    if (args.B_out <= 0 || (in.B_geom > 1 && in.B_geom != args.B_out))
        return fail(kErrArgs, "rasterize_bwd: B_geom must be 1 or equal to B_out");
    if (args.vout_rows <= 0 || !in.cum) return fail(kErrArgs, "rasterize_bwd: empty cotangent");
    // a forward-only render may leave its final buffers out: the backward needs both
    const bool fused_loss = args.loss.kind != kLossNone;
    if (!args.final_Ts || !args.final_idx || (!args.v_out && !fused_loss))
        return fail(kErrArgs, "rasterize_bwd: final_Ts, final_idx and the image cotangent are "
                              "required");
    if (fused_loss && (!args.loss.target || !args.loss.img || !args.loss.v_loss))
        return fail(kErrArgs, "render_bwd: a fused loss needs the target, the forward's image "
                              "and the loss cotangent");
    if (args.v_depths && (!in.depths || !args.v_out_depth || args.vdepth_rows <= 0))
        return fail(kErrArgs, "rasterize_bwd: depth channel needs depths and v_out_depth");
    if ((int64_t)args.B_out * in.n >= ((int64_t)1 << 31))
        return fail(kErrArgs, "rasterize_bwd: more than 2^31 gradient rows");
    if (!args.v_colors || !args.v_opacity)
        return fail(kErrArgs, "rasterize_bwd: missing gradient output");
    return 0;
}

static int rasterize_bwd_core(hipStream_t s, DeviceScratch& sc, const RasterInputs& in,
                              const KeptLists* kept, const BlendBwdArgs& args);

static int rasterize_bwd_impl(hipStream_t s, const RasterInputs& in, const KeptLists* kept,
                              const BlendBwdArgs& args) {
    int rc = check_raster_bwd(in, args);
    if (rc) return rc;
    if (!args.v_xy || !args.v_conic)
        return fail(kErrArgs, "rasterize_bwd: missing gradient output");
    DeviceScratch& sc = scratch_for_current_device();
    ScratchUse use(sc, s);
    rc = use.rc;
    if (rc) return rc;
    return rasterize_bwd_core(s, sc, in, kept, args);
}

// The backward with the device's scratch held.
static int rasterize_bwd_core(hipStream_t s, DeviceScratch& sc, const RasterInputs& in,
                              const KeptLists* kept, const BlendBwdArgs& args) {
    int rc = 0;
    sc.workload(in.B_geom, in.n, key_layout(in.B_geom, in.img_h, in.img_w).num_tiles);
    KeyLayout L;
    const int32_t* ids = nullptr;
    const int32_t* pos = nullptr;
    const int32_t* bins = nullptr;
    int64_t M = 0;
    if (kept) {
        L = key_layout(in.B_geom, in.img_h, in.img_w);
        if (L.overflow) return fail(kErrKeyOverflow, "rasterize_bwd: intersection key overflow");
        ids = kept->ids;
        pos = kept->pos;
        bins = kept->bins;
        M = kept->M;
    } else {
        const int32_t bpi = (in.n + 4095) / 4096;
        rc = ensure_minmax_partials(sc, 2 * (int64_t)bpi * in.B_geom);
        if (rc) return rc;
        SortOutputs o;
        rc = run_sort_and_bin(in, sc, s, &M, &L, nullptr, &o);
        if (rc) return rc;
        ids = o.ids;
        pos = o.pos;
        bins = o.bins;
    }
    const int64_t images = in.B_geom > 1 ? 1 : args.B_out;
    const float4* recs = kept ? reinterpret_cast<const float4*>(kept->records) : nullptr;
    rc = sc.ensure_rgrad(images * M * (args.v_depths ? 10 : 9));
    if (!rc && !recs && M > 0) rc = sc.ensure_recs((int64_t)in.B_geom * in.n);
    if (!rc) rc = sc.ensure_order((int64_t)args.B_out * L.num_tiles);
    if (rc) return rc;
    BlendBwdArgs a = args;
    a.sorted_pos = pos;
    a.M = M;
    a.rgrad = sc.rgrad;
    a.dev_err = sc.tickets + kDeviceError;
    StageTimer tm(s, kStageBlendBwd);
    if (!recs && M > 0) {
        rc = launch_pack_records(in, sc.recs, s);
        if (rc) return fail(rc, "pack_records launch failed");
        recs = sc.recs;
    }
    a.recs = recs;
    if (M == 1) {
        // a lone intersection's bin stays [0, 0) (the reference's bin-edge rule): no blend
        // workgroup visits it, so its partial sums are zero rather than what the slot last held
        rc = fill_zero_i32(reinterpret_cast<int32_t*>(a.rgrad), images * (a.v_depths ? 10 : 9),
                           s);
        if (rc) return rc;
    }
    rc = launch_blend_bwd(in, L, M > 0 ? ids : nullptr, bins, a, sc.tile_order,
                          kept ? kept->order : nullptr, s);
    if (rc) return fail(rc, "blend_bwd launch failed");
    return 0;
}

static BlendBwdArgs bwd_args(const float* final_Ts, const int32_t* final_idx,
                             const float* v_out_img, int64_t vout_rows, int32_t B_out,
                             float* v_colors, float* v_opacity, float* v_xy, float* v_conic,
                             const float* v_out_depth, int64_t vdepth_rows, float* v_depths) {
    BlendBwdArgs a;
    a.final_Ts = final_Ts; a.final_idx = final_idx;
    a.v_out = v_out_img; a.vout_rows = vout_rows; a.B_out = B_out;
    a.sorted_pos = nullptr; a.M = 0; a.rgrad = nullptr;
    a.v_colors = v_colors; a.v_opacity = v_opacity; a.v_xy = v_xy; a.v_conic = v_conic;
    a.v_out_depth = v_out_depth; a.vdepth_rows = vdepth_rows; a.v_depths = v_depths;
    return a;
}

int splat_rasterize_fwd(splat_stream_t stream, const float* colors, int64_t rows_colors,
                        const float* opacities, int64_t rows_opac, const float* map_opacities,
                        int64_t rows_map_opac, const float* background, int64_t rows_bg,
                        const float* xys, const float* depths, const int32_t* radii,
                        const float* conics, const int32_t* cum_tiles_hit,
                        int32_t num_gaussians, int32_t B, int32_t img_h, int32_t img_w,
                        float* final_Ts, int32_t* final_idx, float* out_img,
                        int64_t* num_intersects) {
    const RasterInputs in = raster_inputs(colors, rows_colors, opacities, rows_opac,
                                          map_opacities, rows_map_opac, background, rows_bg, xys,
                                          depths, radii, conics, cum_tiles_hit, num_gaussians, B,
                                          img_h, img_w);
    return rasterize_fwd_impl(static_cast<hipStream_t>(stream), in, nullptr, final_Ts,
                              final_idx, out_img, nullptr, nullptr, nullptr, num_intersects);
}

int splat_rasterize_depth_fwd(splat_stream_t stream, const float* colors, int64_t rows_colors,
                              const float* opacities, int64_t rows_opac,
                              const float* map_opacities, int64_t rows_map_opac,
                              const float* background, int64_t rows_bg, const float* xys,
                              const float* depths, const int32_t* radii, const float* conics,
                              const int32_t* cum_tiles_hit, int32_t num_gaussians, int32_t B,
                              int32_t img_h, int32_t img_w, float* final_Ts, int32_t* final_idx,
                              float* out_img, float* out_depth, int64_t* num_intersects) {
    if (!out_depth) return fail(kErrArgs, "rasterize_depth_fwd: out_depth missing");
    const RasterInputs in = raster_inputs(colors, rows_colors, opacities, rows_opac,
                                          map_opacities, rows_map_opac, background, rows_bg, xys,
                                          depths, radii, conics, cum_tiles_hit, num_gaussians, B,
                                          img_h, img_w);
    return rasterize_fwd_impl(static_cast<hipStream_t>(stream), in, nullptr, final_Ts,
                              final_idx, out_img, out_depth, nullptr, nullptr, num_intersects);
}

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
                             int32_t compensate) {
    if (capacity < 0 || !tile_bins || (capacity > 0 && (!sorted_ids || !sorted_pos)))
        return fail(kErrArgs, "rasterize_fwd_keep: missing sorted-list buffers");
    if ((uintptr_t)records & 15)
        return fail(kErrArgs, "rasterize_fwd_keep: records must be 16-byte aligned");
    const RasterInputs in = raster_inputs(colors, rows_colors, opacities, rows_opac,
                                          map_opacities, rows_map_opac, background, rows_bg, xys,
                                          depths, radii, conics, cum_tiles_hit, num_gaussians, B,
                                          img_h, img_w);
    RasterInputs inc = in;
    inc.compensate = compensate != 0;
    SortTargets tgt;
    tgt.capacity = capacity;
    tgt.ids = sorted_ids;
    tgt.pos = sorted_pos;
    tgt.bins = tile_bins;
    return rasterize_fwd_impl(static_cast<hipStream_t>(stream), inc, &tgt, final_Ts, final_idx,
                              out_img, out_depth, records, tile_order, num_intersects);
}

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
                               int32_t compensate, int32_t fold_shared) {
    if (num_intersects < 0 || !tile_bins ||
        (num_intersects > 0 && (!sorted_ids || !sorted_pos)))
        return fail(kErrArgs, "rasterize_bwd_sorted: invalid sorted lists");
    if ((uintptr_t)records & 15)
        return fail(kErrArgs, "rasterize_bwd_sorted: records must be 16-byte aligned");
    RasterInputs in = raster_inputs(colors, rows_colors, opacities, rows_opac, opacities,
                                    rows_opac, background, rows_bg, xys, depths, nullptr, conics,
                                    cum_tiles_hit, num_gaussians, B_geom, img_h, img_w);
    in.compensate = compensate != 0;
    if (fold_shared && (rows_colors != num_gaussians || rows_opac != num_gaussians))
        return fail(kErrArgs, "rasterize_bwd_sorted: folding needs shared colors and opacities");
    BlendBwdArgs a = bwd_args(final_Ts, final_idx, v_out_img, vout_rows, B_out, v_colors,
                              v_opacity, v_xy, v_conic, v_out_depth, vdepth_rows, v_depths);
    a.fold = fold_shared != 0;
    const KeptLists kept{sorted_ids, sorted_pos, tile_bins, num_intersects, records, tile_order};
    return rasterize_bwd_impl(static_cast<hipStream_t>(stream), in, &kept, a);
}

int splat_rasterize_bwd(splat_stream_t stream, const float* colors, int64_t rows_colors,
                        const float* opacities, int64_t rows_opac, const float* map_opacities,
                        int64_t rows_map_opac, const float* background, int64_t rows_bg,
                        const float* xys, const float* depths, const int32_t* radii,
                        const float* conics, const int32_t* cum_tiles_hit,
                        const float* final_Ts, const int32_t* final_idx, const float* v_out_img,
                        int64_t vout_rows, int32_t num_gaussians, int32_t B_out, int32_t B_geom,
                        int32_t img_h, int32_t img_w, float* v_colors, float* v_opacity,
                        float* v_xy, float* v_conic) {
    const RasterInputs in = raster_inputs(colors, rows_colors, opacities, rows_opac,
                                          map_opacities, rows_map_opac, background, rows_bg, xys,
                                          depths, radii, conics, cum_tiles_hit, num_gaussians,
                                          B_geom, img_h, img_w);
    const BlendBwdArgs a = bwd_args(final_Ts, final_idx, v_out_img, vout_rows, B_out, v_colors,
                                    v_opacity, v_xy, v_conic, nullptr, 0, nullptr);
    return rasterize_bwd_impl(static_cast<hipStream_t>(stream), in, nullptr, a);
}

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
                              float* v_xy, float* v_conic, float* v_depths) {
    if (!v_depths) return fail(kErrArgs, "rasterize_depth_bwd: v_depths missing");
    const RasterInputs in = raster_inputs(colors, rows_colors, opacities, rows_opac,
                                          map_opacities, rows_map_opac, background, rows_bg, xys,
                                          depths, radii, conics, cum_tiles_hit, num_gaussians,
                                          B_geom, img_h, img_w);
    const BlendBwdArgs a = bwd_args(final_Ts, final_idx, v_out_img, vout_rows, B_out, v_colors,
                                    v_opacity, v_xy, v_conic, v_out_depth, vdepth_rows, v_depths);
    return rasterize_bwd_impl(static_cast<hipStream_t>(stream), in, nullptr, a);
}

// ------------------------------------------------------------------ fused render path

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
                     int32_t loss_kind, float* loss) {
    if (B <= 0) return fail(kErrArgs, "render_fwd: invalid sizes");
    if (loss_kind != kLossNone && loss_kind != kLossL1 && loss_kind != kLossMse)
        return fail(kErrArgs, "render_fwd: loss_kind must be 0 (none), 1 (L1) or 2 (MSE)");
    if (loss_kind != kLossNone && (!loss_target || !loss))
        return fail(kErrArgs, "render_fwd: a fused loss needs the target and the loss output");
    const int64_t total = (int64_t)B * num_gaussians;
    ProjectArgs a;
    int rc = project_fwd_args(means3d, rows_means, scales, rows_scales, quats, rows_quats,
                              viewmat, rows_viewmat, opacities, rows_opac, transforms,
                              rows_transforms, transform_ids, num_gaussians, num_transforms,
                              has_transforms, total, img_h, img_w, fx, fy, cx, cy, glob_scale,
                              clip_thresh, xys, depths, radii, conics, num_tiles_hit,
                              cum_tiles_hit, quats_wxyz, &a);
    if (rc) return rc;
    // sorted_pos may be null: a forward with no backward sorts no emission positions
    if (capacity < 0 || !tile_bins || !records || (capacity > 0 && !sorted_ids))
        return fail(kErrArgs, "render_fwd: missing sorted-list or record buffers");
    if ((uintptr_t)records & 15)
        return fail(kErrArgs, "render_fwd: records must be 16-byte aligned");
    if (!out_img) return fail(kErrArgs, "render_fwd: missing image output");
    RasterInputs in = raster_inputs(colors, rows_colors, opacities, rows_opac, opacities,
                                    rows_opac, background, rows_bg, xys, depths, radii, conics,
                                    cum_tiles_hit, num_gaussians, B, img_h, img_w);
    in.compensate = compensate != 0;
    rc = check_raster(in, B);
    if (rc) return rc;
    if (!rows_match(rows_colors, num_gaussians, B))
        return fail(kErrArgs, "render_fwd: colors rows must be num_gaussians or B * num_gaussians");
    hipStream_t s = static_cast<hipStream_t>(stream);
    DeviceScratch& sc = scratch_for_current_device();
    ScratchUse use(sc, s);
    rc = use.rc;
    if (rc) return rc;
    const KeyLayout L = key_layout(B, img_h, img_w);
    if (L.overflow) return fail(kErrKeyOverflow, "render_fwd: intersection key overflow");
    sc.workload(B, num_gaussians, L.num_tiles);
    // the depth range from the projection: packed key, chunks meeting at most two images
    const bool fuse_range = L.packed && num_gaussians >= 1024;
    const int64_t chunks = project_fwd_chunks(total);
    {
        const int32_t bpi = (num_gaussians + 4095) / 4096;
        const int64_t need = std::max<int64_t>(4 * chunks, 2 * (int64_t)bpi * B);
        rc = ensure_minmax_partials(sc, need);
        if (!rc) rc = sc.ensure_sort(0, (int64_t)B * L.num_tiles, B, false);
    }
    if (rc) return rc;
    FusedRecords f;
    f.colors = colors; f.rows_colors = rows_colors; f.compensate = in.compensate;
    f.recs = reinterpret_cast<float4*>(records);
    f.mm_partial = fuse_range ? sc.mm_partial : nullptr;
    f.depth_mm = fuse_range ? sc.depth_mm : nullptr;
    // several chunks: the chunk scan writes the count and the emission finalizes cum_tiles_hit
    int32_t* count_word = reinterpret_cast<int32_t*>(sc.tickets + kCountWord);
    f.count_word = chunks > 1 ? count_word : nullptr;
    f.count_host = chunks > 1 ? sc.pinned_count_dev : nullptr;
    g_last_error.clear();
    {
        StageTimer tm(s, kStageProject);
        rc = launch_project_fwd_fused(a, f, sc, s);
    }
    if (rc) return fail(rc, "render_fwd: projection launch failed");
    SortTargets tgt;
    tgt.capacity = capacity;
    tgt.ids = sorted_ids;
    tgt.pos = sorted_pos;
    tgt.bins = tile_bins;
    tgt.depth_mm = fuse_range ? sc.depth_mm : nullptr;
    if (chunks > 1) {
        tgt.chunk_prefix = sc.chunk_sums;
        tgt.num_tiles_hit = num_tiles_hit;
        tgt.count_src = count_word;
        tgt.count_on_host = true;
    }
    PixelLoss lp;
    lp.kind = loss_kind;
    lp.target = loss_target;
    lp.count = (int64_t)B * img_h * img_w * 3;
    return rasterize_fwd_core(s, sc, in, &tgt, final_Ts, final_idx, out_img, out_depth, records,
                              tile_order, num_intersects, true,
                              loss_kind != kLossNone ? &lp : nullptr, loss);
}

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
                     int32_t loss_kind, const float* out_img, const float* v_loss) {
    const int32_t n = num_gaussians;
    if (n <= 0 || B <= 0) return fail(kErrArgs, "render_bwd: invalid sizes");
    if (loss_kind != kLossNone && loss_kind != kLossL1 && loss_kind != kLossMse)
        return fail(kErrArgs, "render_bwd: loss_kind must be 0 (none), 1 (L1) or 2 (MSE)");
    if (loss_kind != kLossNone) {
        // the image cotangent comes from the fused loss: every output image's rows
        v_out_img = nullptr;
        vout_rows = (int64_t)B * img_h;
    }
    if (!rows_match(rows_means, n, B) || !rows_match(rows_scales, n, B) ||
        !rows_match(rows_quats, n, B) || !rows_match(rows_viewmat, 4, B) ||
        !rows_match(rows_opac, n, B) || !rows_match(rows_colors, n, B))
        return fail(kErrArgs, "render_bwd: operand rows must be num_gaussians (shared) or "
                              "B * num_gaussians (batched); viewmat 4 or 4 * B");
    if (has_transforms && (num_transforms <= 0 || !transforms || !transform_ids ||
                           !v_transforms || !rows_match(rows_transforms, num_transforms, B)))
        return fail(kErrArgs, "render_bwd: transforms requested but not given");
    if (fold_shared && (rows_means != n || rows_scales != n || rows_quats != n ||
                        rows_colors != n || rows_opac != n))
        return fail(kErrArgs, "render_bwd: folding needs shared means, scales, quats, colors "
                              "and opacities");
    if (((uintptr_t)v_quats & 15) || ((uintptr_t)records & 15))
        return fail(kErrArgs, "render_bwd: v_quats and records must be 16-byte aligned");
    if (num_intersects < 0 || !tile_bins || (num_intersects > 0 && (!sorted_ids || !sorted_pos)))
        return fail(kErrArgs, "render_bwd: invalid sorted lists");
    if (!means3d || !scales || !quats || !viewmat || !radii || !v_means || !v_scales ||
        !v_quats)
        return fail(kErrArgs, "render_bwd: missing input or output buffer");
    RasterInputs in = raster_inputs(colors, rows_colors, opacities, rows_opac, opacities,
                                    rows_opac, background, rows_bg, xys, depths, nullptr, conics,
                                    cum_tiles_hit, n, B, img_h, img_w);
    in.compensate = compensate != 0;
    const bool depth = v_out_depth != nullptr;
    const int64_t items = (int64_t)B * n;
    // the 2D cotangents (v_xy, v_conic, v_depth per item) live in library scratch; v_depths is
    // only the depth flag for the check
    BlendBwdArgs ba = bwd_args(final_Ts, final_idx, v_out_img, vout_rows, B, v_colors,
                               v_opacities, nullptr, nullptr, v_out_depth, vdepth_rows,
                               depth ? const_cast<float*>(v_out_depth) : nullptr);
    ba.fold = fold_shared != 0;
    ba.loss.kind = loss_kind;
    ba.loss.target = loss_target;
    ba.loss.img = out_img;
    ba.loss.v_loss = v_loss;
    ba.loss.count = (int64_t)B * img_h * img_w * 3;
    int rc = check_raster_bwd(in, ba);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    DeviceScratch& sc = scratch_for_current_device();
    ScratchUse use(sc, s);
    rc = use.rc;
    if (rc) return rc;
    sc.workload(B, n, key_layout(B, img_h, img_w).num_tiles);
    rc = sc.ensure_item_grads(items);
    if (rc) return rc;
    ba.v_xy = sc.item_grads;
    ba.v_conic = sc.item_grads + 2 * items;
    ba.v_depths = depth ? sc.item_grads + 5 * items : nullptr;
    const KeptLists kept{sorted_ids, sorted_pos, tile_bins, num_intersects, records, tile_order};
    g_last_error.clear();
    rc = rasterize_bwd_core(s, sc, in, &kept, ba);
    if (rc) return rc;
    ProjectBwdArgs pa;
    pa.means = means3d; pa.rows_means = rows_means;
    pa.scales = scales; pa.rows_scales = rows_scales;
    pa.quats = quats; pa.rows_quats = rows_quats;
    pa.viewmat = viewmat; pa.rows_viewmat = rows_viewmat;
    pa.radii = radii; pa.rows_radii = items;
    pa.conics = conics; pa.rows_conics = items;
    pa.v_xy = ba.v_xy; pa.rows_vxy = items;
    pa.v_depth = ba.v_depths; pa.rows_vdepth = items;
    pa.v_conic = ba.v_conic; pa.rows_vconic = items;
    pa.transforms = transforms; pa.rows_transforms = has_transforms ? rows_transforms : 0;
    pa.transform_ids = transform_ids;
    pa.n = n; pa.num_transforms = has_transforms ? num_transforms : 0;
    pa.has_transforms = has_transforms; pa.B = B;
    pa.fx = fx; pa.fy = fy; pa.glob_scale = glob_scale;
    pa.v_mean3d = v_means; pa.v_scale = v_scales; pa.v_quat = v_quats;
    pa.v_viewmat = v_viewmat; pa.v_transforms = has_transforms ? v_transforms : nullptr;
    pa.quats_wxyz = quats_wxyz != 0;
    pa.fold = fold_shared != 0;
    StageTimer tm(s, kStageProjectBwd);
    rc = launch_project_bwd(pa, sc, s);
    if (rc) return fail(rc, "render_bwd: projection backward launch failed");
    return 0;
}

}  // extern "C"
