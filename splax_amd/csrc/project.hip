// Projection forward (fused with the global inclusive scan of the tile counts) and projection
// backward, gfx950.
//
// project_fwd: one thread per flat item (image b, gaussian g), restating _project_kernel
// (splax/_project/_kernels.py:122-248). Each workgroup owns a contiguous chunk of 1024 items;
// after counting tiles it scans its chunk in LDS, writes the chunk-local inclusive prefix to
// cum_tiles_hit and the chunk's total to a partials array. One workgroup then scans the
// partials, and a last pass adds each chunk's offset, which gives the global inclusive scan the
// reference gets from wp.utils.array_scan (splax/_project/_kernels.py:107). A decoupled
// look-back in the projection launch itself measured 0.15 ms slower at 12M items: its status
// polls cross the eight XCD-local L2s.
//
// project_bwd: one thread per flat item, restating _project_bwd_kernel
// (splax/_project/_kernels.py:356-484); the per-image viewmat gradient (formed only when asked
// for) is reduced per wave with DPP, then per workgroup in LDS into 12 partials per (image,
// workgroup), which viewmat_reduce_kernel sums in a fixed order. The transform gradient follows
// the reference's three cases: a workgroup whose gaussians share one transform reduces in LDS
// and adds with one atomic per entry, a workgroup on a slice boundary adds per thread.
#include "splat_common.hpp"
#include "splat_internal.hpp"

namespace splat {

struct ProjectParams {
    const float* means; int64_t rows_means;
    const float* scales; int64_t rows_scales;
    const float* quats; int64_t rows_quats;
    const float* viewmat; int64_t rows_viewmat;
    const float* opac; int64_t rows_opac;
    const float* transforms; int64_t rows_transforms;
    const int32_t* transform_ids;
    int32_t n, num_transforms, has_transforms;
    int64_t total;
    int32_t img_h, img_w;
    float fx, fy, cx, cy, glob_scale, clip_thresh;
    float* xys; float* depths; int32_t* radii; float* conics;
    int32_t* num_tiles_hit; int32_t* cum_tiles_hit;
    int32_t wxyz;  // quaternion storage order: 1 = wxyz (the public API's), 0 = xyzw
    uint32_t* chunk_sums;  // one per workgroup: its chunk's tile total
    // fused render forward (project_fwd_kernel<true>): each item's packed blend record and, per
    // chunk, the depth range of its visible items for the chunk's (at most two) images
    const float* colors; int64_t rows_colors;
    int32_t compensate;
    float4* recs;
    uint32_t* mm_partial;  // [chunks, 4]: ordered (lo, hi) of the first image, then the second
};

constexpr int kProjThreads = 256;
// Items per chunk of the projection's tile-count scan (one forward workgroup each): 1024 keeps the
// chunk-total scan short (about 12 totals per scan thread at 12M items).
constexpr int kProjFwdThreads = 1024;

__device__ __forceinline__ bool apply_transform(const float* transforms, int32_t image_id,
                                                int32_t num_transforms, bool sel_tf,
                                                int32_t tf_id, float* mean, float* R_tf) {
    R_tf[0] = 1.f; R_tf[1] = 0.f; R_tf[2] = 0.f;
    R_tf[3] = 0.f; R_tf[4] = 1.f; R_tf[5] = 0.f;
    R_tf[6] = 0.f; R_tf[7] = 0.f; R_tf[8] = 1.f;
    // ids outside [0, num_transforms) are treated as static
    if (tf_id < 0 || tf_id >= num_transforms) return false;
    int64_t tf_idx = sel_tf ? (int64_t)image_id * num_transforms + tf_id : tf_id;
    const float* m = transforms + tf_idx * 16;
    float t[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        R_tf[3 * i] = m[4 * i];
        R_tf[3 * i + 1] = m[4 * i + 1];
        R_tf[3 * i + 2] = m[4 * i + 2];
        t[i] = m[4 * i + 3];
    }
    float rm[3];
    mat_vec(R_tf, mean, rm);
#pragma unroll
    for (int i = 0; i < 3; ++i) mean[i] = rm[i] + t[i];
    return true;
}

// _project_geom, splax/_project/_kernels.py:647-664
__device__ __forceinline__ void project_geom(const float* mean, const float* q, const float* sc,
                                             float glob_scale, const float* vm, const float* R_tf,
                                             bool moved, float* W, float* p, float* M) {
    float tr[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        W[3 * i] = vm[4 * i];
        W[3 * i + 1] = vm[4 * i + 1];
        W[3 * i + 2] = vm[4 * i + 2];
        tr[i] = vm[4 * i + 3];
    }
    float wm[3];
    mat_vec(W, mean, wm);
#pragma unroll
    for (int i = 0; i < 3; ++i) p[i] = wm[i] + tr[i];
    float R[9];
    quat_to_rot(q[0], q[1], q[2], q[3], R);
    float s[3] = {glob_scale * sc[0], glob_scale * sc[1], glob_scale * sc[2]};
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) M[3 * i + j] = R[3 * i + j] * s[j];
    if (moved) {
        float Mm[9];
        mat_mul(R_tf, M, Mm);
#pragma unroll
        for (int k = 0; k < 9; ++k) M[k] = Mm[k];
    }
}

// What the projection wrote for one item, kept in registers for the fused record packing.
struct ItemOut {
    int32_t count;
    float x, y, depth, a, b, c, opac;
};

// Per-item projection; writes the item's outputs and returns them (count 0 when culled).
__device__ __forceinline__ ItemOut project_item(const ProjectParams& P, int64_t idx) {
    const int32_t n = P.n;
    const int32_t bid = (int32_t)(idx / n), gid = (int32_t)(idx - (int64_t)bid * n);
    const int64_t m_idx = P.rows_means > n ? idx : gid;
    const int64_t s_idx = P.rows_scales > n ? idx : gid;
    const int64_t q_idx = P.rows_quats > n ? idx : gid;
    const int64_t o_idx = P.rows_opac > n ? idx : gid;
    const int64_t vb = (int64_t)(P.rows_viewmat > 4 ? bid : 0) * 4;

    float2 xy = make_float2(0.f, 0.f);
    float depth = 0.f;
    int32_t radius = 0;
    float con0 = 0.f, con1 = 0.f, con2 = 0.f;
    int32_t count = 0;
    const float opac = P.opac[o_idx];

    // Every input of the item is loaded here, ahead of the transform's branch: the compiler
    // does not move loads across it, and loaded after it the quaternion, then the scales and
    // viewmat each cost one more dependent memory round trip per item (config 4's projection
    // took 0.50 ms that way against 0.43 ms).
    float mean[3] = {P.means[3 * m_idx], P.means[3 * m_idx + 1], P.means[3 * m_idx + 2]};
    const float* qp = P.quats + 4 * q_idx;
    const float q_in[4] = {qp[0], qp[1], qp[2], qp[3]};
    const float* scp = P.scales + 3 * s_idx;
    const float sc_in[3] = {scp[0], scp[1], scp[2]};
    const float* vmp = P.viewmat + vb * 4;
    float vm_in[12];
#pragma unroll
    for (int k = 0; k < 12; ++k) vm_in[k] = vmp[k];
    int32_t tf_id = P.has_transforms ? P.transform_ids[gid] : -1;
    float R_tf[9];
    bool moved = apply_transform(P.transforms, bid, P.num_transforms,
                                 P.rows_transforms > P.num_transforms, tf_id, mean, R_tf);
    float W[9], p[3], M[9];
    float q[4] = {q_in[0], q_in[1], q_in[2], q_in[3]};
    if (P.wxyz) {  // (w, x, y, z) -> (x, y, z, w)
        q[0] = q_in[1]; q[1] = q_in[2]; q[2] = q_in[3]; q[3] = q_in[0];
    }
    project_geom(mean, q, sc_in, P.glob_scale, vm_in, R_tf, moved, W, p, M);
    do {
        if (p[2] <= P.clip_thresh) break;
        float V[9];
        mat_mul_nt(M, M, V);
        const float tan_fovx = 0.5f * (float)P.img_w / P.fx;
        const float tan_fovy = 0.5f * (float)P.img_h / P.fy;
        const float lim_x = kFovClamp * tan_fovx;
        const float lim_y = kFovClamp * tan_fovy;
        float tz = p[2];
        float tx = tz * minw(lim_x, maxw(-lim_x, p[0] / tz));
        float ty = tz * minw(lim_y, maxw(-lim_y, p[1] / tz));
        float rz = 1.0f / tz;
        float rz2 = rz * rz;
        float j00 = P.fx * rz, j02 = -P.fx * tx * rz2, j11 = P.fy * rz, j12 = -P.fy * ty * rz2;
        float T0[3], T1[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            T0[j] = j00 * W[j] + j02 * W[6 + j];
            T1[j] = j11 * W[3 + j] + j12 * W[6 + j];
        }
        float TV0[3], TV1[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            TV0[k] = (T0[0] * V[k] + T0[1] * V[3 + k]) + T0[2] * V[6 + k];
            TV1[k] = (T1[0] * V[k] + T1[1] * V[3 + k]) + T1[2] * V[6 + k];
        }
        float c00 = (TV0[0] * T0[0] + TV0[1] * T0[1]) + TV0[2] * T0[2];
        float c01 = (TV0[0] * T1[0] + TV0[1] * T1[1]) + TV0[2] * T1[2];
        float c11 = (TV1[0] * T1[0] + TV1[1] * T1[1]) + TV1[2] * T1[2];
        float cxx = c00 + kDilation, cxy = c01, cyy = c11 + kDilation;
        float det = cxx * cyy - cxy * cxy;
        if (det == 0.0f) break;
        float inv_det = 1.0f / det;
        float a = cyy * inv_det, b = -cxy * inv_det, c = cxx * inv_det;
        float rw = 1.0f / (p[2] + kZEps);
        float center_x = (p[0] * rw) * P.fx + P.cx;
        float center_y = (p[1] * rw) * P.fy + P.cy;
        if (opac < kAlphaThresh) break;
        float t = iso_level(opac);
        float ext = sqrtf(t);
        float radius_x = ceilf(ext * sqrtf(cxx));
        float radius_y = ceilf(ext * sqrtf(cyy));
        if (radius_x <= 0.0f && radius_y <= 0.0f) break;
        if (center_x + radius_x <= 0.0f || center_x - radius_x >= (float)P.img_w ||
            center_y + radius_y <= 0.0f || center_y - radius_y >= (float)P.img_h)
            break;
        const int32_t tb_x = (P.img_w + kBlockWidth - 1) / kBlockWidth;
        const int32_t tb_y = (P.img_h + kBlockWidth - 1) / kBlockWidth;
        Ellipse e = ellipse_init(a, b, c, t, center_x, center_y, tb_x, tb_y);
        int32_t cnt = ellipse_tile_count(e);
        if (cnt <= 0) break;
        count = cnt;
        depth = p[2];
        radius = f2i(maxw(radius_x, radius_y));
        xy = make_float2(center_x, center_y);
        con0 = a;
        con1 = b;
        con2 = c;
    } while (false);
    reinterpret_cast<float2*>(P.xys)[idx] = xy;
    P.depths[idx] = depth;
    P.radii[idx] = radius;
    P.conics[3 * idx] = con0;
    P.conics[3 * idx + 1] = con1;
    P.conics[3 * idx + 2] = con2;
    P.num_tiles_hit[idx] = count;
    return ItemOut{count, xy.x, xy.y, depth, con0, con1, con2, opac};
}

// Items per thread of the fused projection + scan; one workgroup covers 256 * kProjItems items.
// One item per thread keeps the loads coalesced and gives the latency-bound projection the most
// waves in flight.
constexpr int kProjItems = 1;
static_assert(kProjFwdThreads * kProjItems == kProjChunkItems, "one chunk per projection workgroup");

// kFused (the fused render forward): also the item's packed blend record and the chunk's depth
// range partials (the chunk spans at most two images: num_gaussians >= 1024).
template <bool kFused>
__global__ void __launch_bounds__(kProjFwdThreads) project_fwd_kernel(ProjectParams P) {
    __shared__ int32_t s_wave[kProjFwdThreads / 64];
    __shared__ uint32_t s_mm[kProjFwdThreads / 64][4];
    const int tid = threadIdx.x;
    const uint32_t part = blockIdx.x;
    const int64_t base = (int64_t)part * (kProjFwdThreads * kProjItems);
    // Items are blocked per thread (thread t owns base + t*K .. +K-1) so the per-thread running
    // sum plus one block scan gives the inclusive prefix.
    int32_t cnt[kProjItems];
    int32_t local = 0;
    uint32_t mm[4] = {0xffffffffu, 0u, 0xffffffffu, 0u};  // (lo, hi) per image slot
#pragma unroll
    for (int k = 0; k < kProjItems; ++k) {
        int64_t idx = base + (int64_t)tid * kProjItems + k;
        cnt[k] = 0;
        if (idx < P.total) {
            // the record's colour is loaded with the item's other inputs, not after its stores
            float col[3] = {0.f, 0.f, 0.f};
            if constexpr (kFused) {
                const float* cp = P.colors + 3 * (idx % P.rows_colors);
                col[0] = cp[0]; col[1] = cp[1]; col[2] = cp[2];
            }
            const ItemOut o = project_item(P, idx);
            cnt[k] = o.count;
            if constexpr (kFused) {
                float4 r[4];
                pack_record(o.x, o.y, o.a, o.b, o.c, o.opac, P.compensate, col, o.depth, r);
                float4* dst = P.recs + 4 * idx;
#pragma unroll
                for (int q = 0; q < 4; ++q) dst[q] = r[q];
                // visible items (radii > 0) set the range, splax/_rasterize/_sort/_kernels.py:38-73;
                // slot 0 or 1: with n >= 1024 a chunk meets at most two images
                if (P.mm_partial && o.count > 0) {
                    const bool second = idx / P.n != base / P.n;
                    const uint32_t u = f2ord(o.depth);
                    if (second) {
                        mm[2] = u;
                        mm[3] = u;
                    } else {
                        mm[0] = u;
                        mm[1] = u;
                    }
                }
            }
        }
        local += cnt[k];
    }
    // block inclusive scan of `local`
    const int lane = tid & 63, wave = tid >> 6;
    int32_t incl = wave_inclusive_scan_i32(local, lane);
    if (lane == 63) s_wave[wave] = incl;
    if constexpr (kFused) {
        // the wave's (lo, hi) per image slot, in lane 63 (DPP, every lane active here)
        mm[0] = wave_minmax_to_lane63<false>(mm[0]);
        mm[1] = wave_minmax_to_lane63<true>(mm[1]);
        mm[2] = wave_minmax_to_lane63<false>(mm[2]);
        mm[3] = wave_minmax_to_lane63<true>(mm[3]);
        if (lane == 63) {
#pragma unroll
            for (int q = 0; q < 4; ++q) s_mm[wave][q] = mm[q];
        }
    }
    __syncthreads();
    if constexpr (kFused) {
        if (P.mm_partial && tid < 4) {
            uint32_t v = s_mm[0][tid];
#pragma unroll
            for (int w = 1; w < kProjFwdThreads / 64; ++w) {
                const uint32_t o = s_mm[w][tid];
                v = (tid & 1) ? (o > v ? o : v) : (o < v ? o : v);
            }
            P.mm_partial[4 * (int64_t)part + tid] = v;
        }
    }
    int32_t wave_off = 0, block_total = 0;
#pragma unroll
    for (int w = 0; w < kProjFwdThreads / 64; ++w) {
        int32_t v = s_wave[w];
        if (w < wave) wave_off += v;
        block_total += v;
    }
    if (tid == 0) P.chunk_sums[part] = (uint32_t)block_total;
    int32_t run = wave_off + incl - local;
#pragma unroll
    for (int k = 0; k < kProjItems; ++k) {
        int64_t idx = base + (int64_t)tid * kProjItems + k;
        run += cnt[k];
        if (idx < P.total) P.cum_tiles_hit[idx] = run;
    }
}

// Exclusive scan of the chunk totals in place, one 1024-thread workgroup: each thread sums a
// contiguous run of chunks, the runs are scanned in LDS, then each thread writes its run's
// prefixes.
constexpr int kChunkScanThreads = 1024;
// Two independent single-workgroup passes between the projection and the sort, in one launch:
// (1) block 0 (when chunks > 1) turns the chunk totals into exclusive prefixes, which
//     chunk_offset_kernel (or, on the render path, the emission) then adds to the chunks' items,
//     and with total_out non-null writes the grand total (the intersection count) there, and
//     with total_host non-null also into that host-visible word (a system-scope store, so the
//     host reads it once the kernel's completion is signalled, with no copy launch);
// (2) with mm non-null, block b < images folds the fused projection's per-chunk depth-range
//     partials of image b into the image's range of visible items (what minmax_partial_kernel /
//     minmax_final_kernel give): chunk c holds items [1024 c, 1024 c + 1024), its slot 0 the
//     image of its first item, slot 1 the next.
__global__ void __launch_bounds__(kChunkScanThreads)
chunk_scan_kernel(uint32_t* sums, int64_t chunks, const uint32_t* partial, int32_t n, float* mm,
                  int64_t images, int32_t* total_out, int32_t* total_host) {
    __shared__ uint32_t s_wave[kChunkScanThreads / 64];
    __shared__ uint32_t s_lo[kChunkScanThreads / 64], s_hi[kChunkScanThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (blockIdx.x == 0 && chunks > 1) {
        const int64_t per = (chunks + kChunkScanThreads - 1) / kChunkScanThreads;
        const int64_t lo = (int64_t)tid * per;
        const int64_t hi = lo + per < chunks ? lo + per : chunks;
        // runs of up to kChunkScanPer chunks (up to 64Ki chunks, 67M items) are loaded into
        // registers at once, so their load latencies overlap; longer runs take a sequential loop
        constexpr int kChunkScanPer = 64;
        const bool in_regs = per <= kChunkScanPer;
        uint32_t v[kChunkScanPer];
        uint32_t total = 0;
        if (in_regs) {
#pragma unroll
            for (int k = 0; k < kChunkScanPer; ++k) v[k] = lo + k < hi ? sums[lo + k] : 0u;
#pragma unroll
            for (int k = 0; k < kChunkScanPer; ++k) total += v[k];
        } else {
            for (int64_t c = lo; c < hi; ++c) total += sums[c];
        }
        // exclusive prefix of the run totals: a wave scan, then the totals of the waves before
        const uint32_t incl = (uint32_t)wave_inclusive_scan_i32((int32_t)total, lane);
        if (lane == 63) s_wave[wave] = incl;
        __syncthreads();
        uint32_t run = incl - total;
        for (int w = 0; w < wave; ++w) run += s_wave[w];
        if (in_regs) {
#pragma unroll
            for (int k = 0; k < kChunkScanPer; ++k) {
                if (lo + k < hi) sums[lo + k] = run;
                run += v[k];
            }
        } else {
            for (int64_t c = lo; c < hi; ++c) {
                const uint32_t x = sums[c];
                sums[c] = run;
                run += x;
            }
        }
        // the last thread's run ends at the grand total (runs past the chunks are empty); int32
        // wrap-around on overflow is kept, as in cum_tiles_hit
        if (total_out && tid == kChunkScanThreads - 1) *total_out = (int32_t)run;
        if (total_host && tid == kChunkScanThreads - 1)
            __hip_atomic_store(total_host, (int32_t)run, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
    }
    if (mm != nullptr && (int64_t)blockIdx.x < images) {
        const int64_t image = blockIdx.x;
        const int64_t c0 = image * n / kProjFwdThreads;
        int64_t c1 = ((image + 1) * n - 1) / kProjFwdThreads;
        c1 = c1 < chunks - 1 ? c1 : chunks - 1;
        uint32_t lo = 0xffffffffu, hi = 0u;
        for (int64_t c = c0 + tid; c <= c1; c += kChunkScanThreads) {
            const int64_t slot = image - c * kProjFwdThreads / n;  // 0 or 1
            const uint32_t x = partial[4 * c + 2 * slot], y = partial[4 * c + 2 * slot + 1];
            lo = x < lo ? x : lo;
            hi = y > hi ? y : hi;
        }
        // the wave's range in lane 63 (DPP; every lane of the workgroup is here)
        lo = wave_minmax_to_lane63<false>(lo);
        hi = wave_minmax_to_lane63<true>(hi);
        if (lane == 63) {
            s_lo[wave] = lo;
            s_hi[wave] = hi;
        }
        __syncthreads();
        if (tid == 0) {
            lo = 0xffffffffu;
            hi = 0u;
            for (int w = 0; w < kChunkScanThreads / 64; ++w) {
                lo = s_lo[w] < lo ? s_lo[w] : lo;
                hi = s_hi[w] > hi ? s_hi[w] : hi;
            }
            // no visible item: the reference's +-1e30 seeds remain (drange < 0 -> depth_q = 0)
            mm[2 * image] = hi == 0u ? 1.0e30f : ord2f(lo);
            mm[2 * image + 1] = hi == 0u ? -1.0e30f : ord2f(hi);
        }
    }
}

// cum_tiles_hit += the chunk's offset (chunk 0 has none); int32 wrap-around on overflow is kept,
// the host reports a negative total as too many intersections. A chunk is one workgroup of the
// projection, one item per thread.
static_assert(kProjItems == 1, "chunk_offset_kernel maps one thread to one item");
__global__ void __launch_bounds__(kProjFwdThreads) chunk_offset_kernel(int32_t* cum, int64_t total,
                                                           const uint32_t* offsets) {
    const int64_t idx = (int64_t)(blockIdx.x + 1) * kProjFwdThreads + threadIdx.x;
    if (idx < total) cum[idx] = (int32_t)((uint32_t)cum[idx] + offsets[blockIdx.x + 1]);
}

// ------------------------------------------------------------------ projection backward

struct ProjectBwdParams {
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
    int32_t n, num_transforms, has_transforms, B, blocks_per_image;
    float fx, fy, glob_scale;
    float* v_mean3d; float* v_scale; float* v_quat; float* v_viewmat; float* v_transforms;
    float* view_partials;  // [B * blocks_per_image, 12] or null (no viewmat gradient)
    int32_t wxyz;  // quats and v_quat stored wxyz (1) or xyzw (0)
    int32_t fold;  // gaussian gradients summed over the images into n rows
};

// One workgroup per (image, block of gaussians); with kFold one workgroup per block of
// gaussians walks every image in order and sums the gaussian gradients in registers, so the
// shared parameters are read once per gaussian and the per-image rows are never written.
// kTf (rigid transforms given), kView (the viewmat gradient asked for) and kFold are template
// parameters: without them the kernel holds 64 VGPRs (eight waves per SIMD) where the general
// form holds 130 (three).
template <bool kTf, bool kView, bool kFold>
__global__ void __launch_bounds__(kProjThreads) project_bwd_kernel(ProjectBwdParams P) {
    __shared__ float s_red[kProjThreads / 64][12];
    __shared__ int32_t s_tf[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t n = P.n;
    const int32_t first_image = kFold ? 0 : blockIdx.x / P.blocks_per_image;
    const int32_t local_block =
        kFold ? (int32_t)blockIdx.x : (int32_t)blockIdx.x - first_image * P.blocks_per_image;
    const int32_t end_image = kFold ? P.B : first_image + 1;
    const int32_t gid = local_block * kProjThreads + tid;
    float fm[3] = {0.f, 0.f, 0.f}, fs[3] = {0.f, 0.f, 0.f}, fq[4] = {0.f, 0.f, 0.f, 0.f};
    for (int32_t image_id = first_image; image_id < end_image; ++image_id) {
    const int64_t idx = (int64_t)image_id * n + gid;
    float vR[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    float vt[3] = {0, 0, 0};
    float vRtf[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    float vttf[3] = {0, 0, 0};
    bool moved = false;
    int32_t tf_id = -1;
    const bool in_range = gid < n;
    if (in_range && kTf) tf_id = P.transform_ids[gid];
    if (in_range) {
        float zero3[3] = {0.f, 0.f, 0.f};
        float vmean_out[3] = {0.f, 0.f, 0.f}, vscale[3] = {0.f, 0.f, 0.f};
        float vq[4] = {0.f, 0.f, 0.f, 0.f};
        (void)zero3;
        const int64_t r_idx = P.rows_radii > n ? idx : gid;
        // Every input is loaded and the math runs for culled items too (results discarded
        // below): the loads then issue together instead of waiting on radii first.
        const bool vis = P.radii[r_idx] > 0;
        {
            const int64_t m_idx = P.rows_means > n ? idx : gid;
            const int64_t s_idx = P.rows_scales > n ? idx : gid;
            const int64_t q_idx = P.rows_quats > n ? idx : gid;
            const int64_t c_idx = P.rows_conics > n ? idx : gid;
            const int64_t vx_idx = P.rows_vxy > n ? idx : gid;
            const int64_t vd_idx = P.rows_vdepth > n ? idx : gid;
            const int64_t vc_idx = P.rows_vconic > n ? idx : gid;
            const int64_t vb = (int64_t)(P.rows_viewmat > 4 ? image_id : 0) * 4;
            const float* mean_local = P.means + 3 * m_idx;
            float ml[3] = {mean_local[0], mean_local[1], mean_local[2]};
            float mean[3] = {ml[0], ml[1], ml[2]};
            float R_tf[9];
            moved = apply_transform(P.transforms, image_id, P.num_transforms,
                                    P.rows_transforms > P.num_transforms, tf_id, mean, R_tf);
            const float* q = P.quats + 4 * q_idx;
            float qx = q[0], qy = q[1], qz = q[2], qw = q[3];
            if (P.wxyz) {
                qw = q[0]; qx = q[1]; qy = q[2]; qz = q[3];
            }
            float qv[4] = {qx, qy, qz, qw};
            const float* sc = P.scales + 3 * s_idx;
            float scv[3] = {sc[0], sc[1], sc[2]};
            float W[9], p[3], M[9];
            project_geom(mean, qv, scv, P.glob_scale, P.viewmat + vb * 4, R_tf, moved, W, p, M);
            float V[9];
            mat_mul_nt(M, M, V);
            float R[9];
            quat_to_rot(qx, qy, qz, qw, R);
            float s[3] = {P.glob_scale * scv[0], P.glob_scale * scv[1], P.glob_scale * scv[2]};
            const float fx = P.fx, fy = P.fy;
            float rz = 1.0f / p[2];
            float rz2 = rz * rz;
            // J = [[j00, 0, j02], [0, j11, j12], [0, 0, 0]]. The products of this VJP drop every
            // term with a structural zero factor (J's last row; the last row and column of the
            // 2D covariance cotangent) and keep the others in the full products' order; the CPU
            // oracle evaluates the same expressions.
            const float j00 = fx * rz, j02 = -fx * p[0] * rz2;
            const float j11 = fy * rz, j12 = -fy * p[1] * rz2;
            float T0[3], T1[3];  // rows 0 and 1 of T = J W (row 2 is zero)
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                T0[b] = j00 * W[b] + j02 * W[6 + b];
                T1[b] = j11 * W[3 + b] + j12 * W[6 + b];
            }
            const float* cn = P.conics + 3 * c_idx;
            const float* vc = P.v_conic + 3 * vc_idx;
            float X0 = cn[0], X1 = cn[1], X3 = cn[2];
            float G0 = vc[0], G1 = 0.5f * vc[1], G3 = vc[2];
            float XG0 = X0 * G0 + X1 * G1, XG1 = X0 * G1 + X1 * G3;
            float XG2 = X1 * G0 + X3 * G1, XG3 = X1 * G1 + X3 * G3;
            float S0 = XG0 * X0 + XG1 * X1, S1 = XG0 * X1 + XG1 * X3;
            float S2 = XG2 * X0 + XG3 * X1, S3 = XG2 * X1 + XG3 * X3;
            float vcov0 = -S0, vcov1 = -(S1 + S2), vcov2 = -S3;
            // _proj_vjp, splax/_project/_kernels.py:487-533
            float tx = p[0], ty = p[1], tz = p[2];
            float prz = 1.0f / tz;
            float prz2 = prz * prz;
            float prz3 = prz2 * prz;
            float rw = 1.0f / (tz + kZEps);
            const float* vxy = P.v_xy + 2 * vx_idx;
            float vpx = fx * vxy[0], vpy = fy * vxy[1];
            float vvx = vpx * rw, vvy = vpy * rw;
            float vvz = -(vpx * tx + vpy * ty) * rw * rw;
            vvz = vvz + (P.v_depth ? P.v_depth[vd_idx] : 0.0f);  // NULL: zero cotangent
            // v_cov = [[c0, c1, 0], [c1, c2, 0], [0, 0, 0]]
            const float c0 = vcov0, c1 = 0.5f * vcov1, c2 = vcov2;
            // v_V = T^T v_cov T: tmp = T^T v_cov has a zero last column
            float tmp0[3], tmp1[3], v_V[9];
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                tmp0[a] = T0[a] * c0 + T1[a] * c1;
                tmp1[a] = T0[a] * c1 + T1[a] * c2;
            }
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int b = 0; b < 3; ++b) v_V[3 * a + b] = tmp0[a] * T0[b] + tmp1[a] * T1[b];
            // v_T = (2 v_cov) T V: rows 0 and 1 (row 2 is zero)
            const float d0 = 2.0f * c0, d1 = 2.0f * c1, d2 = 2.0f * c2;
            float u0[3], u1[3], v_T[6];
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                u0[b] = d0 * T0[b] + d1 * T1[b];
                u1[b] = d1 * T0[b] + d2 * T1[b];
            }
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                v_T[b] = (u0[0] * V[b] + u0[1] * V[3 + b]) + u0[2] * V[6 + b];
                v_T[3 + b] = (u1[0] * V[b] + u1[1] * V[3 + b]) + u1[2] * V[6 + b];
            }
            // v_J = v_T W^T, rows 0 and 1
            float v_J[6];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 3; ++b)
                    v_J[3 * a + b] = (v_T[3 * a] * W[3 * b] + v_T[3 * a + 1] * W[3 * b + 1]) +
                                     v_T[3 * a + 2] * W[3 * b + 2];
            float v_t_x = -fx * prz2 * v_J[2];
            float v_t_y = -fy * prz2 * v_J[5];
            float v_t_z = -fx * prz2 * v_J[0] + 2.0f * fx * tx * prz3 * v_J[2] -
                          fy * prz2 * v_J[4] + 2.0f * fy * ty * prz3 * v_J[5];
            float v_p[3] = {vvx + v_t_x, vvy + v_t_y, vvz + v_t_z};
            float v_mean_world[3];
            mat_t_vec(W, v_p, v_mean_world);
            float vVs[9], v_M_world[9];
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int b = 0; b < 3; ++b) vVs[3 * a + b] = v_V[3 * a + b] + v_V[3 * b + a];
            mat_mul(vVs, M, v_M_world);
            float v_M[9];
            if (moved) {
                mat_t_vec(R_tf, v_mean_world, vmean_out);
                mat_mul_tn(R_tf, v_M_world, v_M);
                float M_local[9], vmMl[9];
                mat_mul_tn(R_tf, M, M_local);
                mat_mul_nt(v_M_world, M_local, vmMl);
#pragma unroll
                for (int a = 0; a < 3; ++a)
#pragma unroll
                    for (int b = 0; b < 3; ++b)
                        vRtf[3 * a + b] = v_mean_world[a] * ml[b] + vmMl[3 * a + b];
#pragma unroll
                for (int a = 0; a < 3; ++a) vttf[a] = v_mean_world[a];
            } else {
#pragma unroll
                for (int a = 0; a < 3; ++a) vmean_out[a] = v_mean_world[a];
#pragma unroll
                for (int k = 0; k < 9; ++k) v_M[k] = v_M_world[k];
            }
            // _scale_vjp
#pragma unroll
            for (int j = 0; j < 3; ++j)
                vscale[j] = ((R[j] * v_M[j] + R[3 + j] * v_M[3 + j]) + R[6 + j] * v_M[6 + j]) *
                            P.glob_scale;
            // _quat_vjp (xyzw output)
            float r[9];
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int b = 0; b < 3; ++b) r[3 * a + b] = v_M[3 * a + b] * s[b];
            float x = qx, y = qy, z = qz, w = qw;
            vq[3] = 2.0f * ((x * (r[7] - r[5]) + y * (r[2] - r[6])) + z * (r[3] - r[1]));
            vq[0] = 2.0f * (((-2.0f * x * (r[4] + r[8]) + y * (r[3] + r[1])) +
                             z * (r[6] + r[2])) + w * (r[7] - r[5]));
            vq[1] = 2.0f * (((x * (r[3] + r[1]) - 2.0f * y * (r[0] + r[8])) +
                             z * (r[7] + r[5])) + w * (r[2] - r[6]));
            vq[2] = 2.0f * (((x * (r[6] + r[2]) + y * (r[7] + r[5])) -
                             2.0f * z * (r[0] + r[4])) + w * (r[3] - r[1]));
            // _view_vjp: v_R = v_p (x) mean + J^T v_T, v_t = v_p
            float JtvT[9];  // J^T v_T
#pragma unroll
            for (int b = 0; b < 3; ++b) {
                JtvT[b] = j00 * v_T[b];
                JtvT[3 + b] = j11 * v_T[3 + b];
                JtvT[6 + b] = j02 * v_T[b] + j12 * v_T[3 + b];
            }
#pragma unroll
            for (int a = 0; a < 3; ++a) {
#pragma unroll
                for (int b = 0; b < 3; ++b) vR[3 * a + b] = v_p[a] * mean[b] + JtvT[3 * a + b];
                vt[a] = v_p[a];
            }
        }
        if (!vis) {  // culled items contribute nothing (splax/_project/_kernels.py:408)
            moved = false;
#pragma unroll
            for (int k = 0; k < 9; ++k) vR[k] = vRtf[k] = 0.0f;
#pragma unroll
            for (int k = 0; k < 3; ++k) vt[k] = vttf[k] = vmean_out[k] = vscale[k] = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) vq[k] = 0.0f;
        }
        if (kFold) {
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                fm[k] = fm[k] + vmean_out[k];
                fs[k] = fs[k] + vscale[k];
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) fq[k] = fq[k] + vq[k];
        } else {
            P.v_mean3d[3 * idx] = vmean_out[0];
            P.v_mean3d[3 * idx + 1] = vmean_out[1];
            P.v_mean3d[3 * idx + 2] = vmean_out[2];
            P.v_scale[3 * idx] = vscale[0];
            P.v_scale[3 * idx + 1] = vscale[1];
            P.v_scale[3 * idx + 2] = vscale[2];
            reinterpret_cast<float4*>(P.v_quat)[idx] =
                P.wxyz ? make_float4(vq[3], vq[0], vq[1], vq[2])
                       : make_float4(vq[0], vq[1], vq[2], vq[3]);
        }
    }
    // viewmat gradient (when asked for): wave DPP reduction, then across the 4 waves in LDS, one
    // partial per (image, workgroup) that viewmat_reduce_kernel sums in a fixed order (atomics
    // from thousands of workgroups into the same 12 words serialize in the L2)
    if (kView) {
        float red[12];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
#pragma unroll
            for (int b = 0; b < 3; ++b) red[4 * a + b] = vR[3 * a + b];
            red[4 * a + 3] = vt[a];
        }
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            float v = wave_sum_to_lane63(red[k]);
            if (lane == 63) s_red[wave][k] = v;
        }
        __syncthreads();
        if (tid < 12) {
            float v = ((s_red[0][tid] + s_red[1][tid]) + s_red[2][tid]) + s_red[3][tid];
            P.view_partials[((int64_t)image_id * P.blocks_per_image + local_block) * 12 + tid] = v;
        }
    }
    // Transform gradient: uniform block -> block reduction; mixed -> per-thread atomics
    // (splax/_project/_kernels.py:461-484).
    if (kTf) {
        int32_t id = in_range ? tf_id : -1;
        int32_t tmin = block_min_i32(in_range ? tf_id : 2147483647, s_tf);
        int32_t tmax = block_max_i32(in_range ? tf_id : (-2147483647 - 1), s_tf);
        (void)id;
        // ids at or beyond num_transforms are static (apply_transform), like negative ones
        if (tmin == tmax && tmin >= 0 && tmin < P.num_transforms) {
            __syncthreads();
            float rt[12];
#pragma unroll
            for (int a = 0; a < 3; ++a) {
#pragma unroll
                for (int b = 0; b < 3; ++b) rt[4 * a + b] = vRtf[3 * a + b];
                rt[4 * a + 3] = vttf[a];
            }
#pragma unroll
            for (int k = 0; k < 12; ++k) {
                float v = wave_sum_to_lane63(rt[k]);
                if (lane == 63) s_red[wave][k] = v;
            }
            __syncthreads();
            if (tid < 12) {
                float v = ((s_red[0][tid] + s_red[1][tid]) + s_red[2][tid]) + s_red[3][tid];
                int64_t slot = (int64_t)image_id * P.num_transforms + tmin;
                atomicAdd(P.v_transforms + slot * 16 + tid, v);
            }
        } else if (moved && tmin != tmax) {
            int64_t slot = (int64_t)image_id * P.num_transforms + tf_id;
            float* dst = P.v_transforms + slot * 16;
#pragma unroll
            for (int a = 0; a < 3; ++a) {
#pragma unroll
                for (int b = 0; b < 3; ++b) atomicAdd(dst + 4 * a + b, vRtf[3 * a + b]);
                atomicAdd(dst + 4 * a + 3, vttf[a]);
            }
        }
    }
    __syncthreads();  // s_red / s_tf are reused by the next image
    }
    if (kFold && gid < n) {
        P.v_mean3d[3 * gid] = fm[0];
        P.v_mean3d[3 * gid + 1] = fm[1];
        P.v_mean3d[3 * gid + 2] = fm[2];
        P.v_scale[3 * gid] = fs[0];
        P.v_scale[3 * gid + 1] = fs[1];
        P.v_scale[3 * gid + 2] = fs[2];
        reinterpret_cast<float4*>(P.v_quat)[gid] =
            P.wxyz ? make_float4(fq[3], fq[0], fq[1], fq[2])
                   : make_float4(fq[0], fq[1], fq[2], fq[3]);
    }
}

// One workgroup per image: the image's workgroup partials summed in a fixed order (each thread a
// strided run, then the waves), written with the zero bottom row as the viewmat gradient.
__global__ void __launch_bounds__(kProjThreads)
viewmat_reduce_kernel(const float* partials, int32_t blocks_per_image, float* v_viewmat) {
    __shared__ float s_red[kProjThreads / 64][12];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t image = blockIdx.x;
    const float* src = partials + image * blocks_per_image * 12;
    float acc[12];
#pragma unroll
    for (int k = 0; k < 12; ++k) acc[k] = 0.f;
    for (int32_t j = tid; j < blocks_per_image; j += kProjThreads) {
#pragma unroll
        for (int k = 0; k < 12; ++k) acc[k] = acc[k] + src[(int64_t)j * 12 + k];
    }
#pragma unroll
    for (int k = 0; k < 12; ++k) {
        const float v = wave_sum_to_lane63(acc[k]);
        if (lane == 63) s_red[wave][k] = v;
    }
    __syncthreads();
    if (tid < 16)
        v_viewmat[image * 16 + tid] =
            tid < 12 ? ((s_red[0][tid] + s_red[1][tid]) + s_red[2][tid]) + s_red[3][tid] : 0.f;
}

// Chunks (workgroups) of a projection over `total` items: one chunk total of scratch each.
int64_t project_fwd_chunks(int64_t total) {
    const int64_t per_block = (int64_t)kProjFwdThreads * kProjItems;
    return (total + per_block - 1) / per_block;
}

int launch_project_fwd(const ProjectArgs& a, DeviceScratch& sc, hipStream_t stream) {
    if (a.total <= 0) return 0;
    const int64_t blocks = project_fwd_chunks(a.total);
    if (blocks > (int64_t)sc.chunk_sums_cap) {
        int rc = sc.grow_chunk_sums(blocks);
        if (rc) return rc;
    }
    return launch_project_fwd_into(a, sc.chunk_sums, stream);
}

int launch_project_fwd_into(const ProjectArgs& a, uint32_t* chunk_sums, hipStream_t stream) {
    return launch_project_fwd_impl(a, chunk_sums, nullptr, stream);
}

int launch_project_fwd_fused(const ProjectArgs& a, const FusedRecords& f, DeviceScratch& sc,
                             hipStream_t stream) {
    if (a.total <= 0) return 0;
    const int64_t blocks = project_fwd_chunks(a.total);
    if (blocks > (int64_t)sc.chunk_sums_cap) {
        int rc = sc.grow_chunk_sums(blocks);
        if (rc) return rc;
    }
    return launch_project_fwd_impl(a, sc.chunk_sums, &f, stream);
}

int launch_project_fwd_impl(const ProjectArgs& a, uint32_t* chunk_sums, const FusedRecords* f,
                            hipStream_t stream) {
    if (a.total <= 0) return 0;
    const int64_t blocks = project_fwd_chunks(a.total);
    ProjectParams P;
    P.means = a.means; P.rows_means = a.rows_means;
    P.scales = a.scales; P.rows_scales = a.rows_scales;
    P.quats = a.quats; P.rows_quats = a.rows_quats;
    P.viewmat = a.viewmat; P.rows_viewmat = a.rows_viewmat;
    P.opac = a.opacities; P.rows_opac = a.rows_opac;
    P.transforms = a.transforms; P.rows_transforms = a.rows_transforms;
    P.transform_ids = a.transform_ids;
    P.n = a.n; P.num_transforms = a.num_transforms; P.has_transforms = a.has_transforms;
    P.total = a.total; P.img_h = a.img_h; P.img_w = a.img_w;
    P.fx = a.fx; P.fy = a.fy; P.cx = a.cx; P.cy = a.cy;
    P.glob_scale = a.glob_scale; P.clip_thresh = a.clip_thresh;
    P.xys = a.xys; P.depths = a.depths; P.radii = a.radii; P.conics = a.conics;
    P.num_tiles_hit = a.num_tiles_hit; P.cum_tiles_hit = a.cum_tiles_hit;
    P.wxyz = a.quats_wxyz;
    P.chunk_sums = chunk_sums;
    P.colors = f ? f->colors : nullptr; P.rows_colors = f ? f->rows_colors : 1;
    P.compensate = f ? f->compensate : 0;
    P.recs = f ? f->recs : nullptr;
    P.mm_partial = f ? f->mm_partial : nullptr;
    // the render path leaves the chunk offsets to the emission when there are several chunks
    const bool offsets_later = f && f->count_word && blocks > 1;
    if (f)
        hipLaunchKernelGGL(project_fwd_kernel<true>, dim3((unsigned)blocks),
                           dim3(kProjFwdThreads), 0, stream, P);
    else
        hipLaunchKernelGGL(project_fwd_kernel<false>, dim3((unsigned)blocks),
                           dim3(kProjFwdThreads), 0, stream, P);
    const int64_t images = (f && f->depth_mm) ? a.total / a.n : 0;
    if (blocks > 1 || images > 0)
        hipLaunchKernelGGL(chunk_scan_kernel, dim3((unsigned)(images > 1 ? images : 1)),
                           dim3(kChunkScanThreads), 0, stream, P.chunk_sums, blocks,
                           f ? f->mm_partial : nullptr, a.n, images > 0 ? f->depth_mm : nullptr,
                           images, offsets_later ? f->count_word : nullptr,
                           offsets_later ? f->count_host : nullptr);
    if (blocks > 1 && !offsets_later)
        return launch_chunk_offsets(P.cum_tiles_hit, a.total, P.chunk_sums, stream);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

int launch_chunk_offsets(int32_t* cum, int64_t total, const uint32_t* chunk_prefix,
                         hipStream_t stream) {
    const int64_t blocks = project_fwd_chunks(total);
    if (blocks > 1)
        hipLaunchKernelGGL(chunk_offset_kernel, dim3((unsigned)(blocks - 1)), dim3(kProjFwdThreads),
                           0, stream, cum, total, chunk_prefix);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

int launch_project_bwd(const ProjectBwdArgs& a, DeviceScratch& sc, hipStream_t stream) {
    const int32_t blocks_per_image = (a.n + kProjThreads - 1) / kProjThreads;
    // zero the transforms' atomic targets (per-item outputs and the viewmat gradient are fully
    // written by the kernels)
    int64_t ntf = (int64_t)a.B * a.num_transforms * 16;
    int rc = 0;
    if (a.v_transforms && ntf > 0) {
        rc = fill_zero_f32(a.v_transforms, ntf, stream);
        if (rc) return rc;
    }
    if (a.n <= 0 || a.B <= 0)
        return a.v_viewmat && a.B > 0 ? fill_zero_f32(a.v_viewmat, (int64_t)a.B * 16, stream) : 0;
    if (a.v_viewmat) {
        rc = sc.ensure_view_partials((int64_t)a.B * blocks_per_image * 12);
        if (rc) return rc;
    }
    ProjectBwdParams P;
    P.means = a.means; P.rows_means = a.rows_means;
    P.scales = a.scales; P.rows_scales = a.rows_scales;
    P.quats = a.quats; P.rows_quats = a.rows_quats;
    P.viewmat = a.viewmat; P.rows_viewmat = a.rows_viewmat;
    P.radii = a.radii; P.rows_radii = a.rows_radii;
    P.conics = a.conics; P.rows_conics = a.rows_conics;
    P.v_xy = a.v_xy; P.rows_vxy = a.rows_vxy;
    P.v_depth = a.v_depth; P.rows_vdepth = a.rows_vdepth;
    P.v_conic = a.v_conic; P.rows_vconic = a.rows_vconic;
    P.transforms = a.transforms; P.rows_transforms = a.rows_transforms;
    P.transform_ids = a.transform_ids;
    P.n = a.n; P.num_transforms = a.num_transforms; P.has_transforms = a.has_transforms;
    P.B = a.B; P.blocks_per_image = blocks_per_image;
    P.fx = a.fx; P.fy = a.fy; P.glob_scale = a.glob_scale;
    P.v_mean3d = a.v_mean3d; P.v_scale = a.v_scale; P.v_quat = a.v_quat;
    P.v_viewmat = a.v_viewmat; P.v_transforms = a.v_transforms;
    P.view_partials = a.v_viewmat ? sc.view_partials : nullptr;
    P.wxyz = a.quats_wxyz;
    P.fold = a.fold;
    int64_t blocks = (a.fold ? 1 : (int64_t)a.B) * blocks_per_image;
    const int variant = (a.has_transforms ? 4 : 0) | (a.v_viewmat ? 2 : 0) | (a.fold ? 1 : 0);
    const dim3 grid((unsigned)blocks), block(kProjThreads);
    switch (variant) {
        case 0: hipLaunchKernelGGL((project_bwd_kernel<false, false, false>), grid, block, 0, stream, P); break;
        case 1: hipLaunchKernelGGL((project_bwd_kernel<false, false, true>), grid, block, 0, stream, P); break;
        case 2: hipLaunchKernelGGL((project_bwd_kernel<false, true, false>), grid, block, 0, stream, P); break;
        case 3: hipLaunchKernelGGL((project_bwd_kernel<false, true, true>), grid, block, 0, stream, P); break;
        case 4: hipLaunchKernelGGL((project_bwd_kernel<true, false, false>), grid, block, 0, stream, P); break;
        case 5: hipLaunchKernelGGL((project_bwd_kernel<true, false, true>), grid, block, 0, stream, P); break;
        case 6: hipLaunchKernelGGL((project_bwd_kernel<true, true, false>), grid, block, 0, stream, P); break;
        default: hipLaunchKernelGGL((project_bwd_kernel<true, true, true>), grid, block, 0, stream, P); break;
    }
    if (a.v_viewmat)
        hipLaunchKernelGGL(viewmat_reduce_kernel, dim3((unsigned)a.B), dim3(kProjThreads), 0,
                           stream, sc.view_partials, blocks_per_image, a.v_viewmat);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

// ------------------------------------------------------------------ projection without allocation
// splat_project_fwd_noalloc keeps its chunk totals in this fixed array of kNoAllocMaxChunks
// uint32 (256 KiB), which each device the library runs on holds until the process ends. In host
// code `scratch` names a host-side stand-in, not the device array: its device address comes from
// hipGetSymbolAddress, once per device with that device current, and only that address is
// passed to kernels. Every no-allocation call on a device shares the array, so such calls must
// not overlap on one device (they would race on it); nothing in it needs to start at zero (the
// projection writes every chunk total before the scan reads it).
static __device__ __align__(256) uint32_t scratch[kNoAllocMaxChunks];

constexpr int kNoAllocDevices = 64;
static std::mutex g_noalloc_mu;
static uint32_t* g_noalloc_scratch[kNoAllocDevices] = {};

int launch_project_fwd_noalloc(const ProjectArgs& a, hipStream_t stream) {
    if (project_fwd_chunks(a.total) > kNoAllocMaxChunks)
        return fail(kErrArgs, "project_fwd_noalloc: more than " +
                                  std::to_string(kNoAllocMaxChunks * kProjFwdThreads) +
                                  " items (the fixed scratch holds " +
                                  std::to_string(kNoAllocMaxChunks) + " chunk totals)");
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocDevices)
        return fail(kErrRuntime, "project_fwd_noalloc: no usable current device");
    uint32_t* chunk_sums = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        if (!g_noalloc_scratch[dev]) {  // set-up, once per device
            void* ptr = nullptr;
            const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (e != hipSuccess || ptr == nullptr) {
                (void)hipGetLastError();
                return fail(kErrRuntime,
                            std::string("project_fwd_noalloc: hipGetSymbolAddress failed: ") +
                                hipGetErrorString(e));
            }
            g_noalloc_scratch[dev] = static_cast<uint32_t*>(ptr);
        }
        chunk_sums = g_noalloc_scratch[dev];
    }
    return launch_project_fwd_into(a, chunk_sums, stream);
}

}  // namespace splat
