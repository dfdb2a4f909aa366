// Forward and backward alpha blend on gfx950.
//
// One workgroup of 256 threads (four wave64s) per (image, 16x16 tile), as in the reference
// (splax/_rasterize/_kernels.py:63-87,469-500). Each wave owns one 8x8 quadrant of the tile, so a
// small gaussian touches few waves. Records of the tile's sorted range are staged in LDS in
// batches of 256 (structure of arrays: every lane reads the same record, an LDS broadcast). While
// staging, each record gets
//   - sigma_max: a conservative bound (log(255 o) + 1e-3) above which o e^-sigma < 1/255, so a
//     lane skips the exponential for pairs the reference rejects anyway, and
//   - a 4-bit quadrant mask: the quadrants whose pixel centres can reach sigma <= sigma_max,
//     from the ellipse's bounding box; a wave skips records outside its quadrant outright.
// Both only remove pairs that the reference's `sigma < 0 or alpha < 1/255` test rejects, so the
// per-pixel sequence of blended pairs (and every float operation on it) is the reference's.
//
// Backward: the same staging walked back to front from the workgroup's largest final_idx. Per
// record, the contributing lanes of a wave reduce their 9 gradient terms with DPP, one lane adds
// them into the record's LDS accumulator, and after the batch each record issues at most 9 float
// atomics to global memory (instead of 9 per contributing pixel).
#include "splat_common.hpp"
#include "splat_internal.hpp"

namespace splat {

constexpr int kTile = 256;

struct BlendCommon {
    const float* colors; int64_t rows_colors;
    const float* opac; int64_t rows_opac;
    const float* background; int64_t rows_bg;
    const float* xys; const float* conics;
    const int32_t* ids; const int32_t* bins;
    int32_t img_h, img_w, tiles_x, num_tiles;
};

// Pixel of thread `tid` in its tile: wave w = quadrant (w & 1, w >> 1), lane = 8x8 raster.
__device__ __forceinline__ void tile_pixel(int tid, int tile_x, int tile_y, int& i, int& j) {
    const int wave = tid >> 6, lane = tid & 63;
    i = tile_y * kBlockWidth + (wave >> 1) * 8 + (lane >> 3);
    j = tile_x * kBlockWidth + (wave & 1) * 8 + (lane & 7);
}

// Stage record `g` for the tile at (tile_x, tile_y); returns smax and the quadrant mask.
__device__ __forceinline__ void stage_bounds(float x, float y, float a, float b, float c, float o,
                                             int tile_x, int tile_y, float& smax,
                                             uint32_t& qmask) {
    if (o > 0.0f) {
        smax = __logf(o * 255.0f) + 1e-3f;
    } else {
        smax = (o != o) ? __builtin_inff() : -__builtin_inff();
    }
    qmask = 0xfu;
    if (!(smax >= 0.0f)) {  // every pixel rejected (NaN smax only for NaN opacity: keep all)
        if (smax == smax) qmask = 0u;
        return;
    }
    // Points beyond k times the bounding box of {sigma <= smax} have exact sigma >= k^2 smax.
    // The evaluated sigma differs from the exact one by at most ~6e-7 * cond(Q) relative (Q the
    // conic), so with cond(Q) <= (a + c)^2 / det < 1e4 and k = 1.01 every point outside the box
    // evaluates above smax. Worse-conditioned conics keep all four quadrants.
    const float det = a * c - b * b;
    const float tr = a + c;
    const float ex2 = 2.0f * smax * c / det, ey2 = 2.0f * smax * a / det;
    if (a > 0.0f && c > 0.0f && det > 0.0f && tr * tr < 1e4f * det && ex2 < 1e30f &&
        ey2 < 1e30f) {
        const float ex = sqrtf(ex2) * 1.01f + 0.01f, ey = sqrtf(ey2) * 1.01f + 0.01f;
        qmask = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float x0 = (float)(tile_x * kBlockWidth + (q & 1) * 8) + 0.5f;
            const float y0 = (float)(tile_y * kBlockWidth + (q >> 1) * 8) + 0.5f;
            const bool hit = (x + ex >= x0) && (x - ex <= x0 + 7.0f) && (y + ey >= y0) &&
                             (y - ey <= y0 + 7.0f);
            qmask |= hit ? (1u << q) : 0u;
        }
    }
}

// ------------------------------------------------------------------ forward
// _rasterize_kernel, splax/_rasterize/_kernels.py:102-205

struct BlendFwdParams {
    BlendCommon c;
    float* final_Ts; int32_t* final_idx; float* out_img;
};

__global__ void __launch_bounds__(kTile) blend_fwd_kernel(BlendFwdParams P) {
    __shared__ float s_x[kTile], s_y[kTile], s_a[kTile], s_b[kTile], s_c[kTile], s_o[kTile];
    __shared__ float s_smax[kTile], s_r[kTile], s_g[kTile], s_bl[kTile];
    __shared__ uint32_t s_q[kTile];

    const BlendCommon& C = P.c;
    const int tid = threadIdx.x, wave = tid >> 6;
    const int32_t tile_g = blockIdx.x;
    const int32_t image_id = tile_g / C.num_tiles;
    const int32_t tile_local = tile_g - image_id * C.num_tiles;
    const int tile_x = tile_local % C.tiles_x, tile_y = tile_local / C.tiles_x;
    int i, j;
    tile_pixel(tid, tile_x, tile_y, i, j);
    const float px = (float)j + 0.5f, py = (float)i + 0.5f;
    const bool inside = i < C.img_h && j < C.img_w;
    bool done = !inside;

    const int32_t range_start = C.bins[2 * tile_g], range_end = C.bins[2 * tile_g + 1];
    const int32_t num_batches = (range_end - range_start + kTile - 1) / kTile;
    float T = 1.0f;
    int32_t cur_idx = 0;
    float o0 = 0.f, o1 = 0.f, o2 = 0.f;
    const uint32_t wbit = 1u << wave;

    for (int32_t bt = 0; bt < num_batches; ++bt) {
        // every pixel done -> stop; also the barrier before the LDS records are overwritten
        if (__syncthreads_count(done) >= kTile) break;
        const int32_t batch_start = range_start + bt * kTile;
        {
            const int32_t src = iminw(batch_start + tid, range_end - 1);
            const int64_t g = C.ids[src];
            const float2 xy = reinterpret_cast<const float2*>(C.xys)[g];
            const float a = C.conics[3 * g], b = C.conics[3 * g + 1], c = C.conics[3 * g + 2];
            const float o = C.opac[g % C.rows_opac];
            const int64_t cg = g % C.rows_colors;
            float smax;
            uint32_t qm;
            stage_bounds(xy.x, xy.y, a, b, c, o, tile_x, tile_y, smax, qm);
            s_x[tid] = xy.x; s_y[tid] = xy.y;
            s_a[tid] = a; s_b[tid] = b; s_c[tid] = c; s_o[tid] = o;
            s_smax[tid] = smax; s_q[tid] = qm;
            s_r[tid] = C.colors[3 * cg]; s_g[tid] = C.colors[3 * cg + 1];
            s_bl[tid] = C.colors[3 * cg + 2];
        }
        __syncthreads();
        const int32_t batch_size = iminw(kTile, range_end - batch_start);
        if (__ballot(!done) == 0ull) continue;
        for (int32_t t = 0; t < batch_size; ++t) {
            if (!(s_q[t] & wbit)) continue;
            const float dx = s_x[t] - px, dy = s_y[t] - py;
            const float sigma = 0.5f * (s_a[t] * dx * dx + s_c[t] * dy * dy) + s_b[t] * dx * dy;
            if (done || sigma > s_smax[t] || sigma < 0.0f) continue;
            const float alpha = minw(kAlphaMax, s_o[t] * det_expf(-sigma));
            if (alpha < kAlphaThresh) continue;
            const float next_T = T * (1.0f - alpha);
            if (next_T <= kTEps) {
                done = true;
                continue;
            }
            const float vis = alpha * T;
            o0 = o0 + s_r[t] * vis;
            o1 = o1 + s_g[t] * vis;
            o2 = o2 + s_bl[t] * vis;
            T = next_T;
            cur_idx = batch_start + t;
        }
    }
    if (inside) {
        const int64_t bgi = C.rows_bg > 1 ? image_id : 0;
        const float* bg = C.background + 3 * bgi;
        const int64_t pix = ((int64_t)image_id * C.img_h + i) * C.img_w + j;
        P.final_Ts[pix] = T;
        P.final_idx[pix] = cur_idx;
        P.out_img[3 * pix] = o0 + T * bg[0];
        P.out_img[3 * pix + 1] = o1 + T * bg[1];
        P.out_img[3 * pix + 2] = o2 + T * bg[2];
    }
}

int launch_blend_fwd(const RasterInputs& in, const KeyLayout& lay, const int32_t* sorted_ids,
                     const int32_t* tile_bins, float* final_Ts, int32_t* final_idx,
                     float* out_img, hipStream_t stream) {
    const int64_t blocks = (int64_t)in.B_geom * lay.num_tiles;
    if (blocks <= 0) return 0;
    BlendFwdParams P;
    P.c.colors = in.colors; P.c.rows_colors = in.rows_colors;
    P.c.opac = in.opac; P.c.rows_opac = in.rows_opac;
    P.c.background = in.background; P.c.rows_bg = in.rows_bg;
    P.c.xys = in.xys; P.c.conics = in.conics;
    P.c.ids = sorted_ids; P.c.bins = tile_bins;
    P.c.img_h = in.img_h; P.c.img_w = in.img_w;
    P.c.tiles_x = lay.tiles_x; P.c.num_tiles = lay.num_tiles;
    P.final_Ts = final_Ts; P.final_idx = final_idx; P.out_img = out_img;
    hipLaunchKernelGGL(blend_fwd_kernel, dim3((unsigned)blocks), dim3(kTile), 0, stream, P);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

// ------------------------------------------------------------------ backward
// _rasterize_bwd_kernel, splax/_rasterize/_kernels.py:530-665, with _blend_color_vjp
// (:1212-1254). Pairs visited per pixel: sorted indices bin_final down to range_start.

struct BlendBwdParams {
    BlendCommon c;
    const float* final_Ts; const int32_t* final_idx;
    const float* v_out; int64_t vout_rows;
    int32_t n; int32_t sel_geom;
    float* v_colors; float* v_opacity; float* v_xy; float* v_conic;
};

__global__ void __launch_bounds__(kTile) blend_bwd_kernel(BlendBwdParams P) {
    __shared__ float s_x[kTile], s_y[kTile], s_a[kTile], s_b[kTile], s_c[kTile], s_o[kTile];
    __shared__ float s_smax[kTile], s_r[kTile], s_g[kTile], s_bl[kTile];
    __shared__ uint32_t s_q[kTile];
    __shared__ int32_t s_id[kTile];
    __shared__ float s_acc[9][kTile];
    __shared__ int32_t s_max;

    const BlendCommon& C = P.c;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int32_t tile_g = blockIdx.x;  // (output image, tile)
    const int32_t image_id = tile_g / C.num_tiles;
    const int32_t tile_local = tile_g - image_id * C.num_tiles;
    const int32_t geom_image = P.sel_geom ? image_id : 0;
    const int64_t og_base = P.sel_geom ? 0 : (int64_t)image_id * P.n;
    const int tile_x = tile_local % C.tiles_x, tile_y = tile_local / C.tiles_x;
    const int32_t gtile = geom_image * C.num_tiles + tile_local;
    const int32_t range_start = C.bins[2 * gtile], range_end = C.bins[2 * gtile + 1];
    if (range_end <= range_start) return;  // uniform per workgroup
    int i, j;
    tile_pixel(tid, tile_x, tile_y, i, j);
    const float px = (float)j + 0.5f, py = (float)i + 0.5f;
    const bool inside = i < C.img_h && j < C.img_w;
    int32_t bin_final = range_start - 1;
    float T = 1.0f, t_final = 1.0f;
    float v0 = 0.f, v1 = 0.f, v2 = 0.f, bg0 = 0.f, bg1 = 0.f, bg2 = 0.f;
    if (inside) {
        const int64_t frow = (int64_t)geom_image * C.img_h + i;
        bin_final = P.final_idx[frow * C.img_w + j];
        t_final = P.final_Ts[frow * C.img_w + j];
        T = t_final;
        const int64_t vrow = ((int64_t)image_id * C.img_h + i) % P.vout_rows;
        const float* vo = P.v_out + 3 * (vrow * C.img_w + j);
        v0 = vo[0]; v1 = vo[1]; v2 = vo[2];
        const float* bg = C.background + 3 * (C.rows_bg > 1 ? image_id : 0);
        bg0 = bg[0]; bg1 = bg[1]; bg2 = bg[2];
    }
    float buf0 = 0.f, buf1 = 0.f, buf2 = 0.f;
    if (tid == 0) s_max = range_start - 1;
#pragma unroll
    for (int k = 0; k < 9; ++k) s_acc[k][tid] = 0.0f;
    __syncthreads();
    atomicMax(&s_max, bin_final);
    // wave-wide largest final index: a record above it has no contributing lane in this wave
    int32_t wmax = bin_final;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        int32_t o = __shfl_xor(wmax, off, 64);
        wmax = o > wmax ? o : wmax;
    }
    __syncthreads();
    // a final_idx from the matching forward lies inside the tile's range; clamp anything else
    const int32_t start_idx = iminw(s_max, range_end - 1);
    const int32_t num_batches = (start_idx - range_start + kTile) / kTile;
    const uint32_t wbit = 1u << wave;

    for (int32_t bt = 0; bt < num_batches; ++bt) {
        const int32_t batch_end = start_idx - bt * kTile;
        {
            const int32_t src = imaxw(batch_end - tid, range_start);
            const int64_t g = C.ids[src];
            const float2 xy = reinterpret_cast<const float2*>(C.xys)[g];
            const float a = C.conics[3 * g], b = C.conics[3 * g + 1], c = C.conics[3 * g + 2];
            const float o = C.opac[g % C.rows_opac];
            const int64_t cg = g % C.rows_colors;
            float smax;
            uint32_t qm;
            stage_bounds(xy.x, xy.y, a, b, c, o, tile_x, tile_y, smax, qm);
            s_x[tid] = xy.x; s_y[tid] = xy.y;
            s_a[tid] = a; s_b[tid] = b; s_c[tid] = c; s_o[tid] = o;
            s_smax[tid] = smax; s_q[tid] = qm; s_id[tid] = (int32_t)g;
            s_r[tid] = C.colors[3 * cg]; s_g[tid] = C.colors[3 * cg + 1];
            s_bl[tid] = C.colors[3 * cg + 2];
        }
        __syncthreads();
        const int32_t batch_size = iminw(kTile, batch_end - range_start + 1);
        for (int32_t t = 0; t < batch_size; ++t) {
            const int32_t idx = batch_end - t;
            if (idx > wmax || !(s_q[t] & wbit)) continue;  // wave-uniform
            const float dx = s_x[t] - px, dy = s_y[t] - py;
            const float a = s_a[t], b = s_b[t], c = s_c[t];
            const float sigma = 0.5f * (a * dx * dx + c * dy * dy) + b * dx * dy;
            bool valid = idx <= bin_final && !(sigma > s_smax[t]) && sigma >= 0.0f;
            float g0 = 0.f, g1 = 0.f, g2 = 0.f, g3 = 0.f, g4 = 0.f, g5 = 0.f, g6 = 0.f, g7 = 0.f,
                  g8 = 0.f;
            if (valid) {
                const float op = s_o[t];
                const float vis = det_expf(-sigma);
                const float alpha = minw(kAlphaMax, op * vis);
                if (alpha < kAlphaThresh) {
                    valid = false;
                } else {
                    const float cr = s_r[t], cgc = s_g[t], cb = s_bl[t];
                    const float ra = 1.0f / (1.0f - alpha);
                    T = T * ra;
                    const float fac = alpha * T;
                    float v_alpha = (cr * T - buf0 * ra) * v0;
                    v_alpha += (cgc * T - buf1 * ra) * v1;
                    v_alpha += (cb * T - buf2 * ra) * v2;
                    v_alpha += -t_final * ra * bg0 * v0;
                    v_alpha += -t_final * ra * bg1 * v1;
                    v_alpha += -t_final * ra * bg2 * v2;
                    buf0 = buf0 + cr * fac;
                    buf1 = buf1 + cgc * fac;
                    buf2 = buf2 + cb * fac;
                    g0 = v0 * fac;
                    g1 = v1 * fac;
                    g2 = v2 * fac;
                    if (op * vis <= kAlphaMax) {
                        const float v_sigma = -op * vis * v_alpha;
                        g3 = 0.5f * v_sigma * dx * dx;
                        g4 = v_sigma * dx * dy;
                        g5 = 0.5f * v_sigma * dy * dy;
                        g6 = v_sigma * (a * dx + b * dy);
                        g7 = v_sigma * (b * dx + c * dy);
                        g8 = vis * v_alpha;
                    }
                }
            }
            if (__ballot(valid) == 0ull) continue;
            const float r0 = wave_sum_to_lane63(g0), r1 = wave_sum_to_lane63(g1);
            const float r2 = wave_sum_to_lane63(g2), r3 = wave_sum_to_lane63(g3);
            const float r4 = wave_sum_to_lane63(g4), r5 = wave_sum_to_lane63(g5);
            const float r6 = wave_sum_to_lane63(g6), r7 = wave_sum_to_lane63(g7);
            const float r8 = wave_sum_to_lane63(g8);
            if (lane == 63) {
                atomicAdd(&s_acc[0][t], r0); atomicAdd(&s_acc[1][t], r1);
                atomicAdd(&s_acc[2][t], r2); atomicAdd(&s_acc[3][t], r3);
                atomicAdd(&s_acc[4][t], r4); atomicAdd(&s_acc[5][t], r5);
                atomicAdd(&s_acc[6][t], r6); atomicAdd(&s_acc[7][t], r7);
                atomicAdd(&s_acc[8][t], r8);
            }
        }
        __syncthreads();
        if (tid < batch_size) {
            const int64_t og = og_base + s_id[tid];
            float acc[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                acc[k] = s_acc[k][tid];
                s_acc[k][tid] = 0.0f;
            }
            if (acc[0] != 0.f || acc[1] != 0.f || acc[2] != 0.f) {
                atomicAdd(P.v_colors + 3 * og, acc[0]);
                atomicAdd(P.v_colors + 3 * og + 1, acc[1]);
                atomicAdd(P.v_colors + 3 * og + 2, acc[2]);
            }
            if (acc[3] != 0.f || acc[4] != 0.f || acc[5] != 0.f) {
                atomicAdd(P.v_conic + 3 * og, acc[3]);
                atomicAdd(P.v_conic + 3 * og + 1, acc[4]);
                atomicAdd(P.v_conic + 3 * og + 2, acc[5]);
            }
            if (acc[6] != 0.f || acc[7] != 0.f) {
                atomicAdd(P.v_xy + 2 * og, acc[6]);
                atomicAdd(P.v_xy + 2 * og + 1, acc[7]);
            }
            if (acc[8] != 0.f) atomicAdd(P.v_opacity + og, acc[8]);
        }
        __syncthreads();
    }
}

int launch_blend_bwd(const RasterInputs& in, const KeyLayout& lay, const int32_t* sorted_ids,
                     const int32_t* tile_bins, const BlendBwdArgs& a, hipStream_t stream) {
    const int64_t nout = (int64_t)a.B_out * in.n;
    int rc = fill_zero_f32(a.v_colors, 3 * nout, stream);
    if (!rc) rc = fill_zero_f32(a.v_opacity, nout, stream);
    if (!rc) rc = fill_zero_f32(a.v_xy, 2 * nout, stream);
    if (!rc) rc = fill_zero_f32(a.v_conic, 3 * nout, stream);
    if (rc) return rc;
    const int64_t blocks = (int64_t)a.B_out * lay.num_tiles;
    if (blocks <= 0 || sorted_ids == nullptr) return 0;
    BlendBwdParams P;
    P.c.colors = in.colors; P.c.rows_colors = in.rows_colors;
    P.c.opac = in.opac; P.c.rows_opac = in.rows_opac;
    P.c.background = in.background; P.c.rows_bg = in.rows_bg;
    P.c.xys = in.xys; P.c.conics = in.conics;
    P.c.ids = sorted_ids; P.c.bins = tile_bins;
    P.c.img_h = in.img_h; P.c.img_w = in.img_w;
    P.c.tiles_x = lay.tiles_x; P.c.num_tiles = lay.num_tiles;
    P.final_Ts = a.final_Ts; P.final_idx = a.final_idx;
    P.v_out = a.v_out; P.vout_rows = a.vout_rows;
    P.n = in.n; P.sel_geom = in.B_geom > 1;
    P.v_colors = a.v_colors; P.v_opacity = a.v_opacity; P.v_xy = a.v_xy; P.v_conic = a.v_conic;
    hipLaunchKernelGGL(blend_bwd_kernel, dim3((unsigned)blocks), dim3(kTile), 0, stream, P);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

}  // namespace splat
