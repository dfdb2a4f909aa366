// Forward and backward alpha blend on gfx950.
//
// One workgroup of 256 threads (four wave64s) per (image, 16x16 tile), as in the reference
// (splax/_rasterize/_kernels.py:63-87,469-500). Each wave owns one 8x8 quadrant of the tile and
// each 16-lane row of a wave one 4x4 sub-block of it. The tile's sorted range is staged in LDS in
// batches of records (three float4 per record; 256 per forward batch, 128 per backward batch).
// Each packed record carries
//   - sigma_max: a conservative bound (log(255 o) + 1e-3) above which o e^-sigma < 1/255, so a
//     lane skips the exponential for pairs the reference rejects anyway,
// and while staging each record gets
//   - a 16-bit sub-block mask: the 4x4 sub-blocks whose pixel centres can reach
//     sigma <= sigma_max (the forward from the ellipse's exact extent per band of rows, the
//     backward from its bounding box);
// and each row then walks only the compacted, order-preserving list of records that reach its
// sub-block (the four rows of a wave walk their own lists in lockstep, each row reading its own
// record, an LDS broadcast within the row). A wave takes as many steps as its longest row list,
// about 0.7 of the quadrant list a whole-wave walk would take. Both filters remove only pairs
// that the reference's `sigma < 0 or alpha < 1/255` test rejects, so the per-pixel sequence of
// blended pairs (and every float operation on it) is the reference's, and the forward image is
// bit-identical to the CPU oracle.
//
// Backward: the same staging walked back to front from the workgroup's largest final_idx, each
// wave over the list of its whole quadrant (per-row walks there cost more in LDS bank conflicts
// and same-record accumulator collisions than they save in steps). A pixel's contribution to a
// record is nine floats; per record the contributing lanes of a wave reduce them with a
// reduce-scatter (v_permlane32_swap, v_permlane16_swap, then bank-masked DPP adds within rows:
// 19 VALU for nine values) and add the totals into the record's LDS accumulator. After each batch every record
// stores its nine sums (plain stores, no global atomics) at its emission position, where all
// intersections of one item are contiguous; grad_gather_kernel then adds them per item in a
// fixed order and writes the four gradient outputs. The LDS sums of one record over the tile's
// four quadrant waves take two accumulator copies, each added into by two waves, so no sum depends
// on the order in which the waves arrive: the backward is deterministic.
#include <hip/hip_ext.h>

#include <type_traits>

#include "splat_common.hpp"
#include "splat_internal.hpp"

namespace splat {

constexpr int kTile = 256;

struct BlendCommon {
    const float* background; int64_t rows_bg;
    const float4* recs;  // packed records, four float4 per geometry item (pack_records_kernel)
    const int32_t* ids; const int32_t* bins;
    const int32_t* order;  // workgroup -> (image, tile), tile_order_kernel
    int32_t img_h, img_w, tiles_x, num_tiles;
    int64_t total;  // geometry rows (B_geom * n): ids outside [0, total) are ignored
};


// Pixel of thread `tid` in its tile: wave w = quadrant (w & 1, w >> 1), row r = lane >> 4 =
// 4x4 sub-block (r & 1, r >> 1) of the quadrant, lane & 15 = 4x4 raster.
__device__ __forceinline__ void tile_pixel(int tid, int tile_x, int tile_y, int& i, int& j) {
    const int wave = tid >> 6, lane = tid & 63, row = lane >> 4, l = lane & 15;
    i = tile_y * kBlockWidth + (wave >> 1) * 8 + (row >> 1) * 4 + (l >> 2);
    j = tile_x * kBlockWidth + (wave & 1) * 8 + (row & 1) * 4 + (l & 3);
}

// Sub-block (0..15, row-major over the tile's 4x4 grid of 4x4 blocks) of the thread's row.
__device__ __forceinline__ int row_subblock(int tid) {
    const int wave = tid >> 6, row = (tid & 63) >> 4;
    return ((wave >> 1) * 2 + (row >> 1)) * 4 + (wave & 1) * 2 + (row & 1);
}

struct PackParams {
    const float* colors; int64_t rows_colors;
    const float* opac; int64_t rows_opac;
    const float* xys; const float* conics; const float* depths;
    int64_t total;
    int32_t compensate;  // blend with opac * rho(conic)
    float4* recs;
};

// One thread per item computes its record; the block's records leave through LDS so that
// consecutive lanes store consecutive float4s.
__global__ void __launch_bounds__(256) pack_records_kernel(PackParams P) {
    __shared__ float4 s_rec[4 * 256];
    const int64_t base = (int64_t)blockIdx.x * 256;
    const int64_t g = base + threadIdx.x;
    if (g < P.total) {
        const float2 xy = reinterpret_cast<const float2*>(P.xys)[g];
        const int64_t cg = g % P.rows_colors;
        pack_record(xy.x, xy.y, P.conics[3 * g], P.conics[3 * g + 1], P.conics[3 * g + 2],
                    P.opac[g % P.rows_opac], P.compensate, P.colors + 3 * cg,
                    P.depths ? P.depths[g] : 0.0f, s_rec + 4 * threadIdx.x);
    }
    __syncthreads();
    const int64_t left = P.total - base;
    const int count = 4 * (int)(left < 256 ? left : 256);
    float4* dst = P.recs + 4 * base;
    for (int k = threadIdx.x; k < count; k += 256) dst[k] = s_rec[k];
}

// Sub-blocks (bit 4 r + c: block row r, column c of the tile's 4x4 grid of 4x4 pixel blocks)
// of the tile at (tile_x, tile_y) whose pixel centres a packed record can reach.
__device__ __forceinline__ uint32_t subblock_mask(const float4& r0, const float4& r3,
                                                  int tile_x, int tile_y) {
    const uint32_t mode = __float_as_uint(r3.z);
    if (mode == kCullNone) return 0u;
    if (mode != kCullBox) return 0xffffu;
    uint32_t xm = 0u, ym = 0u;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float x0 = (float)(tile_x * kBlockWidth + c * 4) + 0.5f;
        const float y0 = (float)(tile_y * kBlockWidth + c * 4) + 0.5f;
        xm |= ((r0.x + r3.x >= x0) && (r0.x - r3.x <= x0 + 3.0f)) ? (1u << c) : 0u;
        ym |= ((r0.y + r3.y >= y0) && (r0.y - r3.y <= y0 + 3.0f)) ? (1u << c) : 0u;
    }
    uint32_t m = 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r) m |= ((ym >> r) & 1u) ? (xm << (4 * r)) : 0u;
    return m;
}

// The forward's sub-block mask: the sub-blocks whose pixel centres the record can reach, from the
// exact x-extent of its ellipse over each 4-row band of the tile's pixel centres (the box test
// above also keeps sub-blocks that only the box's corners reach; on config 2 the forward's row
// walks take 23% fewer steps with this mask).
// With Q(dx, dy) = a/2 dx^2 + b dx dy + c/2 dy^2 (dx, dy from the centre), the test uses the
// ellipse Q <= s' with s' = 1.0201 sigma_max, i.e. {sigma <= sigma_max} scaled by 1.01: an
// evaluated sigma <= sigma_max has an exact Q within 0.6% of it for the conics the box mode
// accepts ((a + c)^2 / det < 1e4), so every such pixel centre lies inside. The chord of that
// ellipse at height dy is centred at -b dy / a with half-width sqrt(2 a s' - det dy^2) / a, so its
// right end is concave in dy and peaks at the rightmost point (dx, dy) = (ex, -b ex / c), ex =
// sqrt(2 s' c / det); over a band [dy0, dy1] clipped to |dy| <= ey the extent is therefore
// [min of the left ends at dy0 and dy1, or -ex when the leftmost point lies in the band,
//  max of the right ends, or ex when the rightmost point lies in it], widened by m = 0.01 px +
// 1e-3 ex against rounding (the rows are clipped to |dy| <= ey + m, where the chord's width is
// taken as 0 beyond ey). A sub-block is kept when its pixel-centre columns meet that extent.
constexpr float kTightScale2 = 1.0201f;

// The tile-relative quantities of that test for one kCullBox record. The record carries the
// tile-independent parts, formed once per item by the pack: 1 / a in r1.w, the scaled ellipse's
// half-widths as the box's minus its 0.01 px, and the rightmost point's height in r3.w.
struct TightEllipse {
    float det, inv_a, ex, ey, dy_r, m, two_a_s, nb_a, bx, by;
};
__device__ __forceinline__ TightEllipse tight_setup(const float4& r0, const float4& r1,
                                                    const float4& r3, int tile_x, int tile_y) {
    TightEllipse e;
    const float a = 2.0f * r0.z, b = r0.w, c = 2.0f * r1.x;
    const float s2 = 2.0f * (kTightScale2 * r1.z);  // 2 s'
    e.det = a * c - b * b;
    e.inv_a = r1.w;
    e.ex = r3.x - 0.01f;
    e.ey = r3.y - 0.01f;
    e.dy_r = r3.w;  // rightmost point; leftmost at -dy_r
    e.m = 0.01f + 1e-3f * e.ex;
    e.two_a_s = a * s2;
    e.nb_a = -b * e.inv_a;
    e.bx = (float)(tile_x * kBlockWidth) + 0.5f - r0.x;  // dx of the tile's first column
    e.by = (float)(tile_y * kBlockWidth) + 0.5f - r0.y;
    return e;
}

// Bits 4 j .. 4 j + 3 of the mask: the sub-blocks of band j (pixel-centre rows 4 j .. 4 j + 3).
__device__ __forceinline__ uint32_t tight_band(const TightEllipse& e, int j) {
    const float y0 = e.by + (float)(4 * j);
    const float d0 = fmaxf(y0, -e.ey - e.m), d1 = fminf(y0 + 3.0f, e.ey + e.m);
    const float w0 = __builtin_amdgcn_sqrtf(fmaxf(e.two_a_s - e.det * (d0 * d0), 0.0f)) * e.inv_a;
    const float w1 = __builtin_amdgcn_sqrtf(fmaxf(e.two_a_s - e.det * (d1 * d1), 0.0f)) * e.inv_a;
    const float c0 = e.nb_a * d0, c1 = e.nb_a * d1;
    float hi = fmaxf(c0 + w0, c1 + w1), lo = fminf(c0 - w0, c1 - w1);
    hi = (e.dy_r >= d0 && e.dy_r <= d1) ? e.ex : hi;
    lo = (-e.dy_r >= d0 && -e.dy_r <= d1) ? -e.ex : lo;
    hi = hi + e.m;
    lo = lo - e.m;
    const bool band = d0 <= d1;  // the band's rows meet |dy| <= ey + m
    uint32_t bits = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x0 = e.bx + (float)(4 * i);
        bits |= (band && x0 <= hi && x0 + 3.0f >= lo) ? (1u << (4 * j + i)) : 0u;
    }
    return bits;
}

__device__ __forceinline__ uint32_t subblock_mask_tight(const float4& r0, const float4& r1,
                                                        const float4& r3, int tile_x,
                                                        int tile_y) {
    const uint32_t mode = __float_as_uint(r3.z);
    if (mode == kCullNone) return 0u;
    if (mode != kCullBox) return 0xffffu;
    const TightEllipse e = tight_setup(r0, r1, r3, tile_x, tile_y);
    uint32_t mask = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) mask |= tight_band(e, j);
    return mask;
}

// LDS records of one batch: r0 = (x, y, a/2, b), r1 = (c/2, o, sigma_max, 1/a), r2 = (red, green,
// blue, depth), each record's sub-block mask, and compacted record lists: with kRows (the
// forward) one per sub-block, of record byte offsets (16 t for slot t: the address needs no
// shift), otherwise (the backward) one per quadrant wave, of slot indices. The backward's four
// lists (with 128-record batches and two accumulator copies) keep its LDS at 19.7 KB.
template <bool kRows, int kBatch>
struct BatchLds {
    float4 r0[kBatch];
    float4 r1[kBatch];
    float4 r2[kBatch];
    uint16_t mask[kBatch];
    // a backward wave reads its whole list row as one dword per lane: rows of kTile bytes
    typename std::conditional<kRows, uint16_t, uint8_t>::type list[kRows ? 16 : 4][kTile];
};
// Records per batch of the backward: 128 keeps its LDS (records, lists and two accumulator
// copies) at 19.7 KB, so with at most 64 VGPRs eight workgroups share a CU (eight waves per SIMD).
constexpr int kBwdBatch = 128;

// Stages the record of item `id` (the sorted range's entry for slot `tid`) into slot `tid` (one
// barrier), then each wave builds its own record lists from the staged masks, in slot order:
// with kRows the lists of its four sub-blocks (one per 16-lane row), otherwise the list of its
// whole quadrant (a record reaches a quadrant when it reaches one of its sub-blocks, which is the
// 8x8 box test). `live` is false for the clamped tail slots of the last batch (they reach no
// sub-block). Returns the length of the wave's longest list, with kRows plus 65536 times the
// calling lane's row list length.
template <bool kRows, int kBatch>
__device__ __forceinline__ int stage_batch(const BlendCommon& C, BatchLds<kRows, kBatch>& L,
                                           int32_t id, bool live, int tile_x, int tile_y) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, row = lane >> 4;
    int64_t g = id;
    uint32_t m = 0u;
    float4 r0 = make_float4(0.f, 0.f, 0.f, 0.f), r1 = r0, r2 = r0;
    if (live && g >= 0 && g < C.total) {
        const float4* rec = C.recs + 4 * g;
        r0 = rec[0];
        r1 = rec[1];
        r2 = rec[2];
        m = kRows ? subblock_mask_tight(r0, r1, rec[3], tile_x, tile_y)
                  : subblock_mask(r0, rec[3], tile_x, tile_y);
    }
    if (kBatch == kTile || tid < kBatch) {
        L.r0[tid] = r0;
        L.r1[tid] = r1;
        L.r2[tid] = r2;
        L.mask[tid] = (uint16_t)m;
    }
    __syncthreads();
    // this wave's sub-blocks: rows 0..3 -> sb0, sb0 + 1, sb0 + 4, sb0 + 5
    const int sb0 = (wave >> 1) * 8 + (wave & 1) * 2;
    const uint64_t lt = (1ull << lane) - 1ull;
    if constexpr (kRows) {
        int n[4] = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < (kBatch + 63) / 64; ++c) {
            const uint32_t mc =
                (kBatch % 64 == 0 || c * 64 + lane < kBatch) ? L.mask[c * 64 + lane] : 0u;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int b = sb0 + (r & 1) + (r >> 1) * 4;
                const bool bit = (mc >> b) & 1u;
                const uint64_t bal = __ballot(bit);
                if (bit) L.list[b][n[r] + (int)__popcll(bal & lt)] = (uint16_t)((c * 64 + lane) * 16);
                n[r] += (int)__popcll(bal);
            }
        }
        __builtin_amdgcn_wave_barrier();
        const int mine = row == 0 ? n[0] : row == 1 ? n[1] : row == 2 ? n[2] : n[3];
        const int a = n[0] > n[1] ? n[0] : n[1], b = n[2] > n[3] ? n[2] : n[3];
        return (a > b ? a : b) | (mine << 16);
    } else {
        const uint32_t qbits = (0x33u << sb0);  // the quadrant's four sub-blocks
        int nq = 0;
#pragma unroll
        for (int c = 0; c < (kBatch + 63) / 64; ++c) {
            const bool bit = (kBatch % 64 == 0 || c * 64 + lane < kBatch) &&
                             (L.mask[c * 64 + lane] & qbits) != 0u;
            const uint64_t bal = __ballot(bit);
            if (bit) L.list[wave][nq + (int)__popcll(bal & lt)] = (uint8_t)(c * 64 + lane);
            nq += (int)__popcll(bal);
        }
        __builtin_amdgcn_wave_barrier();
        return nq;
    }
}

// Wave-uniform value as a scalar (the compiler cannot prove uniformity of values derived from
// threadIdx.x / LDS on its own; scalar loop control avoids exec-mask branching).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// e^x for x in [-88, 0] (no range handling needed there); equal to det_expf on that domain.
// e^x for the blends' x = -sigma (x <= 0; below 2^-126 the result is garbage, tiny, negative or
// NaN, and every such alpha fails the 1/255 test as the exact one would for opacities below
// 1e30):
// k = round(x log2 e) by adding 1.5 * 2^23, whose integer then sits in the sum's low mantissa
// bits; r = x - k ln2 with float ln2 in one FMA (the blends' |k| is small, so k (ln2 - fl(ln2))
// stays far below an ulp); a degree-6 polynomial of e^r with c0 = c1 = 1 fitted by Lawson's
// iteration (relative error 4.4e-9 on |r| <= ln2 / 2 with these float coefficients); 2^k added
// to the exponent field. At most 1 ulp from e^x on [-8, 0], 2 ulp down to -30 and 5 ulp down to
// -87 (the reduction's error grows with |k|). Ten VALU; the CPU oracle evaluates the same
// sequence.
constexpr float kBlendLn2 = 0x1.62e430p-1f;
constexpr float kBlendExpC5 = 0x1.123a6cp-7f;
__device__ __forceinline__ float blend_exp(float x, float round_c = 0x1.8p23f,
                                           float c5 = kBlendExpC5) {
    // round_c = 1.5 * 2^23 and c5 may come in as register copies of the constants
    const float t = fmaf(x, kLog2e, round_c);
    const float kf = t - 0x1.8p23f;
    const float r = fmaf(kf, -kBlendLn2, x);
    float p = fmaf(r, 0x1.6a2352p-10f, c5);
    p = fmaf(r, p, 0x1.5558f4p-5f);
    p = fmaf(r, p, 0x1.55549p-3f);
    p = fmaf(r, p, 0x1.fffffcp-2f);
    p = fmaf(r, p, 1.0f);
    p = fmaf(r, p, 1.0f);
    return __uint_as_float(__float_as_uint(p) + (__float_as_uint(t) << 23));
}

// The Gaussian exponent 0.5 (a dx^2 + c dy^2) + b dx dy of a packed record (r0.z = a/2,
// r0.w = b, r1.x = c/2) as dx (a/2 dx + b dy) + (c/2 dy) dy: two FMAs, seven VALU with the
// offsets. The CPU oracle evaluates the same expression.
__device__ __forceinline__ float blend_sigma(const float4& r0, const float4& r1, float dx,
                                             float dy) {
    return fmaf(dx, fmaf(r0.z, dx, r0.w * dy), (r1.x * dy) * dy);
}

// 0 <= sigma <= sigma_max as one unsigned compare of the float bits (one VALU where two float
// compares take two). Equal for every record a list holds: its sigma_max is >= 0 and not NaN
// (a record with sigma_max < 0 or NaN is kCullNone and reaches no sub-block); sigma is never
// -0.0 (with c > 0 the term (c/2 dy) dy is +0 or positive, and a rounded sum is -0.0 only when
// both addends are), so a negative sigma has its sign bit set and fails, as a NaN does.
__device__ __forceinline__ bool sigma_in_range(float sigma, float sigma_max) {
    return __float_as_uint(sigma) <= __float_as_uint(sigma_max);
}

// ------------------------------------------------------------------ forward
// _rasterize_kernel, splax/_rasterize/_kernels.py:102-205

struct BlendFwdParams {
    BlendCommon c;
    float* final_Ts; int32_t* final_idx; float* out_img;
    float* out_depth;  // kDepth: expected depth per pixel
    // fused loss (loss_kind != kLossNone): the tile's sum of (img - target)^2 or |img - target|
    // over its pixels' colour values into loss_partials[tile_g]
    int32_t loss_kind; const float* loss_target; double* loss_partials;
};

// kDepth adds the expected-depth channel of _rasterize_depth_kernel
// (splax/_rasterize/_kernels.py:277-383): depth times the same blend weight, no background term.
// At most 72 VGPRs: seven waves per SIMD (0.187 ms at config 2 against 0.195 at the compiler's
// own 79 VGPRs and six; forcing eight spills registers).
template <bool kDepth>
__global__ void __launch_bounds__(kTile, 7) blend_fwd_kernel(BlendFwdParams P) {
    __shared__ BatchLds<true, kTile> L;
    const BlendCommon& C = P.c;
    const int tid = threadIdx.x;
    const int32_t tile_g = C.order[blockIdx.x];
    const int32_t image_id = tile_g / C.num_tiles;
    const int32_t tile_local = tile_g - image_id * C.num_tiles;
    const int tile_x = tile_local % C.tiles_x, tile_y = tile_local / C.tiles_x;
    int i, j;
    tile_pixel(tid, tile_x, tile_y, i, j);
    const int sb = row_subblock(tid);
    const float px = (float)j + 0.5f, py = (float)i + 0.5f;
    const bool inside = i < C.img_h && j < C.img_w;
    bool done = !inside;

    const int32_t range_start = C.bins[2 * tile_g], range_end = C.bins[2 * tile_g + 1];
    const int32_t num_batches = (range_end - range_start + kTile - 1) / kTile;
    float T = 1.0f;
    int32_t cur_idx = 0;
    float o0 = 0.f, o1 = 0.f, o2 = 0.f, od = 0.f;
    // blend_exp's constants that enter as addends held in registers (the compiler would
    // re-materialize them in every step)
    float exp_round = 0x1.8p23f, exp_c5 = kBlendExpC5;
    asm volatile("" : "+v"(exp_round), "+v"(exp_c5));
    const char* rec_base = reinterpret_cast<const char*>(L.r0);

    for (int32_t bt = 0; bt < num_batches; ++bt) {
        // every pixel done -> stop; also the barrier before the LDS records are overwritten
        if (__syncthreads_count(done) >= kTile) break;
        const int32_t batch_start = range_start + bt * kTile;
        const int32_t src = iminw(batch_start + tid, range_end - 1);
        const int lens = stage_batch<true, kTile>(C, L, C.ids[src], batch_start + tid < range_end,
                                                  tile_x, tile_y);
        if (__ballot(!done) == 0ull) continue;
        const int wave_max = lens & 0xffff, my_len = lens >> 16;  // my_len uniform per row
        const uint16_t* list = L.list[sb];
        int32_t last_off = -1;  // the last accepted record of this batch (byte offset)
        for (int k = 0; k < wave_max; ++k) {
            // A lane leaves once its pixel is done or its row's list is walked; the wave walks
            // while any lane is left, which is exec-mask bookkeeping only. (Padding the shorter
            // lists with a record no pixel accepts instead of the length test measured slower.)
            if (done || k >= my_len) break;
            const int off = list[k];
            const float4 r0 = *reinterpret_cast<const float4*>(rec_base + off);
            const float4 r1 = *reinterpret_cast<const float4*>(rec_base + off + sizeof(L.r0));
            // all of r1 in the first read (one full-width read, one address)
            asm volatile("" ::"v"(r1.y));
            const float dx = r0.x - px, dy = r0.y - py;
            const float sigma = blend_sigma(r0, r1, dx, dy);
            // Nested conditions and the one exit above: every other path falls through to the
            // next step, which keeps the loop's control flow in the exec mask.
            if (sigma_in_range(sigma, r1.z)) {
                // v_min: no accepted record has a NaN opacity (the pack culls those), so it
                // equals the reference's compare-and-select minimum here
                const float alpha = fminf(kAlphaMax, r1.y * blend_exp(-sigma, exp_round, exp_c5));
                if (alpha >= kAlphaThresh) {
                    const float next_T = T * (1.0f - alpha);
                    if (next_T <= kTEps) {
                        done = true;  // leaves at the next step
                    } else {
                        const float4 r2 = *reinterpret_cast<const float4*>(
                            rec_base + off + 2 * sizeof(L.r0));
                        const float vis = alpha * T;
                        o0 = fmaf(r2.x, vis, o0);
                        o1 = fmaf(r2.y, vis, o1);
                        o2 = fmaf(r2.z, vis, o2);
                        if constexpr (kDepth) od = fmaf(r2.w, vis, od);
                        T = next_T;
                        last_off = off;
                    }
                }
            }
        }
        if (last_off >= 0) cur_idx = batch_start + (last_off >> 4);
    }
    double err = 0.0;  // this pixel's part of the fused loss
    if (inside) {
        const int64_t bgi = C.rows_bg > 1 ? image_id : 0;
        const float* bg = C.background + 3 * bgi;
        const int64_t pix = ((int64_t)image_id * C.img_h + i) * C.img_w + j;
        // final_Ts / final_idx serve the backward only: a forward-only caller may pass neither
        if (P.final_Ts) P.final_Ts[pix] = T;
        if (P.final_idx) P.final_idx[pix] = cur_idx;
        const float c0 = o0 + T * bg[0], c1 = o1 + T * bg[1], c2 = o2 + T * bg[2];
        P.out_img[3 * pix] = c0;
        P.out_img[3 * pix + 1] = c1;
        P.out_img[3 * pix + 2] = c2;
        if constexpr (kDepth) P.out_depth[pix] = od;
        if (P.loss_kind != kLossNone) {
            // each term exact in double ((float)d^2 has at most 48 significant bits)
            const float* tg = P.loss_target + 3 * pix;
            const float d0 = c0 - tg[0], d1 = c1 - tg[1], d2 = c2 - tg[2];
            err = P.loss_kind == kLossMse
                      ? ((double)d0 * (double)d0 + (double)d1 * (double)d1) + (double)d2 * (double)d2
                      : ((double)fabsf(d0) + (double)fabsf(d1)) + (double)fabsf(d2);
        }
    }
    if (P.loss_kind != kLossNone) {  // uniform; every lane active again for the DPP sum
        __shared__ double s_err[kTile / 64];
        err = wave_sum_f64_to_lane63(err);
        if ((tid & 63) == 63) s_err[tid >> 6] = err;
        __syncthreads();
        if (tid == 0)
            P.loss_partials[tile_g] = ((s_err[0] + s_err[1]) + s_err[2]) + s_err[3];
    }
}

// Packs the records of the in.B_geom * in.n geometry items into recs.
int launch_pack_records(const RasterInputs& in, float4* recs, hipStream_t stream) {
    PackParams K;
    K.colors = in.colors; K.rows_colors = in.rows_colors;
    K.opac = in.opac; K.rows_opac = in.rows_opac;
    K.xys = in.xys; K.conics = in.conics; K.depths = in.depths;
    K.compensate = in.compensate;
    K.total = (int64_t)in.B_geom * in.n;
    K.recs = recs;
    if (K.total <= 0) return 0;
    hipLaunchKernelGGL(pack_records_kernel, dim3((unsigned)((K.total + 255) / 256)), dim3(256),
                       0, stream, K);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

static void fill_common(BlendCommon& c, const RasterInputs& in, const KeyLayout& lay,
                        const int32_t* sorted_ids, const int32_t* tile_bins) {
    c.background = in.background; c.rows_bg = in.rows_bg;
    c.recs = nullptr;
    c.ids = sorted_ids; c.bins = tile_bins; c.order = nullptr;
    c.img_h = in.img_h; c.img_w = in.img_w;
    c.tiles_x = lay.tiles_x; c.num_tiles = lay.num_tiles;
    c.total = (int64_t)in.B_geom * in.n;
}

// ------------------------------------------------------------------ tile dispatch order
// Workgroup b of a blend takes tile order[b]. The images stay in order, so one image's records
// and lists are what the caches hold at a time; inside an image the tiles go by descending
// intersection count, in buckets of eight per octave, so the longest tiles start first and each
// image ends with short ones instead of a straggler. Any permutation gives the same outputs (each
// workgroup owns its tile's pixels and its intersections' gradient slots); positions inside a
// bucket come from LDS atomics.

constexpr int kOrderThreads = 1024;

// 0 for an empty tile, else monotone in the count: c below 8 as is, then 8 steps per octave
// (at most 247 for an int32 count).
__device__ __forceinline__ int order_bucket(int32_t c) {
    if (c <= 0) return 0;
    const int e = 31 - __clz(c);
    return e < 3 ? c : e * 8 + ((c >> (e - 3)) & 7);
}

// Exclusive scan of the 256 bucket counts in s_cnt, in place: waves 0-3 (threads 0-255) scan
// by DPP, then add the totals of the waves before them. Every thread of the workgroup calls it.
__device__ __forceinline__ void order_scan(uint32_t* s_cnt, uint32_t* s_tot, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    uint32_t v = 0, incl = 0;
    if (tid < 256) {
        v = s_cnt[tid];
        incl = (uint32_t)wave_inclusive_scan_i32((int32_t)v, lane);
        if (lane == 63) s_tot[wave] = incl;
    }
    __syncthreads();
    if (tid < 256) {
        uint32_t before = 0;
        for (int w = 0; w < wave; ++w) before += s_tot[w];
        s_cnt[tid] = before + incl - v;
    }
    __syncthreads();
}

constexpr int kOrderPer = 8;  // tiles per thread kept in registers (images up to 8192 tiles)

// One workgroup per image: bucket histogram of the image's tiles, exclusive scan from the largest
// bucket down, scatter into the image's num_tiles entries of order. Bins of the image's geometry
// (image 0 when the geometry is shared). Up to 8192 tiles every thread loads its counts at once
// and keeps their buckets for the scatter; larger images take two strided passes.
__global__ void __launch_bounds__(kOrderThreads)
tile_order_kernel(const int32_t* bins, int32_t num_tiles, int32_t per_image, int32_t* order) {
    __shared__ uint32_t s_cnt[256], s_tot[4];
    const int tid = threadIdx.x;
    const int64_t image = blockIdx.x;
    const int32_t* ib = bins + 2 * (per_image ? image : 0) * (int64_t)num_tiles;
    const int32_t first = (int32_t)(image * num_tiles);
    if (tid < 256) s_cnt[tid] = 0;
    __syncthreads();
    if (num_tiles <= kOrderThreads * kOrderPer) {
        int bk[kOrderPer];
#pragma unroll
        for (int i = 0; i < kOrderPer; ++i) {
            const int32_t t = i * kOrderThreads + tid;
            bk[i] = t < num_tiles ? 255 - order_bucket(ib[2 * t + 1] - ib[2 * t]) : -1;
        }
#pragma unroll
        for (int i = 0; i < kOrderPer; ++i)
            if (bk[i] >= 0) atomicAdd(&s_cnt[bk[i]], 1u);
        __syncthreads();
        order_scan(s_cnt, s_tot, tid);
#pragma unroll
        for (int i = 0; i < kOrderPer; ++i)
            if (bk[i] >= 0) order[first + atomicAdd(&s_cnt[bk[i]], 1u)] = first + i * kOrderThreads + tid;
        return;
    }
    for (int32_t t = tid; t < num_tiles; t += kOrderThreads)
        atomicAdd(&s_cnt[255 - order_bucket(ib[2 * t + 1] - ib[2 * t])], 1u);
    __syncthreads();
    order_scan(s_cnt, s_tot, tid);
    for (int32_t t = tid; t < num_tiles; t += kOrderThreads) {
        const uint32_t at = atomicAdd(&s_cnt[255 - order_bucket(ib[2 * t + 1] - ib[2 * t])], 1u);
        order[first + at] = first + t;
    }
}

// blocks = images * num_tiles workgroups of a blend.
static int launch_tile_order(const int32_t* bins, int64_t blocks, int32_t num_tiles,
                             int32_t per_image, int32_t* order, hipStream_t stream) {
    hipLaunchKernelGGL(tile_order_kernel, dim3((unsigned)(blocks / num_tiles)),
                       dim3(kOrderThreads), 0, stream, bins, num_tiles, per_image, order);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

int launch_blend_fwd(const RasterInputs& in, const KeyLayout& lay, const int32_t* sorted_ids,
                     const int32_t* tile_bins, float* final_Ts, int32_t* final_idx,
                     float* out_img, float* out_depth, const float4* recs, int32_t* order,
                     const PixelLoss* loss, hipStream_t stream) {
    const int64_t blocks = (int64_t)in.B_geom * lay.num_tiles;
    if (blocks <= 0) return 0;
    int rc = launch_tile_order(tile_bins, blocks, lay.num_tiles, 1, order, stream);
    if (rc) return rc;
    BlendFwdParams P;
    fill_common(P.c, in, lay, sorted_ids, tile_bins);
    P.c.recs = recs;
    P.c.order = order;
    P.final_Ts = final_Ts; P.final_idx = final_idx; P.out_img = out_img;
    P.out_depth = out_depth;
    P.loss_kind = loss ? loss->kind : kLossNone;
    P.loss_target = loss ? loss->target : nullptr;
    P.loss_partials = loss ? loss->partials : nullptr;
    hipEvent_t ka, kb;  // null unless this kernel is timed
    (void)kernel_timer_events(kKernelBlendFwd, &ka, &kb);
    if (out_depth)
        hipExtLaunchKernelGGL(blend_fwd_kernel<true>, dim3((unsigned)blocks), dim3(kTile), 0,
                              stream, ka, kb, 0, P);
    else
        hipExtLaunchKernelGGL(blend_fwd_kernel<false>, dim3((unsigned)blocks), dim3(kTile), 0,
                              stream, ka, kb, 0, P);
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
    const int32_t* pos; int64_t M;
    const float* v_out_depth; int64_t vdepth_rows;  // kDepth
    float* rgrad;  // [images][M][NG], images = 1 when geometry is batched, else B_out
    uint32_t* dev_err;  // the device error word: kDevErrKeptLists when a kept list is bad
    // fused loss (loss_kind != kLossNone): the image cotangent of each pixel from the forward's
    // image, the target and the loss cotangent, as loss_bwd_kernel forms it (v_out unused)
    int32_t loss_kind; const float* loss_target; const float* loss_img; const float* v_loss;
    int64_t loss_count;
};

// Partial sums of one intersection: v_colour (3), v_conic (3), the two sums sum v_sigma * dx,
// sum v_sigma * dy (v_xy before the conic is applied), v_opacity, and with the depth channel
// v_depth (NG = 10).
template <int NG>
__device__ __forceinline__ void store_rgrad(float* rgrad, int64_t slot, const float* s) {
    float* r = rgrad + slot * NG;
#pragma unroll
    for (int k = 0; k < NG; ++k) r[k] = s[k];
}

__device__ __forceinline__ float swap32_add(float a, float b) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                              false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap16_add(float a, float b) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false,
                                              false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// keep + the `send` value of the lane that DPP control kCtrl names (all lanes valid).
template <int kCtrl>
__device__ __forceinline__ float dpp_pair_add(float keep, float send) {
    const int r = __builtin_amdgcn_update_dpp(0, __float_as_int(send), kCtrl, 0xf, 0xf, false);
    return keep + __int_as_float(r);
}

// x + x[row_mirror] (lane l of each 16-lane row with lane 15 - l) written only into the lanes
// of the 4-lane banks kBanks of each row, d kept in the others: one v_add_f32_dpp with a bank
// mask, where a select of what to keep and what to send plus the add take three VALU. The
// compiler does not form the bank-masked add from the DPP builtins, so it is written here, with
// the two wait states a DPP read of a VGPR written by the previous VALU instruction needs.
template <int kBanks>
__device__ __forceinline__ float dpp_add_mirror_banks(float d, float x) {
    static_assert(kBanks == 0x3 || kBanks == 0xc, "banks 0-1 or 2-3");
    if constexpr (kBanks == 0x3)
        asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_mirror row_mask:0xf bank_mask:0x3"
            : "+v"(d) : "v"(x));
    else
        asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_mirror row_mask:0xf bank_mask:0xc"
            : "+v"(d) : "v"(x));
    return d;
}
// The same with row_half_mirror (lane j of each 8-lane half with lane 7 - j): banks 0 and 2
// (kBanks 0x5) or 1 and 3 (0xa).
template <int kBanks>
__device__ __forceinline__ float dpp_add_half_mirror_banks(float d, float x) {
    static_assert(kBanks == 0x5 || kBanks == 0xa, "banks 0 and 2 or 1 and 3");
    if constexpr (kBanks == 0x5)
        asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0x5"
            : "+v"(d) : "v"(x));
    else
        asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0xa"
            : "+v"(d) : "v"(x));
    return d;
}

// Reduce-scatter of three values over each 16-lane row. Lane l pairs with 15 - l (row_mirror):
// the lower half sums a and the upper half b, and c is summed on its own; then lane j of each
// 8-lane half pairs with 7 - j (row_half_mirror), the lower quad summing the a/b partial and the
// upper one c; two quad butterflies finish. Lanes 0-3 of the row then hold the row sum of a,
// lanes 8-11 that of b, lanes 4-7 and 12-15 that of c: seven VALU (the halves' different sums
// are bank-masked DPP adds), where four DPP steps per value take twelve and leave three values to
// add into LDS.
__device__ __forceinline__ float row_reduce_scatter3(float a, float b, float c) {
    float r = dpp_add_mirror_banks<0x3>(a, a);  // lanes 0-7: a + a[15 - l]
    r = dpp_add_mirror_banks<0xc>(r, b);        // lanes 8-15: b + b[15 - l]
    c = dpp_pair_add<0x140>(c, c);              // row_mirror
    float s = dpp_add_half_mirror_banks<0x5>(r, r);  // lanes 0-3, 8-11: the a / b partials
    s = dpp_add_half_mirror_banks<0xa>(s, c);        // lanes 4-7, 12-15: the c partials
    s = dpp_pair_add<0xb1>(s, s);  // quad_perm [1, 0, 3, 2]
    s = dpp_pair_add<0x4e>(s, s);  // quad_perm [2, 3, 0, 1]
    return s;
}

// Record accumulator slot k of batch record t, copy c ([t][c][kAccSlots] layout: the lanes that
// add at once hit different banks). Slots 0-7 hold g0..g7; slots 8-11 hold per-row partials of
// the last sums, which the batch readout adds: g8 from each of the four rows, or with the depth
// channel g8 from rows 0-1 and g9 from rows 2-3. Waves 0 and 1 add into copy 0, waves 2 and 3
// into copy 1, so a slot receives at most two adds into its zero: 0 + a + b rounds as 0 + b + a
// (float addition commutes), whatever order the waves arrive in, and the readout adds copy 0 and
// copy 1 in that order. Every sum is therefore the same from run to run.
constexpr int kAccSlots = 12;
constexpr int kAccCopies = 2;
constexpr int kAccStride = kAccSlots * kAccCopies;
#define ACC(t, k) acc[(t) * kAccStride + (k)]

// kDepth adds the depth channel of _rasterize_bwd_depth_kernel / _blend_depth_vjp
// (splax/_rasterize/_kernels.py:935-1080,1257-1302): the record's depth joins the colour dot
// product (v_alpha and the accumulator), and v_depth = v_out_depth * fac is a tenth sum.
template <bool kDepth>
__global__ void __launch_bounds__(kTile, 8) blend_bwd_kernel(BlendBwdParams P) {
    constexpr int NG = kDepth ? 10 : 9;
    __shared__ BatchLds<false, kBwdBatch> L;
    __shared__ float acc[kBwdBatch * kAccStride];
    __shared__ int32_t s_max;

    const BlendCommon& C = P.c;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int32_t tile_g = C.order[blockIdx.x];  // (output image, tile)
    // The order and the bins may come from the caller (a kept forward's). An order entry out of
    // range skips the workgroup, and a bin range outside [0, M] is clamped to it, so nothing is
    // read out of bounds; either sets kDevErrKeptLists in the device error word, because the
    // gradients of that call are then not the forward's (uniform, before any barrier).
    if ((uint32_t)tile_g >= gridDim.x) {
        if (threadIdx.x == 0) atomicOr(P.dev_err, kDevErrKeptLists);
        return;
    }
    const int32_t image_id = tile_g / C.num_tiles;
    const int32_t tile_local = tile_g - image_id * C.num_tiles;
    const int32_t geom_image = P.sel_geom ? image_id : 0;
    const int tile_x = tile_local % C.tiles_x, tile_y = tile_local / C.tiles_x;
    const int32_t gtile = geom_image * C.num_tiles + tile_local;
    int32_t range_start = C.bins[2 * gtile], range_end = C.bins[2 * gtile + 1];
    if (range_start < 0 || (int64_t)range_end > P.M) {
        if (threadIdx.x == 0) atomicOr(P.dev_err, kDevErrKeptLists);
        range_start = imaxw(range_start, 0);
        range_end = (int32_t)((int64_t)range_end > P.M ? P.M : (int64_t)range_end);
    }
    if (range_end <= range_start) return;  // uniform per workgroup
    int i, j;
    tile_pixel(tid, tile_x, tile_y, i, j);
    const float px = (float)j + 0.5f, py = (float)i + 0.5f;
    const bool inside = i < C.img_h && j < C.img_w;
    int32_t bin_final = range_start - 1;
    float T = 1.0f, v0 = 0.f, v1 = 0.f, v2 = 0.f, tfbg = 0.f, vd = 0.f;
    if (inside) {
        const int64_t frow = (int64_t)geom_image * C.img_h + i;
        bin_final = P.final_idx[frow * C.img_w + j];
        const float t_final = P.final_Ts[frow * C.img_w + j];
        T = t_final;
        // The cotangents enter halved (exact), so every product below that is linear in them
        // (v_alpha, v_sigma and all sums but the conic's a and c terms) is half the reference's;
        // the batch readout doubles those sums, exactly again. The conic's a and c terms,
        // 0.5 v_sigma dx dx and 0.5 v_sigma dy dy, need no 0.5 factor of their own then.
        if (P.loss_kind != kLossNone) {
            // v = 2 (img - target) * (g / count) (MSE) or sign(img - target) * (g / count) (L1),
            // the same float operations as loss_bwd_kernel, then halved as below
            const int64_t pix = ((int64_t)image_id * C.img_h + i) * C.img_w + j;
            const float scale = *P.v_loss / (float)P.loss_count;
            float v[3];
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                const float d = P.loss_img[3 * pix + k] - P.loss_target[3 * pix + k];
                const float sg = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : d);
                v[k] = P.loss_kind == kLossMse ? (d + d) * scale : sg * scale;
            }
            v0 = 0.5f * v[0]; v1 = 0.5f * v[1]; v2 = 0.5f * v[2];
        } else {
            const int64_t vrow = ((int64_t)image_id * C.img_h + i) % P.vout_rows;
            const float* vo = P.v_out + 3 * (vrow * C.img_w + j);
            v0 = 0.5f * vo[0]; v1 = 0.5f * vo[1]; v2 = 0.5f * vo[2];
        }
        const float* bg = C.background + 3 * (C.rows_bg > 1 ? image_id : 0);
        tfbg = t_final * ((bg[0] * v0 + bg[1] * v1) + bg[2] * v2);
        if constexpr (kDepth)
            vd = 0.5f * P.v_out_depth[(((int64_t)image_id * C.img_h + i) % P.vdepth_rows) *
                                          C.img_w + j];
    }
    // T_final (bg . v) plus sum_k buffer_k * v_k of the reference's colour accumulator, as one
    // running sum
    float acc_v = tfbg;
    if (tid == 0) s_max = range_start - 1;
    for (int k = tid; k < kBwdBatch * kAccStride; k += kTile) acc[k] = 0.0f;
    __syncthreads();
    atomicMax(&s_max, bin_final);
    // wave-wide largest final index: a record above it has no contributing lane in this wave
    // (a DPP maximum into lane 63 with the sign bit flipped, so the unsigned order is the signed
    // one; every lane is active here)
    const uint32_t wm = wave_minmax_to_lane63<true>((uint32_t)bin_final ^ 0x80000000u);
    const int32_t wmax =
        (int32_t)((uint32_t)__builtin_amdgcn_readlane((int)wm, 63) ^ 0x80000000u);
    __syncthreads();
    // a final_idx from the matching forward lies inside the tile's range; clamp anything else
    const int32_t start_idx = iminw(s_max, range_end - 1);
    const int32_t num_batches = (start_idx - range_start + kBwdBatch) / kBwdBatch;
    const int64_t rg_off = P.sel_geom ? 0 : (int64_t)image_id * P.M;
    {
        // intersections above every final index of the tile contribute nothing
        float zeros[NG];
#pragma unroll
        for (int k = 0; k < NG; ++k) zeros[k] = 0.0f;
        for (int32_t jj = start_idx + 1 + tid; jj < range_end; jj += kTile) {
            const int32_t e = P.pos[jj];
            if (e >= 0 && e < P.M) store_rgrad<NG>(P.rgrad, rg_off + e, zeros);
        }
    }

    const int row = lane >> 4, l16 = lane & 15;
    // After the wave reduction below, lane 0 of row r holds the sum of g[ka], lane 8 that of
    // g[4 + ka] and lane 4 the row's partial for slot 8 + r; they alone add into LDS.
    const int ka = (row == 0) ? 0 : (row == 1) ? 2 : (row == 2) ? 1 : 3;
    const bool adds = l16 == 0 || l16 == 4 || l16 == 8;
    const int kslot = (l16 == 0 ? ka : l16 == 8 ? 4 + ka : 8 + row) + kAccSlots * (wave >> 1);
    // The sorted id and emission position of each batch slot are loaded one batch ahead, so a
    // batch's staging waits on its records only, not on the ids that name them (the backward
    // 0.431 -> 0.425 ms at config 2, 2.084 -> 2.064 at config 4; the same in the forward blend
    // measured slower, 0.846 -> 0.858 ms at config 4).
    int32_t next_id = 0, next_pos = -1;
    if (num_batches > 0 && tid < kBwdBatch) {
        const int32_t src0 = imaxw(start_idx - tid, range_start);
        next_id = C.ids[src0];
        next_pos = start_idx - tid >= range_start ? P.pos[src0] : -1;
    }
    for (int32_t bt = 0; bt < num_batches; ++bt) {
        const int32_t batch_end = start_idx - bt * kBwdBatch;
        const bool live = tid < kBwdBatch && batch_end - tid >= range_start;
        const int32_t id = next_id;
        const int32_t my_pos = live ? next_pos : -1;  // emission position of slot tid
        if (bt + 1 < num_batches && tid < kBwdBatch) {
            const int32_t nsrc = imaxw(batch_end - kBwdBatch - tid, range_start);
            next_id = C.ids[nsrc];
            next_pos = batch_end - kBwdBatch - tid >= range_start ? P.pos[nsrc] : -1;
        }
        const int len = uniform(stage_batch<false, kBwdBatch>(C, L, id, live, tile_x, tile_y));
        // the wave's list in one register: lane l holds entries 4l .. 4l + 3
        const uint32_t list4 = reinterpret_cast<const uint32_t*>(L.list[uniform(wave)])[lane];
        uint32_t word = 0;
        for (int k = 0; k < len; ++k) {
            if ((k & 3) == 0) word = __builtin_amdgcn_readlane(list4, k >> 2);
            const int t = (int)((word >> (8 * (k & 3))) & 255u);
            const int32_t idx = batch_end - t;
            if (idx > wmax) continue;  // wave-uniform
            const float4 r0 = L.r0[t], r1 = L.r1[t], r2 = L.r2[t];
            // the whole record in the first reads (full-width reads, one address)
            asm volatile("" ::"v"(r1.y), "v"(r2.x), "v"(r2.y), "v"(r2.z), "v"(r2.w));
            const float dx = r0.x - px, dy = r0.y - py;
            const float sigma = blend_sigma(r0, r1, dx, dy);
            // bitwise: no short-circuit branch around the sigma_max read
            const bool in_range = (idx <= bin_final) & sigma_in_range(sigma, r1.z);
            if (__builtin_amdgcn_ballot_w64(in_range) == 0ull) continue;
            // Every lane computes and the lanes outside the accepted set are masked by selects
            // (an exec-masked instruction costs the same issue slot), so the wave reduction
            // below always sees exact zeros there and no branch is needed.
            const float vis = blend_exp(-sigma);
            const float ov = r1.y * vis;
            const float alpha_c = fminf(kAlphaMax, ov);  // as in the forward
            const bool valid = in_range && alpha_c >= kAlphaThresh;
            // a lane outside the accepted set blends alpha = 0 (a select, so whatever vis is):
            // T / (1 - 0) = T and its weight alpha T is zero, so T and the running sum need no
            // select of their own
            const float alpha = valid ? alpha_c : 0.0f;
            const float d = 1.0f - alpha;
            float ra = __builtin_amdgcn_rcpf(d);
            ra = fmaf(ra, fmaf(-d, ra, 1.0f), ra);
            T = T * ra;
            const float fac = alpha * T;
            float cv = fmaf(r2.x, v0, fmaf(r2.y, v1, r2.z * v2));
            if constexpr (kDepth) cv = fmaf(r2.w, vd, cv);  // depth as a fourth channel
            const float v_alpha = fmaf(T, cv, -ra * acc_v);  // halved
            acc_v = fmaf(cv, fac, acc_v);
            const bool geo = valid && ov <= kAlphaMax;
            // selects, not products with a masked zero: outside the accepted set vis and ov may be
            // inf or NaN (blend_exp is defined for sigma <= kBlendSigmaCap only)
            const float vs = geo ? -ov * v_alpha : 0.0f;  // v_sigma, halved
            const float hx = vs * dx, hy = vs * dy;
            const float g0 = v0 * fac, g1 = v1 * fac, g2 = v2 * fac;
            const float g3 = hx * dx, g4 = hx * dy, g5 = hy * dy;  // g3, g5 whole
            const float g6 = hx, g7 = hy;
            // the opacity term vis v_alpha is -v_sigma / o with the record's o, so the sum of
            // v_sigma is carried and the readout divides by -o once per record
            const float g8 = vs;
            const float g9 = kDepth ? vd * fac : 0.0f;
            // reduce-scatter over the wave: after the swaps, row r of qa holds g0/g2/g1/g3 and
            // of qb g4/g6/g5/g7 (rows 0..3); qc is g8 unswapped (each row reduces its own lanes)
            // or with depth the one swap of g8 with g9 (rows 0-1 then carry g8, rows 2-3 g9).
            // The row reduce-scatter leaves each sum in one adding lane.
            const float p01 = swap32_add(g0, g1), p23 = swap32_add(g2, g3);
            const float p45 = swap32_add(g4, g5), p67 = swap32_add(g6, g7);
            const float qa = swap16_add(p01, p23), qb = swap16_add(p45, p67);
            const float qc = kDepth ? swap32_add(g8, g9) : g8;
            const float sum = row_reduce_scatter3(qa, qb, qc);
            // An empty use keeps the last DPP add in this block: sunk into the branch below it
            // would no longer fuse with its DPP move.
            asm volatile("" ::"v"(sum));
            if (adds) atomicAdd(&acc[t * kAccStride + kslot], sum);
        }
        __syncthreads();
        if (tid < kBwdBatch) {
            float s[NG], part[4];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                // the halved sums doubled (the conic's a and c terms, slots 3 and 5, are whole)
                const float v = ACC(tid, k) + ACC(tid, kAccSlots + k);
                s[k] = (k == 3 || k == 5) ? v : 2.0f * v;
                ACC(tid, k) = 0.0f;
                ACC(tid, kAccSlots + k) = 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                part[r] = ACC(tid, 8 + r) + ACC(tid, kAccSlots + 8 + r);
                ACC(tid, 8 + r) = 0.0f;
                ACC(tid, kAccSlots + 8 + r) = 0.0f;
            }
            // v_opacity = sum vis v_alpha = -(sum v_sigma) / o (o >= 1/255 for every accepted
            // pair; a record with none sums to zero, which stays zero)
            float vsig;
            if constexpr (kDepth) {
                vsig = 2.0f * (part[0] + part[1]);
                s[9] = 2.0f * (part[2] + part[3]);
            } else {
                vsig = 2.0f * ((part[0] + part[1]) + (part[2] + part[3]));
            }
            s[8] = vsig != 0.0f ? -vsig / L.r1[tid].y : 0.0f;
            if (my_pos >= 0 && my_pos < P.M) store_rgrad<NG>(P.rgrad, rg_off + my_pos, s);
        }
        __syncthreads();
    }
}

#undef ACC

// Per output item: sum of its intersections' partial gradients in emission order (fixed, so
// deterministic; the conic and xy sums in double, the others in float), then
// v_xy = (a Sx + b Sy, b Sx + c Sy) with the item's conic (a, b, c), in double, which equals the
// reference's per-pair sum of
// v_sigma (a dx + b dy, b dx + c dy) (splax/_rasterize/_kernels.py:1246-1250) up to rounding; each
// output is rounded to float once. Every output is written. The double sums keep the gather's
// rounding out of the gradients of needle-thin items, whose projection VJP multiplies it by up
// to cond(conic)^2.
struct GatherParams {
    const int32_t* cum; const float* conics; const float* rgrad;
    int64_t M; int64_t nout; int32_t n; int32_t sel_geom;
    float* v_colors; float* v_opacity; float* v_xy; float* v_conic;
    float* v_depths;  // NG == 10
    const float* opac; int64_t rows_opac; int32_t compensate;
    int32_t fold;  // v_colors / v_opacity summed over the images into n rows
};

// With P.fold one thread per gaussian walks the images in order: per-item v_xy / v_conic /
// v_depths rows as always, the colour and opacity cotangents summed into the gaussian's row.
// The workgroup's items of one pass (one image with P.fold) read their rows cooperatively
// (block_gather) when they lie in one contiguous range of rgrad: always with per-item geometry,
// and with shared geometry when the workgroup's items belong to one output image.
template <int NG>
__global__ void __launch_bounds__(256) grad_gather_kernel(GatherParams P) {
    __shared__ float s_buf[kGatherChunk * NG];
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t limit = P.fold ? (int64_t)P.n : P.nout;
    const int64_t t_first = (int64_t)blockIdx.x * 256;
    const int64_t t_last = (t_first + 255 < limit ? t_first + 255 : limit - 1);
    const bool valid = t < limit;
    const int32_t images = P.fold ? (int32_t)(P.nout / P.n) : 1;
    double fc0 = 0.0, fc1 = 0.0, fc2 = 0.0, fo = 0.0;
    for (int32_t image = 0; image < images; ++image) {
    const int64_t og = P.fold ? (int64_t)image * P.n + t : t;
    int64_t gi = og, off = 0;
    if (!P.sel_geom) {
        const int64_t b = og / P.n;
        gi = og - b * P.n;
        off = b * P.M;
    }
    int64_t lo = 0, hi = 0;
    // the item's conic (and with compensation its opacity) load with its range, ahead of the
    // row sums rather than behind them
    float ca = 0.f, cb = 0.f, cc = 0.f, op = 0.f;
    if (valid) {
        ca = P.conics[3 * gi];
        cb = P.conics[3 * gi + 1];
        cc = P.conics[3 * gi + 2];
        if (P.compensate) op = P.opac[gi % P.rows_opac];
        lo = gi > 0 ? (int64_t)P.cum[gi - 1] : 0;
        hi = P.cum[gi];
        lo = lo < 0 ? 0 : lo;
        hi = hi > P.M ? P.M : hi;
        hi = hi < lo ? lo : hi;
    }
    // the workgroup's range (uniform)
    const int64_t og_first = P.fold ? (int64_t)image * P.n + t_first : t_first;
    const int64_t og_last = P.fold ? (int64_t)image * P.n + t_last : t_last;
    const bool one_range = P.sel_geom || og_first / P.n == og_last / P.n;
    double s[NG];
    if (one_range) {
        int64_t gf = og_first, gl = og_last, woff = 0;
        if (!P.sel_geom) {
            const int64_t b = og_first / P.n;
            gf -= b * P.n;
            gl -= b * P.n;
            woff = b * P.M;
        }
        int64_t wlo = gf > 0 ? (int64_t)P.cum[gf - 1] : 0, whi = P.cum[gl];
        wlo = wlo < 0 ? 0 : wlo;
        whi = whi > P.M ? P.M : whi;
        block_gather<NG, 256>(P.rgrad, woff, wlo, whi, lo, hi, s_buf, s);
    } else {
        GatherSums<NG> acc;
        acc.clear();
        for (int64_t e = lo; e < hi; ++e) acc.add_row(P.rgrad + (off + e) * NG);
        acc.out(s);
    }
    if (!valid) continue;
    float vc[3] = {(float)s[3], (float)s[4], (float)s[5]};
    float vo = (float)s[8];
    float vx = 0.f, vy = 0.f;
    if (s[6] != 0.0 || s[7] != 0.0 || P.compensate) {
        vx = (float)((double)ca * s[6] + (double)cb * s[7]);
        vy = (float)((double)cb * s[6] + (double)cc * s[7]);
        if (P.compensate) vo = compensation_vjp(vo, op, ca, cb, cc, vc);
    }
    P.v_conic[3 * og] = vc[0];
    P.v_conic[3 * og + 1] = vc[1];
    P.v_conic[3 * og + 2] = vc[2];
    P.v_xy[2 * og] = vx;
    P.v_xy[2 * og + 1] = vy;
    if constexpr (NG == 10) P.v_depths[og] = (float)s[9];
    if (P.fold) {
        fc0 = fc0 + s[0];
        fc1 = fc1 + s[1];
        fc2 = fc2 + s[2];
        fo = fo + (double)vo;
    } else {
        P.v_colors[3 * og] = (float)s[0];
        P.v_colors[3 * og + 1] = (float)s[1];
        P.v_colors[3 * og + 2] = (float)s[2];
        P.v_opacity[og] = vo;
    }
    }
    if (P.fold && valid) {
        P.v_colors[3 * t] = (float)fc0;
        P.v_colors[3 * t + 1] = (float)fc1;
        P.v_colors[3 * t + 2] = (float)fc2;
        P.v_opacity[t] = (float)fo;
    }
}

int launch_blend_bwd(const RasterInputs& in, const KeyLayout& lay, const int32_t* sorted_ids,
                     const int32_t* tile_bins, const BlendBwdArgs& a, int32_t* order,
                     const int32_t* kept_order, hipStream_t stream) {
    const int64_t nout = (int64_t)a.B_out * in.n;
    const int32_t sel_geom = in.B_geom > 1;
    const int64_t blocks = (int64_t)a.B_out * lay.num_tiles;
    const bool depth = a.v_depths != nullptr;
    if (blocks > 0 && sorted_ids != nullptr && a.M > 0) {
        // the forward's order covers its B_geom images; shared geometry with B_out > 1 orders
        // each output image by image 0's bins here
        const bool reuse = kept_order != nullptr && a.B_out == in.B_geom;
        if (!reuse) {
            const int rc =
                launch_tile_order(tile_bins, blocks, lay.num_tiles, sel_geom, order, stream);
            if (rc) return rc;
        }
        BlendBwdParams P;
        fill_common(P.c, in, lay, sorted_ids, tile_bins);
        P.c.recs = a.recs;
        P.c.order = reuse ? kept_order : order;
        P.final_Ts = a.final_Ts; P.final_idx = a.final_idx;
        P.v_out = a.v_out; P.vout_rows = a.vout_rows;
        P.n = in.n; P.sel_geom = sel_geom;
        P.pos = a.sorted_pos; P.M = a.M;
        P.v_out_depth = a.v_out_depth; P.vdepth_rows = a.vdepth_rows;
        P.rgrad = a.rgrad;
        P.dev_err = a.dev_err;
        P.loss_kind = a.loss.kind; P.loss_target = a.loss.target; P.loss_img = a.loss.img;
        P.v_loss = a.loss.v_loss; P.loss_count = a.loss.count;
        hipEvent_t ka, kb;  // null unless this kernel is timed
        (void)kernel_timer_events(kKernelBlendBwd, &ka, &kb);
        if (depth)
            hipExtLaunchKernelGGL(blend_bwd_kernel<true>, dim3((unsigned)blocks), dim3(kTile),
                                  0, stream, ka, kb, 0, P);
        else
            hipExtLaunchKernelGGL(blend_bwd_kernel<false>, dim3((unsigned)blocks), dim3(kTile),
                                  0, stream, ka, kb, 0, P);
        if (hipGetLastError() != hipSuccess) return kErrLaunch;
    }
    if (nout <= 0) return 0;
    GatherParams G;
    G.cum = in.cum; G.conics = in.conics; G.rgrad = a.rgrad;
    G.M = (sorted_ids != nullptr) ? a.M : 0;
    G.nout = nout; G.n = in.n; G.sel_geom = sel_geom;
    G.v_colors = a.v_colors; G.v_opacity = a.v_opacity; G.v_xy = a.v_xy; G.v_conic = a.v_conic;
    G.v_depths = a.v_depths;
    G.opac = in.opac; G.rows_opac = in.rows_opac; G.compensate = in.compensate;
    G.fold = a.fold;
    const int64_t threads = a.fold ? (int64_t)in.n : nout;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (depth)
        hipLaunchKernelGGL(grad_gather_kernel<10>, grid, dim3(256), 0, stream, G);
    else
        hipLaunchKernelGGL(grad_gather_kernel<9>, grid, dim3(256), 0, stream, G);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

}  // namespace splat
