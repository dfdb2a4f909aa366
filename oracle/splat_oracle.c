/* CPU oracle for the gaussian-splat render path — TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, one function per reference kernel, the algorithm of amacati/splax's render
 * path (projection, opacity-aware tile intersection, key emission, stable sort, bin edges, forward
 * blend, blend VJP, projection VJP). It is the checker for the GPU library and the timed CPU
 * baseline; nothing in the product links it. It shares no source with the HIP kernels.
 *
 * Arithmetic contract (shared by this oracle and the GPU kernels, so their outputs can be compared
 * bit for bit):
 *   - IEEE binary32 with round-to-nearest-even, no FMA contraction (-ffp-contract=off); an FMA is
 *     used only where written explicitly as fmaf().
 *   - Division and sqrt are correctly rounded.
 *   - exp and log are the fixed-sequence routines oracle_expf / oracle_logf below (Cody-Waite
 *     range reduction plus a Taylor / atanh series), not a libm call, because libm and the GPU's
 *     device library round differently in the last place. The blends' exp(-sigma) is its own
 *     shorter sequence, oracle_blend_expf (magic-constant rounding, a degree-6 polynomial and an
 *     exponent-field scale), and their sigma and colour sums are written with fmaf.
 *   - min(a, b) = a < b ? a : b and max(a, b) = a > b ? a : b (scalar min/max semantics of the
 *     reference's Warp kernels); float -> int32 truncates toward zero and saturates, NaN -> 0.
 *   - 3x3 products associate as (a0*b0 + a1*b1) + a2*b2.
 * The reference itself compiles with Warp fast_math (splax/_intersect.py:15), so its exact float
 * bits are not reproducible without Warp; the contract fixes one well-defined rounding instead.
 *
 * Parity pinning (tests/test_oracle_*.py): log/exp against numpy float64 within a few ulp;
 * projection against closed forms and a float64 torch restatement in matrix form; the tile walk
 * against brute-force pixel coverage; scan / sort / bins against numpy closed forms; the blend
 * against a float64 brute-force renderer; both VJPs against torch autograd and finite
 * differences.
 */
#include "splat_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* splax/_intersect.py:17-20 */
#define BLOCK_WIDTH 16
#define BLOCK_SIZE 256
static const float GAUSSIAN_EXTEND_SQ = 0x1.62d844p+3f; /* float32(3.33 * 3.33) */
static const float ALPHA_THRESHOLD = 0x1.010102p-8f;    /* float32(1 / 255) */
static const float ALPHA_MAX = 0x1.ff7ceep-1f;          /* float32(0.999) */
static const float T_EPS = 0x1.a36e2ep-14f;             /* float32(1e-4) */
/* Largest sigma the blends accept: oracle_blend_expf(-87) is still a normal float. A larger sigma
 * is rejected, as the exact alpha would be for opacities below 2.4e35 (the GPU caps its packed
 * sigma_max at the same value). */
static const float BLEND_SIGMA_CAP = 87.0f;
static const float DILATION = 0x1.333334p-2f;           /* float32(0.3) */
static const float FOV_CLAMP = 0x1.4ccccdp+0f;          /* float32(1.3) */
static const float Z_EPS = 0x1.0c6f7ap-20f;             /* float32(1e-6) */

/* ---------------------------------------------------------------- scalar helpers */

static inline float fminw(float a, float b) { return a < b ? a : b; }
static inline float fmaxw(float a, float b) { return a > b ? a : b; }
static inline int32_t iminw(int32_t a, int32_t b) { return a < b ? a : b; }
static inline int32_t imaxw(int32_t a, int32_t b) { return a > b ? a : b; }

static inline int32_t f2i(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static const float LN2_HI = 0x1.62ep-1f;      /* ln2 with the low 12 mantissa bits cleared */
static const float LN2_LO = 0x1.0bfbe8p-15f;  /* float32(ln2 - LN2_HI) */
static const float LOG2E = 0x1.715476p+0f;

/* Natural log for finite x > 0. x = 2^k m with m in (sqrt(2)/2, sqrt(2)], f = m - 1 (exact),
 * s = f / (2 + f), log(m) = 2 atanh(s) = 2s + 2s z (1/3 + z/5 + z^2/7 + z^3/9), z = s^2 (|s| <=
 * 0.1716, truncation < 1e-9), log(x) = k ln2_hi + (k ln2_lo + log(m)). */
float oracle_logf(float x) {
    int32_t k = 0;
    uint32_t ix = f2u(x);
    if (ix < 0x00800000u) { /* subnormal: scale into the normal range */
        x = x * 0x1p25f;
        k = -25;
        ix = f2u(x);
    }
    k += (int32_t)(ix >> 23) - 127;
    float m = u2f((ix & 0x007fffffu) | 0x3f800000u);
    if (m > 0x1.6a09e6p+0f) {
        m = m * 0.5f;
        k += 1;
    }
    float f = m - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    float p = fmaf(z, 0x1.c71c72p-4f, 0x1.24924ap-3f); /* 1/9, 1/7 */
    p = fmaf(z, p, 0x1.99999ap-3f);                    /* 1/5 */
    p = fmaf(z, p, 0x1.555556p-2f);                    /* 1/3 */
    float hs = s + s;
    float lm = fmaf(hs * z, p, hs);
    float kf = (float)k;
    return fmaf(kf, LN2_HI, fmaf(kf, LN2_LO, lm));
}

/* e^x. k = rint(x log2 e), r = x - k ln2 (two FMAs), e^r by its degree-7 Taylor polynomial on
 * |r| <= 0.347 (truncation < 1.3e-8 relative), scaled by 2^k. NaN and x <= -104 give 0. */
float oracle_expf(float x) {
    if (!(x > -104.0f)) return 0.0f;
    if (x > 88.75f) return INFINITY;
    float kf = rintf(x * LOG2E);
    float r = fmaf(kf, -LN2_HI, x);
    r = fmaf(kf, -LN2_LO, r);
    float p = fmaf(r, 0x1.a01a02p-13f, 0x1.6c16c2p-10f); /* 1/5040, 1/720 */
    p = fmaf(r, p, 0x1.111112p-7f);                      /* 1/120 */
    p = fmaf(r, p, 0x1.555556p-5f);                      /* 1/24 */
    p = fmaf(r, p, 0x1.555556p-3f);                      /* 1/6 */
    p = fmaf(r, p, 0.5f);
    p = fmaf(r, p, 1.0f);
    p = fmaf(r, p, 1.0f);
    return ldexpf(p, (int)kf);
}

/* The blends' Gaussian exponent 0.5 (a dx^2 + c dy^2) + b dx dy (splax/_rasterize/_kernels.py:187,
 * 1039), evaluated as dx (a/2 dx + b dy) + (c/2 dy) dy with two FMAs (the same value in exact
 * arithmetic; the halving of a and c is exact). */
static inline float blend_sigma(const float* cn, float dx, float dy) {
    const float ha = 0.5f * cn[0], hc = 0.5f * cn[2];
    return fmaf(dx, fmaf(ha, dx, cn[1] * dy), (hc * dy) * dy);
}

/* e^x for the blends' x = -sigma <= 0: k = round(x log2 e) by adding 1.5 * 2^23 (the integer then
 * sits in the low mantissa bits of the sum), r = x - k fl(ln2) in one FMA, e^r by a degree-6
 * polynomial with c0 = c1 = 1 fitted by Lawson's iteration (relative error 4.4e-9 on
 * |r| <= ln2 / 2 with these float coefficients), and 2^k added to the exponent field as an
 * integer: at most 1 ulp from e^x on [-8, 0], 2 ulp down to -30, 5 ulp down to -87
 * (tests/test_oracle_math.py). Below 2^-126 the result is not e^x but tiny,
 * negative or NaN, so an alpha built from it fails the 1/255 test as the exact one would for
 * opacities below 1e30. */
float oracle_blend_expf(float x) {
    const float t = fmaf(x, LOG2E, 0x1.8p23f);
    const float kf = t - 0x1.8p23f;
    const float r = fmaf(kf, -0x1.62e430p-1f, x);
    float p = fmaf(r, 0x1.6a2352p-10f, 0x1.123a6cp-7f);
    p = fmaf(r, p, 0x1.5558f4p-5f);
    p = fmaf(r, p, 0x1.55549p-3f);
    p = fmaf(r, p, 0x1.fffffcp-2f);
    p = fmaf(r, p, 1.0f);
    p = fmaf(r, p, 1.0f);
    uint32_t pb, tb;
    memcpy(&pb, &p, 4);
    memcpy(&tb, &t, 4);
    pb += tb << 23;
    float y;
    memcpy(&y, &pb, 4);
    return y;
}

/* ---------------------------------------------------------------- 3x3 helpers (row major) */

static inline void mat_mul(const float* a, const float* b, float* c) {
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            c[3 * i + j] = (a[3 * i] * b[j] + a[3 * i + 1] * b[3 + j]) + a[3 * i + 2] * b[6 + j];
}
static inline void mat_mul_tn(const float* a, const float* b, float* c) { /* a^T b */
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            c[3 * i + j] = (a[i] * b[j] + a[3 + i] * b[3 + j]) + a[6 + i] * b[6 + j];
}
static inline void mat_mul_nt(const float* a, const float* b, float* c) { /* a b^T */
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            c[3 * i + j] =
                (a[3 * i] * b[3 * j] + a[3 * i + 1] * b[3 * j + 1]) + a[3 * i + 2] * b[3 * j + 2];
}
static inline void mat_vec(const float* a, const float* v, float* o) {
    for (int i = 0; i < 3; ++i) o[i] = (a[3 * i] * v[0] + a[3 * i + 1] * v[1]) + a[3 * i + 2] * v[2];
}
static inline void mat_t_vec(const float* a, const float* v, float* o) {
    for (int i = 0; i < 3; ++i) o[i] = (a[i] * v[0] + a[3 + i] * v[1]) + a[6 + i] * v[2];
}

/* Rotation of quaternion q = (x, y, z, w): R = (2w^2 - 1) I + 2 v v^T + 2 w [v]_x with v = (x, y,
 * z), i.e. the columns are q rotating the basis vectors. This is warp-lang 1.15.0's
 * quat_to_matrix (called at splax/_project/_kernels.py:426,661); for a unit quaternion it equals
 * the textbook matrix. */
static inline void quat_to_rot(const float* q, float* R) {
    float x = q[0], y = q[1], z = q[2], w = q[3];
    float x2 = x + x, y2 = y + y, z2 = z + z, w2 = w + w;
    float c = w2 * w - 1.0f;
    R[0] = c + x * x2;
    R[1] = x * y2 - z * w2;
    R[2] = x * z2 + y * w2;
    R[3] = y * x2 + z * w2;
    R[4] = c + y * y2;
    R[5] = y * z2 - x * w2;
    R[6] = z * x2 - y * w2;
    R[7] = z * y2 + x * w2;
    R[8] = c + z * z2;
}

/* _load_affine, splax/_project/_kernels.py:609-624: rows r0..r0+2 of a row-major (rows, 4) array */
static inline void load_affine(const float* m, float* R, float* t) {
    for (int i = 0; i < 3; ++i) {
        R[3 * i] = m[4 * i];
        R[3 * i + 1] = m[4 * i + 1];
        R[3 * i + 2] = m[4 * i + 2];
        t[i] = m[4 * i + 3];
    }
}

/* ---------------------------------------------------------------- ellipse walk
 * splax/_intersect.py:23-183 (SNUGBOX tight bbox + AccuTile column walk). */

typedef struct {
    float A, B, C, disc, t, px, py;
    float bbox_min[2], bbox_max[2], bbox_argmin[2], bbox_argmax[2];
    int32_t rect_min[2], rect_max[2];
    int valid, isY;
} Ellipse;

/* ellipse_init, splax/_intersect.py:46-107 */
static void ellipse_init(float A, float B, float C, float t, float px, float py, int32_t tw,
                         int32_t th, Ellipse* s) {
    memset(s, 0, sizeof(*s));
    s->A = A;
    s->B = B;
    s->C = C;
    s->t = t;
    s->px = px;
    s->py = py;
    float disc = B * B - A * C;
    s->disc = disc;
    float ntd = -t / disc;
    float x_extent = sqrtf(ntd * C);
    float y_extent = sqrtf(ntd * A);
    float bmin0 = px - x_extent, bmin1 = py - y_extent;
    float bmax0 = px + x_extent, bmax1 = py + y_extent;
    float bx_c = B * x_extent / C;
    float by_a = B * y_extent / A;
    float amin0 = py + bx_c, amin1 = px + by_a;
    float amax0 = py - bx_c, amax1 = px - by_a;
    const float ts = (float)BLOCK_WIDTH;
    int32_t rminx = imaxw(0, iminw(tw, f2i(bmin0 / ts)));
    int32_t rminy = imaxw(0, iminw(th, f2i(bmin1 / ts)));
    int32_t rmaxx = imaxw(0, iminw(tw, f2i(bmax0 / ts + 1.0f)));
    int32_t rmaxy = imaxw(0, iminw(th, f2i(bmax1 / ts + 1.0f)));
    int32_t x_span = rmaxx - rminx, y_span = rmaxy - rminy;
    if (y_span * x_span == 0) return;
    int isY = y_span < x_span;
    s->isY = isY;
    if (isY) {
        s->rect_min[0] = rminy; s->rect_min[1] = rminx;
        s->rect_max[0] = rmaxy; s->rect_max[1] = rmaxx;
        s->bbox_min[0] = bmin1; s->bbox_min[1] = bmin0;
        s->bbox_max[0] = bmax1; s->bbox_max[1] = bmax0;
        s->bbox_argmin[0] = amin1; s->bbox_argmin[1] = amin0;
        s->bbox_argmax[0] = amax1; s->bbox_argmax[1] = amax0;
    } else {
        s->rect_min[0] = rminx; s->rect_min[1] = rminy;
        s->rect_max[0] = rmaxx; s->rect_max[1] = rmaxy;
        s->bbox_min[0] = bmin0; s->bbox_min[1] = bmin1;
        s->bbox_max[0] = bmax0; s->bbox_max[1] = bmax1;
        s->bbox_argmin[0] = amin0; s->bbox_argmin[1] = amin1;
        s->bbox_argmax[0] = amax0; s->bbox_argmax[1] = amax1;
    }
    s->valid = 1;
}

/* _ellipse_intersect, splax/_intersect.py:110-133 */
static void ellipse_intersect(const Ellipse* s, float coord, float* out) {
    float p_u, p_v, coeff;
    if (s->isY) {
        p_u = s->py; p_v = s->px; coeff = s->A;
    } else {
        p_u = s->px; p_v = s->py; coeff = s->C;
    }
    float h = coord - p_u;
    float sq = sqrtf(s->disc * h * h + s->t * coeff);
    float bh = -s->B * h;
    out[0] = (bh - sq) / coeff + p_v;
    out[1] = (bh + sq) / coeff + p_v;
}

/* ellipse_init_span, splax/_intersect.py:136-143 */
static void ellipse_init_span(const Ellipse* s, float* I) {
    float min_line0 = (float)s->rect_min[0] * (float)BLOCK_WIDTH;
    if (s->bbox_min[0] <= min_line0) {
        ellipse_intersect(s, min_line0, I);
        return;
    }
    I[0] = s->bbox_max[1];
    I[1] = s->bbox_min[1];
}

/* ellipse_column_tile_range, splax/_intersect.py:146-169. Writes [min_v, max_v) and rolls I. */
static void ellipse_column(const Ellipse* s, int32_t u, float* I, int32_t* min_v, int32_t* max_v) {
    const float block = (float)BLOCK_WIDTH;
    float min_line = (float)u * block;
    float max_line = min_line + block;
    float Imax[2];
    if (max_line <= s->bbox_max[0]) {
        ellipse_intersect(s, max_line, Imax);
    } else {
        Imax[0] = I[0];
        Imax[1] = I[1];
    }
    float emin, emax;
    if (min_line <= s->bbox_argmin[1] && s->bbox_argmin[1] < max_line)
        emin = s->bbox_min[1];
    else
        emin = fminw(I[0], Imax[0]);
    if (min_line <= s->bbox_argmax[1] && s->bbox_argmax[1] < max_line)
        emax = s->bbox_max[1];
    else
        emax = fmaxw(I[1], Imax[1]);
    *min_v = imaxw(s->rect_min[1], iminw(s->rect_max[1], f2i(emin / block)));
    *max_v = iminw(s->rect_max[1], imaxw(s->rect_min[1], f2i(emax / block + 1.0f)));
    I[0] = Imax[0];
    I[1] = Imax[1];
}

/* ellipse_tile_count, splax/_intersect.py:172-183 */
static int32_t ellipse_tile_count(const Ellipse* s) {
    if (!s->valid) return 0;
    float I[2];
    ellipse_init_span(s, I);
    int32_t count = 0;
    for (int32_t u = s->rect_min[0]; u < s->rect_max[0]; ++u) {
        int32_t mn, mx;
        ellipse_column(s, u, I, &mn, &mx);
        count += mx - mn;
    }
    return count;
}

/* opacity-aware isocontour level t, splax/_project/_kernels.py:227 and
 * splax/_rasterize/_sort/_kernels.py:132-133 */
static inline float iso_level(float opac) {
    return fminw(GAUSSIAN_EXTEND_SQ, 2.0f * oracle_logf(opac / ALPHA_THRESHOLD));
}

int oracle_key_layout(int32_t B, int32_t img_h, int32_t img_w, int32_t* out) {
    int32_t tbx = (img_w + BLOCK_WIDTH - 1) / BLOCK_WIDTH;
    int32_t tby = (img_h + BLOCK_WIDTH - 1) / BLOCK_WIDTH;
    int32_t nt = tbx * tby;
    int32_t tile_bits = 0, image_bits = 0;
    while ((1LL << tile_bits) <= (int64_t)(nt - 1) && nt > 1) ++tile_bits; /* (nt-1).bit_length() */
    while ((1LL << image_bits) <= (int64_t)(B - 1) && B > 1) ++image_bits;
    out[0] = tbx;
    out[1] = tby;
    out[2] = nt;
    out[3] = tile_bits;
    out[4] = image_bits;
    out[5] = 31 - image_bits - tile_bits;
    return out[5] >= 16;
}

/* _use_32bit_keys, splax/_rasterize/_sort/_sort.py:23-26 (which the reference's tests patch to
 * force the 64-bit key): with the switch set, every layout takes the 64-bit key. */
static int g_force_wide = 0;
void oracle_set_wide_keys(int force) { g_force_wide = force != 0; }

/* 0: packed 32-bit key; 1: 64-bit key; -2: even the 64-bit key overflows (image + tile bits
 * above 32, splax/_rasterize/_sort/_sort.py:61-66). */
int oracle_key_mode(int32_t B, int32_t img_h, int32_t img_w) {
    int32_t L[6];
    int packed = oracle_key_layout(B, img_h, img_w, L);
    if (packed && !g_force_wide) return 0;
    if (L[3] + L[4] > 32) return -2;
    return 1;
}

/* ---------------------------------------------------------------- projection forward
 * _project_kernel, splax/_project/_kernels.py:122-248, with _apply_transform (:627-644) and
 * _project_geom (:647-664); the inclusive scan of splax/_project/_kernels.py:107. */

static void project_geom(const float* mean_in, const float* quat, const float* scale,
                         float glob_scale, const float* vm_rows, const float* R_tf, int moved,
                         float* W, float* p, float* M, float* mean_out) {
    float trans[3];
    load_affine(vm_rows, W, trans);
    float wm[3];
    mat_vec(W, mean_in, wm);
    for (int i = 0; i < 3; ++i) p[i] = wm[i] + trans[i];
    float R[9];
    quat_to_rot(quat, R);
    float s[3] = {glob_scale * scale[0], glob_scale * scale[1], glob_scale * scale[2]};
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) M[3 * i + j] = R[3 * i + j] * s[j];
    if (moved) {
        float Mm[9];
        mat_mul(R_tf, M, Mm);
        memcpy(M, Mm, sizeof(Mm));
    }
    if (mean_out) memcpy(mean_out, mean_in, 3 * sizeof(float));
}

static int apply_transform(const float* transforms, int32_t image_id, int32_t num_transforms,
                           int sel_transforms, int32_t tf_id, float* mean, float* R_tf) {
    static const float I3[9] = {1, 0, 0, 0, 1, 0, 0, 0, 1};
    memcpy(R_tf, I3, sizeof(I3));
    /* ids outside [0, num_transforms) are treated as static, as in the GPU library */
    if (tf_id < 0 || tf_id >= num_transforms) return 0;
    int64_t tf_idx = sel_transforms ? (int64_t)image_id * num_transforms + tf_id : tf_id;
    float t[3], rm[3];
    load_affine(transforms + tf_idx * 16, R_tf, t);
    mat_vec(R_tf, mean, rm);
    for (int i = 0; i < 3; ++i) mean[i] = rm[i] + t[i];
    return 1;
}

int oracle_project_fwd(const float* means3d, int64_t rows_means, const float* scales,
                       int64_t rows_scales, const float* quats, int64_t rows_quats,
                       const float* viewmat, int64_t rows_viewmat, const float* opacities,
                       int64_t rows_opac, const float* transforms, int64_t rows_transforms,
                       const int32_t* transform_ids, int32_t n, int32_t num_transforms,
                       int32_t has_transforms, int64_t total, int32_t img_h, int32_t img_w,
                       float fx, float fy, float cx, float cy, float glob_scale,
                       float clip_thresh, float* xys, float* depths, int32_t* radii,
                       float* conics, int32_t* num_tiles_hit, int32_t* cum_tiles_hit) {
    const int sel_means = rows_means > n, sel_scales = rows_scales > n, sel_quats = rows_quats > n;
    const int sel_view = rows_viewmat > 4, sel_opac = rows_opac > n;
    const int sel_tf = rows_transforms > num_transforms;
    const int32_t tb_x = (img_w + BLOCK_WIDTH - 1) / BLOCK_WIDTH;
    const int32_t tb_y = (img_h + BLOCK_WIDTH - 1) / BLOCK_WIDTH;
    const float tan_fovx = 0.5f * (float)img_w / fx;
    const float tan_fovy = 0.5f * (float)img_h / fy;
    const float lim_x = FOV_CLAMP * tan_fovx;
    const float lim_y = FOV_CLAMP * tan_fovy;
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int32_t bid = (int32_t)(idx / n), gid = (int32_t)(idx % n);
        int64_t m_idx = sel_means ? idx : gid, s_idx = sel_scales ? idx : gid;
        int64_t q_idx = sel_quats ? idx : gid, o_idx = sel_opac ? idx : gid;
        int64_t vb = (int64_t)(sel_view ? bid : 0) * 4;
        xys[2 * idx] = 0.0f;
        xys[2 * idx + 1] = 0.0f;
        depths[idx] = 0.0f;
        radii[idx] = 0;
        conics[3 * idx] = conics[3 * idx + 1] = conics[3 * idx + 2] = 0.0f;
        num_tiles_hit[idx] = 0;

        float mean[3] = {means3d[3 * m_idx], means3d[3 * m_idx + 1], means3d[3 * m_idx + 2]};
        int32_t tf_id = has_transforms ? transform_ids[gid] : -1;
        float R_tf[9];
        int moved = apply_transform(transforms, bid, num_transforms, sel_tf, tf_id, mean, R_tf);
        float W[9], p[3], M[9];
        project_geom(mean, quats + 4 * q_idx, scales + 3 * s_idx, glob_scale, viewmat + vb * 4,
                     R_tf, moved, W, p, M, NULL);
        if (p[2] <= clip_thresh) continue;
        float V[9];
        mat_mul_nt(M, M, V);

        float tz = p[2];
        float tx = tz * fminw(lim_x, fmaxw(-lim_x, p[0] / tz));
        float ty = tz * fminw(lim_y, fmaxw(-lim_y, p[1] / tz));
        float rz = 1.0f / tz;
        float rz2 = rz * rz;
        float j00 = fx * rz, j02 = -fx * tx * rz2, j11 = fy * rz, j12 = -fy * ty * rz2;
        float T0[3], T1[3];
        for (int j = 0; j < 3; ++j) {
            T0[j] = j00 * W[j] + j02 * W[6 + j];
            T1[j] = j11 * W[3 + j] + j12 * W[6 + j];
        }
        float TV0[3], TV1[3];
        for (int k = 0; k < 3; ++k) {
            TV0[k] = (T0[0] * V[k] + T0[1] * V[3 + k]) + T0[2] * V[6 + k];
            TV1[k] = (T1[0] * V[k] + T1[1] * V[3 + k]) + T1[2] * V[6 + k];
        }
        float c00 = (TV0[0] * T0[0] + TV0[1] * T0[1]) + TV0[2] * T0[2];
        float c01 = (TV0[0] * T1[0] + TV0[1] * T1[1]) + TV0[2] * T1[2];
        float c11 = (TV1[0] * T1[0] + TV1[1] * T1[1]) + TV1[2] * T1[2];
        float cxx = c00 + DILATION, cxy = c01, cyy = c11 + DILATION;
        float det = cxx * cyy - cxy * cxy;
        if (det == 0.0f) continue;
        float inv_det = 1.0f / det;
        float con0 = cyy * inv_det, con1 = -cxy * inv_det, con2 = cxx * inv_det;

        float rw = 1.0f / (p[2] + Z_EPS);
        float center_x = (p[0] * rw) * fx + cx;
        float center_y = (p[1] * rw) * fy + cy;

        float opac = opacities[o_idx];
        if (opac < ALPHA_THRESHOLD) continue;
        float t = iso_level(opac);
        float ext = sqrtf(t);
        float radius_x = ceilf(ext * sqrtf(cxx));
        float radius_y = ceilf(ext * sqrtf(cyy));
        if (radius_x <= 0.0f && radius_y <= 0.0f) continue;
        if (center_x + radius_x <= 0.0f || center_x - radius_x >= (float)img_w ||
            center_y + radius_y <= 0.0f || center_y - radius_y >= (float)img_h)
            continue;
        Ellipse e;
        ellipse_init(con0, con1, con2, t, center_x, center_y, tb_x, tb_y, &e);
        int32_t count = ellipse_tile_count(&e);
        if (count <= 0) continue;
        num_tiles_hit[idx] = count;
        depths[idx] = p[2];
        radii[idx] = f2i(fmaxw(radius_x, radius_y));
        xys[2 * idx] = center_x;
        xys[2 * idx + 1] = center_y;
        conics[3 * idx] = con0;
        conics[3 * idx + 1] = con1;
        conics[3 * idx + 2] = con2;
    }
    int32_t acc = 0;
    for (int64_t i = 0; i < total; ++i) {
        acc += num_tiles_hit[i];
        cum_tiles_hit[i] = acc;
    }
    return 0;
}

/* ---------------------------------------------------------------- keys, sort, bins */

/* _seed_minmax + _depth_minmax, splax/_rasterize/_sort/_kernels.py:31-73: per-image [dmin, dmax]
 * over visible items (radii > 0), sentinels +-1e30. */
static void depth_minmax(const float* depths, const int32_t* radii, int64_t total, int32_t n,
                         int32_t B, float* mm) {
    for (int32_t b = 0; b < B; ++b) {
        mm[2 * b] = 1.0e30f;
        mm[2 * b + 1] = -1.0e30f;
    }
    for (int64_t idx = 0; idx < total; ++idx) {
        if (radii[idx] <= 0) continue;
        int32_t im = (int32_t)(idx / n);
        mm[2 * im] = fminw(mm[2 * im], depths[idx]);
        mm[2 * im + 1] = fmaxw(mm[2 * im + 1], depths[idx]);
    }
}

/* _map_intersects_32bit, splax/_rasterize/_sort/_kernels.py:76-153 */
int64_t oracle_emit_keys(const float* xys, const float* depths, const int32_t* radii,
                         const float* conics, const float* map_opac, int64_t rows_map_opac,
                         const int32_t* cum, int32_t n, int32_t B, int32_t img_h, int32_t img_w,
                         int32_t* keys, int32_t* ids, int64_t cap, float* depth_mm_out) {
    int32_t L[6];
    if (!oracle_key_layout(B, img_h, img_w, L)) return -2;
    const int32_t tbx = L[0], tby = L[1], tile_bits = L[3], depth_bits = L[5];
    const int64_t total = (int64_t)B * n;
    float* mm = (float*)malloc(sizeof(float) * 2 * (size_t)(B > 0 ? B : 1));
    depth_minmax(depths, radii, total, n, B, mm);
    if (depth_mm_out) memcpy(depth_mm_out, mm, sizeof(float) * 2 * (size_t)B);
    const int64_t M = total > 0 ? cum[total - 1] : 0;
    if (M > cap) {
        free(mm);
        return -3;
    }
    const int32_t qmax = (1 << depth_bits) - 1;
    const float maxq = (float)qmax;
#pragma omp parallel for schedule(dynamic, 4096)
    for (int64_t idx = 0; idx < total; ++idx) {
        if (radii[idx] <= 0) continue;
        int32_t bid = (int32_t)(idx / n);
        int64_t cur = idx > 0 ? cum[idx - 1] : 0;
        float dmin = mm[2 * bid];
        float drange = mm[2 * bid + 1] - dmin;
        int32_t dq = 0;
        if (drange > 0.0f) {
            float f = (depths[idx] - dmin) / drange;
            dq = iminw(imaxw(f2i(f * maxq), 0), qmax);
        }
        int32_t iid_enc = (int32_t)((uint32_t)bid << (depth_bits + tile_bits));
        float opac = map_opac[idx % rows_map_opac];
        float t = iso_level(opac);
        Ellipse e;
        ellipse_init(conics[3 * idx], conics[3 * idx + 1], conics[3 * idx + 2], t, xys[2 * idx],
                     xys[2 * idx + 1], tbx, tby, &e);
        if (!e.valid) continue;
        float I[2];
        ellipse_init_span(&e, I);
        for (int32_t u = e.rect_min[0]; u < e.rect_max[0]; ++u) {
            int32_t mn, mx;
            ellipse_column(&e, u, I, &mn, &mx);
            for (int32_t v = mn; v < mx; ++v) {
                int32_t tile_id = e.isY ? u * tbx + v : v * tbx + u;
                keys[cur] = iid_enc | (tile_id << depth_bits) | dq;
                ids[cur] = (int32_t)idx;
                ++cur;
            }
        }
    }
    free(mm);
    return M;
}

/* Stable ascending LSD radix sort of non-negative int32 keys with int32 values (the contract of
 * warp-lang 1.15.0's radix_sort_pairs, called at splax/_rasterize/_sort/_sort.py:136). */
static void radix_sort_pairs(int32_t* keys, int32_t* vals, int64_t m) {
    if (m <= 1) return;
    int32_t* k2 = (int32_t*)malloc(sizeof(int32_t) * (size_t)m);
    int32_t* v2 = (int32_t*)malloc(sizeof(int32_t) * (size_t)m);
    int32_t *ks = keys, *vs = vals, *kd = k2, *vd = v2;
    for (int pass = 0; pass < 4; ++pass) {
        int64_t cnt[257];
        memset(cnt, 0, sizeof(cnt));
        const int sh = 8 * pass;
        for (int64_t i = 0; i < m; ++i) cnt[(((uint32_t)ks[i]) >> sh & 255u) + 1]++;
        for (int d = 0; d < 256; ++d) cnt[d + 1] += cnt[d];
        for (int64_t i = 0; i < m; ++i) {
            int64_t dst = cnt[((uint32_t)ks[i]) >> sh & 255u]++;
            kd[dst] = ks[i];
            vd[dst] = vs[i];
        }
        int32_t* t;
        t = ks; ks = kd; kd = t;
        t = vs; vs = vd; vd = t;
    }
    /* four passes: the result is back in the caller's arrays */
    free(k2);
    free(v2);
}

/* _tile_bin_edges_32bit, splax/_rasterize/_sort/_kernels.py:214-241, including its M == 1
 * behaviour (index 0 returns before writing an end, so a lone bin stays [0, 0)). Bins of tiles
 * without intersections stay (0, 0) from the zeroing at splax/_rasterize/_sort/_sort.py:80-82. */
static void tile_bin_edges(const int32_t* sorted_keys, int64_t M, int32_t num_tiles,
                           int32_t tile_bits, int32_t depth_bits, int32_t* bins) {
    const int32_t mask = (1 << tile_bits) - 1;
    for (int64_t idx = 0; idx < M; ++idx) {
        int32_t key = sorted_keys[idx] >> depth_bits;
        int32_t cur = (key >> tile_bits) * num_tiles + (key & mask);
        if (idx == 0) {
            bins[2 * cur] = 0;
            continue;
        }
        if (idx == M - 1) bins[2 * cur + 1] = (int32_t)M;
        int32_t kp = sorted_keys[idx - 1] >> depth_bits;
        int32_t prev = (kp >> tile_bits) * num_tiles + (kp & mask);
        if (prev != cur) {
            bins[2 * prev + 1] = (int32_t)idx;
            bins[2 * cur] = (int32_t)idx;
        }
    }
}

/* _map_intersects_64bit, splax/_rasterize/_sort/_kernels.py:156-211: the same tile walk, key
 * (image << (32 + tile_bits)) | (tile << 32) | the depth's raw float bits (int32, widened with
 * sign extension; a visible item's depth is positive, so its bits order like the value). */
int64_t oracle_emit_keys_wide(const float* xys, const float* depths, const int32_t* radii,
                              const float* conics, const float* map_opac, int64_t rows_map_opac,
                              const int32_t* cum, int32_t n, int32_t B, int32_t img_h,
                              int32_t img_w, int64_t* keys, int32_t* ids, int64_t cap) {
    int32_t L[6];
    oracle_key_layout(B, img_h, img_w, L);
    const int32_t tbx = L[0], tby = L[1], tile_bits = L[3];
    if (L[3] + L[4] > 32) return -2;
    const int64_t total = (int64_t)B * n;
    const int64_t M = total > 0 ? cum[total - 1] : 0;
    if (M > cap) return -3;
#pragma omp parallel for schedule(dynamic, 4096)
    for (int64_t idx = 0; idx < total; ++idx) {
        if (radii[idx] <= 0) continue;
        int32_t bid = (int32_t)(idx / n);
        int64_t cur = idx > 0 ? cum[idx - 1] : 0;
        int32_t dbits;
        memcpy(&dbits, depths + idx, sizeof(dbits));
        const int64_t depth_id = (int64_t)dbits;
        const int64_t iid_enc = (int64_t)((uint64_t)bid << (32 + tile_bits));
        float opac = map_opac[idx % rows_map_opac];
        float t = iso_level(opac);
        Ellipse e;
        ellipse_init(conics[3 * idx], conics[3 * idx + 1], conics[3 * idx + 2], t, xys[2 * idx],
                     xys[2 * idx + 1], tbx, tby, &e);
        if (!e.valid) continue;
        float I[2];
        ellipse_init_span(&e, I);
        for (int32_t u = e.rect_min[0]; u < e.rect_max[0]; ++u) {
            int32_t mn, mx;
            ellipse_column(&e, u, I, &mn, &mx);
            for (int32_t v = mn; v < mx; ++v) {
                int64_t tile_id = e.isY ? (int64_t)u * tbx + v : (int64_t)v * tbx + u;
                keys[cur] = iid_enc | (int64_t)((uint64_t)tile_id << 32) | depth_id;
                ids[cur] = (int32_t)idx;
                ++cur;
            }
        }
    }
    return M;
}

/* Stable ascending LSD radix sort of 64-bit keys (as unsigned, i.e. by (image, tile, depth))
 * with int32 values; bytes on which every key agrees are skipped. */
static void radix_sort_pairs64(int64_t* keys, int32_t* vals, int64_t m) {
    if (m <= 1) return;
    uint64_t all_or = 0, all_and = ~0ull;
    for (int64_t i = 0; i < m; ++i) {
        all_or |= (uint64_t)keys[i];
        all_and &= (uint64_t)keys[i];
    }
    const uint64_t varying = all_or ^ all_and;
    int64_t* k2 = (int64_t*)malloc(sizeof(int64_t) * (size_t)m);
    int32_t* v2 = (int32_t*)malloc(sizeof(int32_t) * (size_t)m);
    int64_t *ks = keys, *kd = k2;
    int32_t *vs = vals, *vd = v2;
    for (int pass = 0; pass < 8; ++pass) {
        const int sh = 8 * pass;
        if (!((varying >> sh) & 255u)) continue;
        int64_t cnt[257];
        memset(cnt, 0, sizeof(cnt));
        for (int64_t i = 0; i < m; ++i) cnt[(((uint64_t)ks[i]) >> sh & 255u) + 1]++;
        for (int d = 0; d < 256; ++d) cnt[d + 1] += cnt[d];
        for (int64_t i = 0; i < m; ++i) {
            int64_t dst = cnt[((uint64_t)ks[i]) >> sh & 255u]++;
            kd[dst] = ks[i];
            vd[dst] = vs[i];
        }
        int64_t* tk = ks; ks = kd; kd = tk;
        int32_t* tv = vs; vs = vd; vd = tv;
    }
    if (ks != keys) {
        memcpy(keys, ks, sizeof(int64_t) * (size_t)m);
        memcpy(vals, vs, sizeof(int32_t) * (size_t)m);
    }
    free(k2);
    free(v2);
}

/* _tile_bin_edges_64bit, splax/_rasterize/_sort/_kernels.py:244-269 (same M == 1 behaviour). */
static void tile_bin_edges64(const int64_t* sorted_keys, int64_t M, int32_t num_tiles,
                             int32_t tile_bits, int32_t* bins) {
    const int64_t mask = ((int64_t)1 << tile_bits) - 1;
    for (int64_t idx = 0; idx < M; ++idx) {
        int64_t key = (int64_t)((uint64_t)sorted_keys[idx] >> 32);
        int32_t cur = (int32_t)(key >> tile_bits) * num_tiles + (int32_t)(key & mask);
        if (idx == 0) {
            bins[2 * cur] = 0;
            continue;
        }
        if (idx == M - 1) bins[2 * cur + 1] = (int32_t)M;
        int64_t kp = (int64_t)((uint64_t)sorted_keys[idx - 1] >> 32);
        int32_t prev = (int32_t)(kp >> tile_bits) * num_tiles + (int32_t)(kp & mask);
        if (prev != cur) {
            bins[2 * prev + 1] = (int32_t)idx;
            bins[2 * cur] = (int32_t)idx;
        }
    }
}

/* sort_and_bin, 64-bit key path (splax/_rasterize/_sort/_sort.py:143-170) */
int64_t oracle_sort_and_bin_wide(const float* xys, const float* depths, const int32_t* radii,
                                 const float* conics, const float* map_opac,
                                 int64_t rows_map_opac, const int32_t* cum, int32_t n, int32_t B,
                                 int32_t img_h, int32_t img_w, int64_t* sorted_keys,
                                 int32_t* sorted_ids, int64_t cap, int32_t* tile_bins) {
    int32_t L[6];
    oracle_key_layout(B, img_h, img_w, L);
    if (L[3] + L[4] > 32) return -2;
    memset(tile_bins, 0, sizeof(int32_t) * 2 * (size_t)B * (size_t)L[2]);
    int64_t M = oracle_emit_keys_wide(xys, depths, radii, conics, map_opac, rows_map_opac, cum,
                                      n, B, img_h, img_w, sorted_keys, sorted_ids, cap);
    if (M <= 0) return M;
    radix_sort_pairs64(sorted_keys, sorted_ids, M);
    tile_bin_edges64(sorted_keys, M, L[2], L[3], tile_bins);
    return M;
}

/* Sorted ids and bins through whichever key the layout takes (ids [cap], bins [B*tiles*2]). */
static int64_t sort_ids_and_bins(const float* xys, const float* depths, const int32_t* radii,
                                 const float* conics, const float* map_opac,
                                 int64_t rows_map_opac, const int32_t* cum, int32_t n, int32_t B,
                                 int32_t img_h, int32_t img_w, int32_t* ids, int64_t cap,
                                 int32_t* bins);

/* sort_and_bin, splax/_rasterize/_sort/_sort.py:29-171 (packed 32-bit key path) */
int64_t oracle_sort_and_bin(const float* xys, const float* depths, const int32_t* radii,
                            const float* conics, const float* map_opac, int64_t rows_map_opac,
                            const int32_t* cum, int32_t n, int32_t B, int32_t img_h,
                            int32_t img_w, int32_t* sorted_keys, int32_t* sorted_ids,
                            int64_t cap, int32_t* tile_bins) {
    int32_t L[6];
    if (!oracle_key_layout(B, img_h, img_w, L) || g_force_wide) return -2;
    memset(tile_bins, 0, sizeof(int32_t) * 2 * (size_t)B * (size_t)L[2]);
    int64_t M = oracle_emit_keys(xys, depths, radii, conics, map_opac, rows_map_opac, cum, n, B,
                                 img_h, img_w, sorted_keys, sorted_ids, cap, NULL);
    if (M <= 0) return M;
    radix_sort_pairs(sorted_keys, sorted_ids, M);
    tile_bin_edges(sorted_keys, M, L[2], L[3], L[5], tile_bins);
    return M;
}

static int64_t sort_ids_and_bins(const float* xys, const float* depths, const int32_t* radii,
                                 const float* conics, const float* map_opac,
                                 int64_t rows_map_opac, const int32_t* cum, int32_t n, int32_t B,
                                 int32_t img_h, int32_t img_w, int32_t* ids, int64_t cap,
                                 int32_t* bins) {
    const int mode = oracle_key_mode(B, img_h, img_w);
    if (mode < 0) return mode;
    const size_t m = (size_t)(cap > 0 ? cap : 1);
    if (mode == 0) {
        int32_t* keys = (int32_t*)malloc(sizeof(int32_t) * m);
        int64_t M = oracle_sort_and_bin(xys, depths, radii, conics, map_opac, rows_map_opac, cum,
                                        n, B, img_h, img_w, keys, ids, cap, bins);
        free(keys);
        return M;
    }
    int64_t* keys = (int64_t*)malloc(sizeof(int64_t) * m);
    int64_t M = oracle_sort_and_bin_wide(xys, depths, radii, conics, map_opac, rows_map_opac,
                                         cum, n, B, img_h, img_w, keys, ids, cap, bins);
    free(keys);
    return M;
}

/* ---------------------------------------------------------------- forward blend
 * _rasterize_kernel, splax/_rasterize/_kernels.py:102-205. Per pixel the blend walks the tile's
 * sorted range front to back; the block-wide batching and early-exit vote of the reference do not
 * change any pixel's result, so the oracle walks each pixel's range directly. With out_depth the
 * walk also accumulates the expected depth, _rasterize_depth_kernel (:277-383): depth[g] times the
 * same blend weight, no background term. */

void oracle_blend_fwd(const float* colors, int64_t rows_colors, const float* opacities,
                      int64_t rows_opac, const float* background, int64_t rows_bg,
                      const float* xys, const float* conics, const int32_t* sorted_ids,
                      const int32_t* tile_bins, int32_t B, int32_t img_h, int32_t img_w,
                      float* final_Ts, int32_t* final_idx, float* out_img, int64_t* stats,
                      const float* depths, float* out_depth) {
    const int32_t tbx = (img_w + BLOCK_WIDTH - 1) / BLOCK_WIDTH;
    const int32_t tby = (img_h + BLOCK_WIDTH - 1) / BLOCK_WIDTH;
    const int32_t num_tiles = tbx * tby;
    const int sel_bg = rows_bg > 1;
    int64_t pc = 0, pr = 0;
    const int64_t rows_total = (int64_t)B * img_h;
#pragma omp parallel for schedule(dynamic, 4) reduction(+ : pc, pr)
    for (int64_t row = 0; row < rows_total; ++row) {
        const int32_t image = (int32_t)(row / img_h), i = (int32_t)(row % img_h);
        const float* bg = background + 3 * (sel_bg ? image : 0);
        {
            for (int32_t j = 0; j < img_w; ++j) {
                int32_t tile = image * num_tiles + (i / BLOCK_WIDTH) * tbx + j / BLOCK_WIDTH;
                int32_t start = tile_bins[2 * tile], end = tile_bins[2 * tile + 1];
                float px = (float)j + 0.5f, py = (float)i + 0.5f;
                float T = 1.0f;
                int32_t cur_idx = 0;
                float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, od = 0.0f;
                for (int32_t k = start; k < end; ++k) {
                    int64_t g = sorted_ids[k];
                    float dx = xys[2 * g] - px, dy = xys[2 * g + 1] - py;
                    float sigma = blend_sigma(conics + 3 * g, dx, dy);
                    float op = opacities[g % rows_opac];
                    float alpha = fminw(ALPHA_MAX, op * oracle_blend_expf(-sigma));
                    /* !(alpha >= threshold): a NaN opacity is rejected, as the GPU's pack
                     * culls such records */
                    if (sigma < 0.0f || sigma > BLEND_SIGMA_CAP || !(alpha >= ALPHA_THRESHOLD)) {
                        ++pr;
                        continue;
                    }
                    float next_T = T * (1.0f - alpha);
                    if (next_T <= T_EPS) {
                        ++pr;
                        break;
                    }
                    ++pc;
                    float vis = alpha * T;
                    const float* c = colors + 3 * (g % rows_colors);
                    o0 = fmaf(c[0], vis, o0);
                    o1 = fmaf(c[1], vis, o1);
                    o2 = fmaf(c[2], vis, o2);
                    if (out_depth) od = fmaf(depths[g], vis, od);
                    T = next_T;
                    cur_idx = k;
                }
                int64_t row = (int64_t)image * img_h + i;
                int64_t pix = row * img_w + j;
                final_Ts[pix] = T;
                final_idx[pix] = cur_idx;
                out_img[3 * pix] = o0 + T * bg[0];
                out_img[3 * pix + 1] = o1 + T * bg[1];
                out_img[3 * pix + 2] = o2 + T * bg[2];
                if (out_depth) out_depth[pix] = od;
            }
        }
    }
    if (stats) {
        stats[0] = pc;
        stats[1] = pr;
    }
}

int64_t oracle_rasterize_fwd(const float* colors, int64_t rows_colors, const float* opacities,
                             int64_t rows_opac, const float* map_opac, int64_t rows_map_opac,
                             const float* background, int64_t rows_bg, const float* xys,
                             const float* depths, const int32_t* radii, const float* conics,
                             const int32_t* cum, int32_t n, int32_t B, int32_t img_h,
                             int32_t img_w, float* final_Ts, int32_t* final_idx, float* out_img,
                             int64_t* stats, float* out_depth) {
    int32_t L[6];
    oracle_key_layout(B, img_h, img_w, L);
    const int64_t total = (int64_t)B * n;
    const int64_t M = total > 0 ? cum[total - 1] : 0;
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)(M > 0 ? M : 1));
    int32_t* bins = (int32_t*)malloc(sizeof(int32_t) * 2 * (size_t)B * (size_t)L[2]);
    int64_t m = sort_ids_and_bins(xys, depths, radii, conics, map_opac, rows_map_opac, cum, n, B,
                                  img_h, img_w, ids, M, bins);
    if (m >= 0)
        oracle_blend_fwd(colors, rows_colors, opacities, rows_opac, background, rows_bg, xys,
                         conics, ids, bins, B, img_h, img_w, final_Ts, final_idx, out_img, stats,
                         depths, out_depth);
    free(ids);
    free(bins);
    return m;
}

/* ---------------------------------------------------------------- backward blend
 * _rasterize_bwd_warp + _rasterize_bwd_kernel, splax/_rasterize/_kernels.py:386-500,530-665, with
 * _blend_color_vjp (:1212-1254). Per pixel the walk visits sorted indices bin_final down to
 * range_start, exactly the pairs the staged and aggregated reference kernels visit. Gradients are
 * accumulated in double here (the reference's float atomics have no fixed order). With v_depths,
 * the depth-channel backward _rasterize_bwd_depth_warp / _kernel (:797-1080) with
 * _blend_depth_vjp (:1257-1302): the depth term joins v_alpha after the colour terms, its own
 * accumulator dbuffer, and v_depth = v_out_depth * fac per pair.
 *
 * truth != 0 evaluates the same walk in double: the pairs and their accept decisions (sigma
 * range, alpha threshold, the 0.999 clamp) are the float walk's, and every value after them
 * (sigma, e^-sigma, alpha, T, the colour buffer, v_alpha and the gradient terms) is formed in
 * double from the float32 inputs. That is the float64 truth of the reference's backward formulas
 * at the float forward's decisions, against which float32 evaluations are measured. */

static int64_t rasterize_bwd_walk(const float* colors, int64_t rows_colors,
                                  const float* opacities, int64_t rows_opac,
                                  const float* map_opac, int64_t rows_map_opac,
                                  const float* background, int64_t rows_bg, const float* xys,
                                  const float* depths, const int32_t* radii, const float* conics,
                                  const int32_t* cum, const float* final_Ts,
                                  const int32_t* final_idx, const float* v_out_img,
                                  int64_t vout_rows, int32_t n, int32_t B_out, int32_t B_geom,
                                  int32_t img_h, int32_t img_w, int64_t* stats,
                                  const float* v_out_depth, int64_t vdepth_rows, int with_depth,
                                  int truth, double* acc) {
    const int NG = with_depth ? 10 : 9;
    int32_t L[6];
    oracle_key_layout(B_geom, img_h, img_w, L);
    const int32_t tbx = L[0], num_tiles = L[2];
    const int64_t total = (int64_t)B_geom * n;
    const int64_t M = total > 0 ? cum[total - 1] : 0;
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)(M > 0 ? M : 1));
    int32_t* bins = (int32_t*)malloc(sizeof(int32_t) * 2 * (size_t)B_geom * (size_t)num_tiles);
    int64_t m = sort_ids_and_bins(xys, depths, radii, conics, map_opac, rows_map_opac, cum, n,
                                  B_geom, img_h, img_w, ids, M, bins);
    const int sel_geom = B_geom > 1, sel_bg = rows_bg > 1;
    int64_t qc = 0, qr = 0;
    if (m > 0) {
        const int64_t rows_total = (int64_t)B_out * img_h;
#pragma omp parallel for schedule(dynamic, 4) reduction(+ : qc, qr)
        for (int64_t row = 0; row < rows_total; ++row) {
            const int32_t image = (int32_t)(row / img_h), i = (int32_t)(row % img_h);
            const int32_t geom_image = sel_geom ? image : 0;
            const int64_t og_base = sel_geom ? 0 : (int64_t)image * n;
            const float* bg = background + 3 * (sel_bg ? image : 0);
            for (int32_t j = 0; j < img_w; ++j) {
                int32_t tile_local = (i / BLOCK_WIDTH) * tbx + j / BLOCK_WIDTH;
                int32_t tile = geom_image * num_tiles + tile_local;
                int32_t start = bins[2 * tile], end = bins[2 * tile + 1];
                if (end <= start) continue;
                int64_t frow = (int64_t)geom_image * img_h + i;
                int32_t bin_final = final_idx[frow * img_w + j];
                float t_final = final_Ts[frow * img_w + j];
                float T = t_final;
                const float* vo =
                    v_out_img + 3 * ((((int64_t)image * img_h + i) % vout_rows) * img_w + j);
                const float vd =
                    with_depth
                        ? v_out_depth[(((int64_t)image * img_h + i) % vdepth_rows) * img_w + j]
                        : 0.0f;
                float px = (float)j + 0.5f, py = (float)i + 0.5f;
                float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f, db = 0.0f;
                /* truth: the same state in double */
                double Td = (double)t_final, b0d = 0.0, b1d = 0.0, b2d = 0.0, dbd = 0.0;
                for (int32_t k = bin_final; k >= start; --k) {
                    int64_t g = ids[k];
                    float dx = xys[2 * g] - px, dy = xys[2 * g + 1] - py;
                    const float* cn = conics + 3 * g;
                    float a = cn[0], b = cn[1], c = cn[2];
                    float sigma = blend_sigma(cn, dx, dy);
                    if (sigma < 0.0f || sigma > BLEND_SIGMA_CAP) {
                        ++qr;
                        continue;
                    }
                    float vis = oracle_blend_expf(-sigma);
                    float op = opacities[g % rows_opac];
                    float alpha = fminw(ALPHA_MAX, op * vis);
                    if (!(alpha >= ALPHA_THRESHOLD)) {
                        ++qr;
                        continue;
                    }
                    ++qc;
                    const float* col = colors + 3 * (g % rows_colors);
                    const int geo = op * vis <= ALPHA_MAX;
                    const float dep = with_depth ? depths[g] : 0.0f;
                    double* o = acc + NG * (og_base + g);
                    double gr[10] = {0};
                    if (truth) {
                        const double dxd = (double)xys[2 * g] - ((double)j + 0.5);
                        const double dyd = (double)xys[2 * g + 1] - ((double)i + 0.5);
                        const double sd = 0.5 * ((double)a * dxd * dxd + (double)c * dyd * dyd) +
                                          (double)b * dxd * dyd;
                        const double visd = exp(-sd);
                        const double ad = geo ? (double)op * visd : (double)ALPHA_MAX;
                        const double rad = 1.0 / (1.0 - ad);
                        Td = Td * rad;
                        const double facd = ad * Td;
                        double va = ((double)col[0] * Td - b0d * rad) * (double)vo[0] +
                                    ((double)col[1] * Td - b1d * rad) * (double)vo[1] +
                                    ((double)col[2] * Td - b2d * rad) * (double)vo[2];
                        if (with_depth) va += ((double)dep * Td - dbd * rad) * (double)vd;
                        va -= (double)t_final * rad *
                              ((double)bg[0] * vo[0] + (double)bg[1] * vo[1] +
                               (double)bg[2] * vo[2]);
                        b0d += (double)col[0] * facd;
                        b1d += (double)col[1] * facd;
                        b2d += (double)col[2] * facd;
                        if (with_depth) dbd += (double)dep * facd;
                        gr[0] = vo[0] * facd;
                        gr[1] = vo[1] * facd;
                        gr[2] = vo[2] * facd;
                        if (geo) {
                            const double vs = -(double)op * visd * va;
                            gr[3] = 0.5 * vs * dxd * dxd;
                            gr[4] = vs * dxd * dyd;
                            gr[5] = 0.5 * vs * dyd * dyd;
                            gr[6] = vs * ((double)a * dxd + (double)b * dyd);
                            gr[7] = vs * ((double)b * dxd + (double)c * dyd);
                            gr[8] = visd * va;
                        }
                        gr[9] = (double)vd * facd;
                    } else {
                        /* _blend_color_vjp */
                        float ra = 1.0f / (1.0f - alpha);
                        T = T * ra;
                        float fac = alpha * T;
                        float v_alpha = (col[0] * T - b0 * ra) * vo[0];
                        v_alpha += (col[1] * T - b1 * ra) * vo[1];
                        v_alpha += (col[2] * T - b2 * ra) * vo[2];
                        if (with_depth) v_alpha += (dep * T - db * ra) * vd;
                        v_alpha += -t_final * ra * bg[0] * vo[0];
                        v_alpha += -t_final * ra * bg[1] * vo[1];
                        v_alpha += -t_final * ra * bg[2] * vo[2];
                        b0 = b0 + col[0] * fac;
                        b1 = b1 + col[1] * fac;
                        b2 = b2 + col[2] * fac;
                        if (with_depth) db = db + dep * fac;
                        gr[0] = (double)(vo[0] * fac);
                        gr[1] = (double)(vo[1] * fac);
                        gr[2] = (double)(vo[2] * fac);
                        if (geo) {
                            float v_sigma = -op * vis * v_alpha;
                            gr[3] = (double)(0.5f * v_sigma * dx * dx);
                            gr[4] = (double)(v_sigma * dx * dy);
                            gr[5] = (double)(0.5f * v_sigma * dy * dy);
                            gr[6] = (double)(v_sigma * (a * dx + b * dy));
                            gr[7] = (double)(v_sigma * (b * dx + c * dy));
                            gr[8] = (double)(vis * v_alpha);
                        }
                        gr[9] = (double)(vd * fac);
                    }
                    const int ng = geo ? 9 : 3;
                    if (with_depth) {
#pragma omp atomic
                        o[9] += gr[9];
                    }
                    for (int q = 0; q < ng; ++q) {
#pragma omp atomic
                        o[q] += gr[q];
                    }
                }
            }
        }
    }
    if (stats) {
        stats[0] = qc;
        stats[1] = qr;
    }
    free(ids);
    free(bins);
    return m;
}

int64_t oracle_rasterize_bwd(const float* colors, int64_t rows_colors, const float* opacities,
                             int64_t rows_opac, const float* map_opac, int64_t rows_map_opac,
                             const float* background, int64_t rows_bg, const float* xys,
                             const float* depths, const int32_t* radii, const float* conics,
                             const int32_t* cum, const float* final_Ts, const int32_t* final_idx,
                             const float* v_out_img, int64_t vout_rows, int32_t n, int32_t B_out,
                             int32_t B_geom, int32_t img_h, int32_t img_w, float* v_colors,
                             float* v_opacity, float* v_xy, float* v_conic, int64_t* stats,
                             const float* v_out_depth, int64_t vdepth_rows, float* v_depths) {
    const int with_depth = v_depths != NULL;
    const int NG = with_depth ? 10 : 9;
    const int64_t nout = (int64_t)B_out * n;
    double* acc = (double*)calloc((size_t)(nout > 0 ? nout : 1) * NG, sizeof(double));
    int64_t m = rasterize_bwd_walk(colors, rows_colors, opacities, rows_opac, map_opac,
                                   rows_map_opac, background, rows_bg, xys, depths, radii, conics,
                                   cum, final_Ts, final_idx, v_out_img, vout_rows, n, B_out,
                                   B_geom, img_h, img_w, stats, v_out_depth, vdepth_rows,
                                   with_depth, 0, acc);
    for (int64_t g = 0; g < nout; ++g) {
        const double* o = acc + NG * g;
        if (with_depth) v_depths[g] = (float)o[9];
        v_colors[3 * g] = (float)o[0];
        v_colors[3 * g + 1] = (float)o[1];
        v_colors[3 * g + 2] = (float)o[2];
        v_conic[3 * g] = (float)o[3];
        v_conic[3 * g + 1] = (float)o[4];
        v_conic[3 * g + 2] = (float)o[5];
        v_xy[2 * g] = (float)o[6];
        v_xy[2 * g + 1] = (float)o[7];
        v_opacity[g] = (float)o[8];
    }
    free(acc);
    return m;
}

/* The float64 truth of oracle_rasterize_bwd (the walk above with truth set): the per-item sums
 * [nout, 9] (or 10 with v_out_depth) in the order v_colour (3), v_conic (3), v_xy (2),
 * v_opacity, v_depth, in double. */
int64_t oracle_rasterize_bwd_f64(const float* colors, int64_t rows_colors, const float* opacities,
                                 int64_t rows_opac, const float* map_opac, int64_t rows_map_opac,
                                 const float* background, int64_t rows_bg, const float* xys,
                                 const float* depths, const int32_t* radii, const float* conics,
                                 const int32_t* cum, const float* final_Ts,
                                 const int32_t* final_idx, const float* v_out_img,
                                 int64_t vout_rows, int32_t n, int32_t B_out, int32_t B_geom,
                                 int32_t img_h, int32_t img_w, const float* v_out_depth,
                                 int64_t vdepth_rows, double* out) {
    const int with_depth = v_out_depth != NULL;
    const int NG = with_depth ? 10 : 9;
    const int64_t nout = (int64_t)B_out * n;
    memset(out, 0, sizeof(double) * (size_t)(nout > 0 ? nout : 0) * NG);
    return rasterize_bwd_walk(colors, rows_colors, opacities, rows_opac, map_opac, rows_map_opac,
                              background, rows_bg, xys, depths, radii, conics, cum, final_Ts,
                              final_idx, v_out_img, vout_rows, n, B_out, B_geom, img_h, img_w,
                              NULL, v_out_depth, vdepth_rows, with_depth, 1, out);
}

/* ---------------------------------------------------------------- projection backward
 * _project_bwd_kernel, splax/_project/_kernels.py:356-484, with _proj_vjp (:487-533),
 * _transform_vjp (:536-557), _scale_vjp (:560-567), _quat_vjp (:570-599) and _view_vjp
 * (:602-606). Per item the math is fixed; the viewmat and transform reductions are summed in
 * double here. */

int oracle_project_bwd(const float* means3d, int64_t rows_means, const float* scales,
                       int64_t rows_scales, const float* quats, int64_t rows_quats,
                       const float* viewmat, int64_t rows_viewmat, const int32_t* radii,
                       int64_t rows_radii, const float* conics, int64_t rows_conics,
                       const float* v_xy_in, int64_t rows_vxy, const float* v_depth_in,
                       int64_t rows_vdepth, const float* v_conic_in, int64_t rows_vconic,
                       const float* transforms, int64_t rows_transforms,
                       const int32_t* transform_ids, int32_t n, int32_t num_transforms,
                       int32_t has_transforms, int32_t B, float fx, float fy, float glob_scale,
                       float* v_mean3d, float* v_scale, float* v_quat, float* v_viewmat,
                       float* v_transforms) {
    const int sel_means = rows_means > n, sel_scales = rows_scales > n, sel_quats = rows_quats > n;
    const int sel_view = rows_viewmat > 4, sel_radii = rows_radii > n;
    const int sel_conics = rows_conics > n, sel_vxy = rows_vxy > n, sel_vdepth = rows_vdepth > n;
    const int sel_vconic = rows_vconic > n, sel_tf = rows_transforms > num_transforms;
    const int64_t total = (int64_t)B * n;
    double* vview = (double*)calloc((size_t)B * 16, sizeof(double));
    const int64_t ntf = (int64_t)B * (num_transforms > 0 ? num_transforms : 1);
    double* vtf = (double*)calloc((size_t)ntf * 16, sizeof(double));
#pragma omp parallel
    {
    double* vview_loc = (double*)calloc((size_t)B * 16, sizeof(double));
    double* vtf_loc = (double*)calloc((size_t)ntf * 16, sizeof(double));
#pragma omp for schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int32_t image_id = (int32_t)(idx / n), gid = (int32_t)(idx % n);
        for (int k = 0; k < 3; ++k) v_mean3d[3 * idx + k] = 0.0f, v_scale[3 * idx + k] = 0.0f;
        for (int k = 0; k < 4; ++k) v_quat[4 * idx + k] = 0.0f;
        int64_t r_idx = sel_radii ? idx : gid;
        if (radii[r_idx] <= 0) continue;
        int64_t m_idx = sel_means ? idx : gid, s_idx = sel_scales ? idx : gid;
        int64_t q_idx = sel_quats ? idx : gid, c_idx = sel_conics ? idx : gid;
        int64_t vx_idx = sel_vxy ? idx : gid, vd_idx = sel_vdepth ? idx : gid;
        int64_t vc_idx = sel_vconic ? idx : gid;
        int64_t vb = (int64_t)(sel_view ? image_id : 0) * 4;
        int32_t tf_id = has_transforms ? transform_ids[gid] : -1;
        const float* mean_local = means3d + 3 * m_idx;
        float mean[3] = {mean_local[0], mean_local[1], mean_local[2]};
        float R_tf[9];
        int moved = apply_transform(transforms, image_id, num_transforms, sel_tf, tf_id, mean, R_tf);
        float W[9], p[3], M[9];
        const float* q = quats + 4 * q_idx;
        project_geom(mean, q, scales + 3 * s_idx, glob_scale, viewmat + vb * 4, R_tf, moved, W, p,
                     M, NULL);
        float V[9];
        mat_mul_nt(M, M, V);
        float R[9];
        quat_to_rot(q, R);
        const float* sc = scales + 3 * s_idx;
        float s[3] = {glob_scale * sc[0], glob_scale * sc[1], glob_scale * sc[2]};
        float rz = 1.0f / p[2];
        float rz2 = rz * rz;
        /* J = [[j00, 0, j02], [0, j11, j12], [0, 0, 0]] from the unclamped position (:428-431).
         * The products of this VJP drop every term with a structural zero factor (J's last row;
         * the last row and column of the 2D covariance cotangent) and keep the others in the full
         * 3x3 products' order, as the GPU kernel does. */
        const float j00 = fx * rz, j02 = -fx * p[0] * rz2;
        const float j11 = fy * rz, j12 = -fy * p[1] * rz2;
        float T0[3], T1[3]; /* rows 0 and 1 of T = J W (row 2 is zero) */
        for (int b = 0; b < 3; ++b) {
            T0[b] = j00 * W[b] + j02 * W[6 + b];
            T1[b] = j11 * W[3 + b] + j12 * W[6 + b];
        }
        /* S = X G X, vcov2d (:434-439) */
        const float* cn = conics + 3 * c_idx;
        const float* vc = v_conic_in + 3 * vc_idx;
        float X[4] = {cn[0], cn[1], cn[1], cn[2]};
        float G[4] = {vc[0], 0.5f * vc[1], 0.5f * vc[1], vc[2]};
        float XG[4] = {X[0] * G[0] + X[1] * G[2], X[0] * G[1] + X[1] * G[3],
                       X[2] * G[0] + X[3] * G[2], X[2] * G[1] + X[3] * G[3]};
        float S[4] = {XG[0] * X[0] + XG[1] * X[2], XG[0] * X[1] + XG[1] * X[3],
                      XG[2] * X[0] + XG[3] * X[2], XG[2] * X[1] + XG[3] * X[3]};
        float vcov[3] = {-S[0], -(S[1] + S[2]), -S[3]};
        /* _proj_vjp (:487-533) */
        float tx = p[0], ty = p[1], tz = p[2];
        float prz = 1.0f / tz;
        float prz2 = prz * prz;
        float prz3 = prz2 * prz;
        float rw = 1.0f / (tz + Z_EPS);
        const float* vxy = v_xy_in + 2 * vx_idx;
        float vpx = fx * vxy[0], vpy = fy * vxy[1];
        float vvx = vpx * rw, vvy = vpy * rw;
        float vvz = -(vpx * tx + vpy * ty) * rw * rw;
        vvz = vvz + v_depth_in[vd_idx];
        /* v_cov = [[c0, c1, 0], [c1, c2, 0], [0, 0, 0]] */
        const float c0 = vcov[0], c1 = 0.5f * vcov[1], c2 = vcov[2];
        /* v_V = T^T v_cov T (T^T v_cov has a zero last column) */
        float tmp0[3], tmp1[3], v_V[9];
        for (int a = 0; a < 3; ++a) {
            tmp0[a] = T0[a] * c0 + T1[a] * c1;
            tmp1[a] = T0[a] * c1 + T1[a] * c2;
        }
        for (int a = 0; a < 3; ++a)
            for (int b = 0; b < 3; ++b) v_V[3 * a + b] = tmp0[a] * T0[b] + tmp1[a] * T1[b];
        /* v_T = (2 v_cov) T V, rows 0 and 1 (row 2 is zero) */
        const float d0 = 2.0f * c0, d1 = 2.0f * c1, d2 = 2.0f * c2;
        float u0[3], u1[3], v_T[6];
        for (int b = 0; b < 3; ++b) {
            u0[b] = d0 * T0[b] + d1 * T1[b];
            u1[b] = d1 * T0[b] + d2 * T1[b];
        }
        for (int b = 0; b < 3; ++b) {
            v_T[b] = (u0[0] * V[b] + u0[1] * V[3 + b]) + u0[2] * V[6 + b];
            v_T[3 + b] = (u1[0] * V[b] + u1[1] * V[3 + b]) + u1[2] * V[6 + b];
        }
        /* v_J = v_T W^T, rows 0 and 1 */
        float v_J[6];
        for (int a = 0; a < 2; ++a)
            for (int b = 0; b < 3; ++b)
                v_J[3 * a + b] = (v_T[3 * a] * W[3 * b] + v_T[3 * a + 1] * W[3 * b + 1]) +
                                 v_T[3 * a + 2] * W[3 * b + 2];
        float v_t_x = -fx * prz2 * v_J[2];
        float v_t_y = -fy * prz2 * v_J[5];
        float v_t_z = -fx * prz2 * v_J[0] + 2.0f * fx * tx * prz3 * v_J[2] - fy * prz2 * v_J[4] +
                      2.0f * fy * ty * prz3 * v_J[5];
        float v_p[3] = {vvx + v_t_x, vvy + v_t_y, vvz + v_t_z};
        /* world-space cotangents (:441-442) */
        float v_mean_world[3];
        mat_t_vec(W, v_p, v_mean_world);
        float vVs[9], v_M_world[9];
        for (int a = 0; a < 3; ++a)
            for (int b = 0; b < 3; ++b) vVs[3 * a + b] = v_V[3 * a + b] + v_V[3 * b + a];
        mat_mul(vVs, M, v_M_world);
        /* _transform_vjp (:536-557) */
        float v_mean_out[3], v_M[9], v_R_tf[9] = {0}, v_t_tf[3] = {0};
        if (moved) {
            mat_t_vec(R_tf, v_mean_world, v_mean_out);
            mat_mul_tn(R_tf, v_M_world, v_M);
            float M_local[9];
            mat_mul_tn(R_tf, M, M_local);
            float vmMl[9];
            mat_mul_nt(v_M_world, M_local, vmMl);
            for (int a = 0; a < 3; ++a)
                for (int b = 0; b < 3; ++b)
                    v_R_tf[3 * a + b] = v_mean_world[a] * mean_local[b] + vmMl[3 * a + b];
            for (int a = 0; a < 3; ++a) v_t_tf[a] = v_mean_world[a];
        } else {
            memcpy(v_mean_out, v_mean_world, sizeof(v_mean_out));
            memcpy(v_M, v_M_world, sizeof(v_M));
        }
        for (int k = 0; k < 3; ++k) v_mean3d[3 * idx + k] = v_mean_out[k];
        /* _scale_vjp (:560-567) */
        for (int jj = 0; jj < 3; ++jj)
            v_scale[3 * idx + jj] =
                ((R[jj] * v_M[jj] + R[3 + jj] * v_M[3 + jj]) + R[6 + jj] * v_M[6 + jj]) *
                glob_scale;
        /* _quat_vjp (:570-599), gradient of the unit-form rotation, output xyzw */
        float vR[9];
        for (int a = 0; a < 3; ++a)
            for (int b = 0; b < 3; ++b) vR[3 * a + b] = v_M[3 * a + b] * s[b];
        float x = q[0], y = q[1], z = q[2], w = q[3];
        float vq_w = 2.0f * ((x * (vR[7] - vR[5]) + y * (vR[2] - vR[6])) + z * (vR[3] - vR[1]));
        float vq_x = 2.0f * (((-2.0f * x * (vR[4] + vR[8]) + y * (vR[3] + vR[1])) +
                              z * (vR[6] + vR[2])) + w * (vR[7] - vR[5]));
        float vq_y = 2.0f * (((x * (vR[3] + vR[1]) - 2.0f * y * (vR[0] + vR[8])) +
                              z * (vR[7] + vR[5])) + w * (vR[2] - vR[6]));
        float vq_z = 2.0f * (((x * (vR[6] + vR[2]) + y * (vR[7] + vR[5])) -
                              2.0f * z * (vR[0] + vR[4])) + w * (vR[3] - vR[1]));
        v_quat[4 * idx] = vq_x;
        v_quat[4 * idx + 1] = vq_y;
        v_quat[4 * idx + 2] = vq_z;
        v_quat[4 * idx + 3] = vq_w;
        /* _view_vjp (:602-606): v_R = v_p (x) mean + J^T v_T, v_t = v_p */
        float JtvT[9]; /* J^T v_T */
        for (int b = 0; b < 3; ++b) {
            JtvT[b] = j00 * v_T[b];
            JtvT[3 + b] = j11 * v_T[3 + b];
            JtvT[6 + b] = j02 * v_T[b] + j12 * v_T[3 + b];
        }
        double* vv = vview_loc + 16 * (int64_t)image_id;
        for (int a = 0; a < 3; ++a) {
            for (int b = 0; b < 3; ++b) vv[4 * a + b] += v_p[a] * mean[b] + JtvT[3 * a + b];
            vv[4 * a + 3] += v_p[a];
        }
        if (moved) {
            double* vt = vtf_loc + 16 * ((int64_t)image_id * num_transforms + tf_id);
            for (int a = 0; a < 3; ++a) {
                for (int b = 0; b < 3; ++b) vt[4 * a + b] += v_R_tf[3 * a + b];
                vt[4 * a + 3] += v_t_tf[a];
            }
        }
    }
#pragma omp critical
    {
        for (int64_t k = 0; k < (int64_t)B * 16; ++k) vview[k] += vview_loc[k];
        for (int64_t k = 0; k < ntf * 16; ++k) vtf[k] += vtf_loc[k];
    }
    free(vview_loc);
    free(vtf_loc);
    }
    for (int64_t k = 0; k < (int64_t)B * 16; ++k) v_viewmat[k] = (float)vview[k];
    if (num_transforms > 0)
        for (int64_t k = 0; k < (int64_t)B * num_transforms * 16; ++k)
            v_transforms[k] = (float)vtf[k];
    free(vview);
    free(vtf);
    return 0;
}

/* ---------------------------------------------------------------- vector helpers for tests */

void oracle_logf_n(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_logf(x[i]);
}

void oracle_expf_n(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_expf(x[i]);
}

void oracle_blend_expf_n(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_blend_expf(x[i]);
}

#ifdef _OPENMP
#include <omp.h>
#endif

/* Thread count of the OpenMP loops (projection, emission, blends, projection VJP). */
int oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}
