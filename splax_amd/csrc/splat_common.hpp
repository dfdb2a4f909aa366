// Shared device code of the gfx950 splat library: constants, fixed-sequence float math and the
// opacity-aware ellipse tile walk. Projection (tile count) and key emission both call the same
// inline functions from this header, so the counted and the emitted tile totals agree exactly
// (the invariant splax relies on in splax/_intersect.py:1-8).
//
// Arithmetic contract: IEEE binary32, round-to-nearest-even, no FMA contraction (the library is
// compiled with -ffp-contract=off); FMAs appear only as explicit fmaf(). Division and sqrt are
// correctly rounded (HIP's default). min(a, b) = a < b ? a : b, max(a, b) = a > b ? a : b, and
// float -> int32 truncates toward zero, saturates, and maps NaN to 0. 3x3 products associate as
// (a0*b0 + a1*b1) + a2*b2. These rules make every non-atomic output reproducible on any IEEE
// machine that follows the same sequence.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace splat {

// splax/_intersect.py:17-20
constexpr int kBlockWidth = 16;
constexpr int kBlockSize = 256;
constexpr float kExtendSq = 0x1.62d844p+3f;   // float32(3.33 * 3.33)
constexpr float kAlphaThresh = 0x1.010102p-8f; // float32(1 / 255)
constexpr float kAlphaMax = 0x1.ff7ceep-1f;    // float32(0.999)
constexpr float kTEps = 0x1.a36e2ep-14f;       // float32(1e-4)
constexpr float kDilation = 0x1.333334p-2f;    // float32(0.3), splax/_project/_kernels.py:204-206
constexpr float kFovClamp = 0x1.4ccccdp+0f;    // float32(1.3), splax/_project/_kernels.py:191-192
constexpr float kZEps = 0x1.0c6f7ap-20f;       // float32(1e-6), splax/_project/_kernels.py:215
constexpr float kDilation2 = 0x1.70a3d8p-4f;   // float32(0.3 * 0.3), splax/_project/_project.py:115

// Antialiasing compensation rho = sqrt(clip(1 - eps (a + c) + eps^2 (a c - b^2), 0, 1)),
// splax/_project/_project.py:113-117, in the expression's own evaluation order; rho2 receives the
// unclipped argument. NaN propagates as through the reference's maximum / minimum.
__device__ __forceinline__ float compensation_rho(float a, float b, float c, float& rho2) {
    rho2 = (1.0f - kDilation * (a + c)) + kDilation2 * (a * c - b * b);
    float cl = rho2 < 0.0f ? 0.0f : rho2;
    cl = cl > 1.0f ? 1.0f : cl;
    return sqrtf(cl);
}

// Cotangents of blend_opac = opac * rho(conic) (splax/_render.py:105-109 with
// splax/_project/_project.py:113-117) for a blend-opacity cotangent vbo, by reverse-mode rules of
// the reference's expression: sqrt' = 0.5 / rho, maximum / minimum pass 1 strictly inside, 1/2 at
// a tie and 0 outside. Returns the raw-opacity cotangent and adds the conic cotangent to vc.
// Items without intersections carry vbo = 0 and a zero conic (rho = 1), so the where(radii > 0)
// select adds nothing for them.
__device__ __forceinline__ float compensation_vjp(float vbo, float o, float a, float b, float c,
                                                  float vc[3]) {
    float rho2;
    const float rho = compensation_rho(a, b, c, rho2);
    const float v_o = vbo * rho;
    const float v_rho = vbo * o;
    const float v_cl = v_rho * (0.5f / rho);
    const float m_lo = rho2 > 0.0f ? 1.0f : (rho2 == 0.0f ? 0.5f : 0.0f);
    const float y = rho2 > 0.0f ? rho2 : 0.0f;
    const float m_hi = y < 1.0f ? 1.0f : (y == 1.0f ? 0.5f : 0.0f);
    const float v_r2 = (v_cl * m_hi) * m_lo;
    const float v_s = -(kDilation * v_r2);  // through 1 - eps (a + c)
    const float v_t = kDilation2 * v_r2;    // through eps^2 (a c - b b)
    vc[0] = vc[0] + (v_s + v_t * c);
    vc[1] = vc[1] + (-(v_t * b) - v_t * b);
    vc[2] = vc[2] + (v_s + v_t * a);
    return v_o;
}

// Floats as order-preserving unsigned integers (for min / max reductions) and back.
__device__ __forceinline__ uint32_t f2ord(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(uint32_t u) {
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

__device__ __forceinline__ float minw(float a, float b) { return a < b ? a : b; }
__device__ __forceinline__ float maxw(float a, float b) { return a > b ? a : b; }
__device__ __forceinline__ int32_t iminw(int32_t a, int32_t b) { return a < b ? a : b; }
__device__ __forceinline__ int32_t imaxw(int32_t a, int32_t b) { return a > b ? a : b; }

__device__ __forceinline__ int32_t f2i(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return 2147483647;
    if (f <= -2147483648.0f) return (-2147483647 - 1);
    return (int32_t)f;
}

constexpr float kLn2Hi = 0x1.62ep-1f;      // ln2 with the low 12 mantissa bits cleared
constexpr float kLn2Lo = 0x1.0bfbe8p-15f;  // float32(ln2 - kLn2Hi)
constexpr float kLog2e = 0x1.715476p+0f;

// Natural log for finite x > 0: x = 2^k m, m in (sqrt(2)/2, sqrt(2)], s = (m-1)/(m+1),
// log m = 2 atanh(s) by its series through s^9, log x = k ln2_hi + (k ln2_lo + log m).
__device__ __forceinline__ float det_logf(float x) {
    int32_t k = 0;
    uint32_t ix = __float_as_uint(x);
    if (ix < 0x00800000u) {
        x = x * 0x1p25f;
        k = -25;
        ix = __float_as_uint(x);
    }
    k += (int32_t)(ix >> 23) - 127;
    float m = __uint_as_float((ix & 0x007fffffu) | 0x3f800000u);
    if (m > 0x1.6a09e6p+0f) {
        m = m * 0.5f;
        k += 1;
    }
    float f = m - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    float p = fmaf(z, 0x1.c71c72p-4f, 0x1.24924ap-3f);
    p = fmaf(z, p, 0x1.99999ap-3f);
    p = fmaf(z, p, 0x1.555556p-2f);
    float hs = s + s;
    float lm = fmaf(hs * z, p, hs);
    float kf = (float)k;
    return fmaf(kf, kLn2Hi, fmaf(kf, kLn2Lo, lm));
}

// e^x: k = rint(x log2 e), r = x - k ln2 (two FMAs), degree-7 Taylor polynomial of e^r,
// scaled by 2^k. NaN and x <= -104 give 0.
__device__ __forceinline__ float det_expf(float x) {
    if (!(x > -104.0f)) return 0.0f;
    if (x > 88.75f) return __builtin_inff();
    float kf = rintf(x * kLog2e);
    float r = fmaf(kf, -kLn2Hi, x);
    r = fmaf(kf, -kLn2Lo, r);
    float p = fmaf(r, 0x1.a01a02p-13f, 0x1.6c16c2p-10f);
    p = fmaf(r, p, 0x1.111112p-7f);
    p = fmaf(r, p, 0x1.555556p-5f);
    p = fmaf(r, p, 0x1.555556p-3f);
    p = fmaf(r, p, 0.5f);
    p = fmaf(r, p, 1.0f);
    p = fmaf(r, p, 1.0f);
    return ldexpf(p, (int)kf);
}

// ------------------------------------------------------------------ render_log's parameter map
// splax/_render.py:161-164: scales = exp(log_scales), quats / (|quats| + 1e-8), sigmoid of the
// colour and opacity logits, with sigmoid(x) = 1 / (1 + det_expf(-x)) and
// |q| = sqrt(((q0^2 + q1^2) + q2^2) + q3^2). The reverse-mode rules follow the reference's
// primitives: exp' = exp, logistic' = s (1 - s), sqrt' = 0.5 / sqrt, x / s gives g / s and
// -(g x) / s^2 to the divisor, and the square's two uses add 2 q v.
constexpr float kQuatEps = 0x1.5798eep-27f;  // float32(1e-8), splax/_render.py:162

__device__ __forceinline__ float map_sigmoid(float x) { return 1.0f / (1.0f + det_expf(-x)); }

__device__ __forceinline__ float quat_norm(const float q[4]) {
    return sqrtf(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
}

// Cotangent of a log-scale from its scale's cotangent g.
__device__ __forceinline__ float map_exp_vjp(float g, float log_scale) {
    return g * det_expf(log_scale);
}
// Cotangent of a logit from its sigmoid's cotangent g.
__device__ __forceinline__ float map_sigmoid_vjp(float g, float logit) {
    const float s = map_sigmoid(logit);
    return g * (s * (1.0f - s));
}
// Cotangent of the raw quaternion component k from the normalized quaternion's cotangents vy.
__device__ __forceinline__ float map_quat_vjp(const float q[4], const float vy[4], int k) {
    const float nrm = quat_norm(q);
    const float s = nrm + kQuatEps;
    // y = q / s: the divisor's cotangent sums -(g q) / s^2 over the four components
    const float inv_s2 = 1.0f / (s * s);
    float v_s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) v_s = v_s + (-(vy[j] * q[j])) * inv_s2;
    const float v_ss = v_s * (0.5f / nrm);  // s = sqrt(sum q^2) + eps
    return vy[k] / s + (v_ss * q[k] + v_ss * q[k]);
}

// Opacity-aware isocontour level, splax/_project/_kernels.py:227.
__device__ __forceinline__ float iso_level(float opac) {
    return minw(kExtendSq, 2.0f * det_logf(opac / kAlphaThresh));
}

// Rotation of the xyzw quaternion q: R = (2w^2 - 1) I + 2 v v^T + 2 w [v]_x (warp-lang's
// quat_to_matrix, called at splax/_project/_kernels.py:426,661). Row major.
__device__ __forceinline__ void quat_to_rot(float x, float y, float z, float w, float* R) {
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

__device__ __forceinline__ void mat_mul(const float* a, const float* b, float* c) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            c[3 * i + j] = (a[3 * i] * b[j] + a[3 * i + 1] * b[3 + j]) + a[3 * i + 2] * b[6 + j];
}
__device__ __forceinline__ void mat_mul_tn(const float* a, const float* b, float* c) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            c[3 * i + j] = (a[i] * b[j] + a[3 + i] * b[3 + j]) + a[6 + i] * b[6 + j];
}
__device__ __forceinline__ void mat_mul_nt(const float* a, const float* b, float* c) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            c[3 * i + j] =
                (a[3 * i] * b[3 * j] + a[3 * i + 1] * b[3 * j + 1]) + a[3 * i + 2] * b[3 * j + 2];
}
__device__ __forceinline__ void mat_vec(const float* a, const float* v, float* o) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
        o[i] = (a[3 * i] * v[0] + a[3 * i + 1] * v[1]) + a[3 * i + 2] * v[2];
}
__device__ __forceinline__ void mat_t_vec(const float* a, const float* v, float* o) {
#pragma unroll
    for (int i = 0; i < 3; ++i) o[i] = (a[i] * v[0] + a[3 + i] * v[1]) + a[6 + i] * v[2];
}

// ------------------------------------------------------------------ ellipse tile walk
// splax/_intersect.py:23-183: SNUGBOX tight bbox of A x^2 + 2B xy + C y^2 <= t, then the AccuTile
// column walk over the shorter tile span. Component 0 of the bbox_* / rect_* pairs is the walk's
// outer axis.
struct Ellipse {
    float A, B, C, disc, t, px, py;
    float bmin0, bmin1, bmax0, bmax1, amin1, amax1;
    int32_t rmin0, rmin1, rmax0, rmax1;
    bool valid, isY;
};

__device__ __forceinline__ Ellipse ellipse_init(float A, float B, float C, float t, float px,
                                                float py, int32_t tw, int32_t th) {
    Ellipse s;
    s.valid = false;
    s.isY = false;
    s.A = A;
    s.B = B;
    s.C = C;
    s.t = t;
    s.px = px;
    s.py = py;
    float disc = B * B - A * C;
    s.disc = disc;
    float ntd = -t / disc;
    float x_extent = sqrtf(ntd * C);
    float y_extent = sqrtf(ntd * A);
    float bmin_x = px - x_extent, bmin_y = py - y_extent;
    float bmax_x = px + x_extent, bmax_y = py + y_extent;
    float bx_c = B * x_extent / C;
    float by_a = B * y_extent / A;
    // argmin = (py + bx_c, px + by_a), argmax = (py - bx_c, px - by_a); only the cross-axis
    // component [1] of the (possibly swapped) pair is read by the walk.
    const float ts = (float)kBlockWidth;
    int32_t rminx = imaxw(0, iminw(tw, f2i(bmin_x / ts)));
    int32_t rminy = imaxw(0, iminw(th, f2i(bmin_y / ts)));
    int32_t rmaxx = imaxw(0, iminw(tw, f2i(bmax_x / ts + 1.0f)));
    int32_t rmaxy = imaxw(0, iminw(th, f2i(bmax_y / ts + 1.0f)));
    int32_t x_span = rmaxx - rminx, y_span = rmaxy - rminy;
    s.rmin0 = s.rmin1 = s.rmax0 = s.rmax1 = 0;
    s.bmin0 = s.bmin1 = s.bmax0 = s.bmax1 = s.amin1 = s.amax1 = 0.0f;
    if (y_span * x_span == 0) return s;
    bool isY = y_span < x_span;
    s.isY = isY;
    if (isY) {
        s.rmin0 = rminy; s.rmin1 = rminx; s.rmax0 = rmaxy; s.rmax1 = rmaxx;
        s.bmin0 = bmin_y; s.bmin1 = bmin_x; s.bmax0 = bmax_y; s.bmax1 = bmax_x;
        s.amin1 = py + bx_c; s.amax1 = py - bx_c;
    } else {
        s.rmin0 = rminx; s.rmin1 = rminy; s.rmax0 = rmaxx; s.rmax1 = rmaxy;
        s.bmin0 = bmin_x; s.bmin1 = bmin_y; s.bmax0 = bmax_x; s.bmax1 = bmax_y;
        s.amin1 = px + by_a; s.amax1 = px - by_a;
    }
    s.valid = true;
    return s;
}

// _ellipse_intersect, splax/_intersect.py:110-133
__device__ __forceinline__ void ellipse_intersect(const Ellipse& s, float coord, float& lo,
                                                  float& hi) {
    float p_u = s.isY ? s.py : s.px;
    float p_v = s.isY ? s.px : s.py;
    float coeff = s.isY ? s.A : s.C;
    float h = coord - p_u;
    float sq = sqrtf(s.disc * h * h + s.t * coeff);
    float bh = -s.B * h;
    lo = (bh - sq) / coeff + p_v;
    hi = (bh + sq) / coeff + p_v;
}

// ellipse_init_span, splax/_intersect.py:136-143
__device__ __forceinline__ void ellipse_init_span(const Ellipse& s, float& I0, float& I1) {
    float min_line0 = (float)s.rmin0 * (float)kBlockWidth;
    if (s.bmin0 <= min_line0) {
        ellipse_intersect(s, min_line0, I0, I1);
    } else {
        I0 = s.bmax1;
        I1 = s.bmin1;
    }
}

// ellipse_column_tile_range, splax/_intersect.py:146-169: [min_v, max_v) of outer column u.
__device__ __forceinline__ void ellipse_column(const Ellipse& s, int32_t u, float& I0, float& I1,
                                               int32_t& min_v, int32_t& max_v) {
    const float block = (float)kBlockWidth;
    float min_line = (float)u * block;
    float max_line = min_line + block;
    float J0 = I0, J1 = I1;
    if (max_line <= s.bmax0) ellipse_intersect(s, max_line, J0, J1);
    float emin, emax;
    if (min_line <= s.amin1 && s.amin1 < max_line)
        emin = s.bmin1;
    else
        emin = minw(I0, J0);
    if (min_line <= s.amax1 && s.amax1 < max_line)
        emax = s.bmax1;
    else
        emax = maxw(I1, J1);
    min_v = imaxw(s.rmin1, iminw(s.rmax1, f2i(emin / block)));
    max_v = iminw(s.rmax1, imaxw(s.rmin1, f2i(emax / block + 1.0f)));
    I0 = J0;
    I1 = J1;
}

// ellipse_tile_count, splax/_intersect.py:172-183
__device__ __forceinline__ int32_t ellipse_tile_count(const Ellipse& s) {
    if (!s.valid) return 0;
    float I0, I1;
    ellipse_init_span(s, I0, I1);
    int32_t count = 0;
    for (int32_t u = s.rmin0; u < s.rmax0; ++u) {
        int32_t mn, mx;
        ellipse_column(s, u, I0, I1, mn, mx);
        count += mx - mn;
    }
    return count;
}

// ------------------------------------------------------------------ wave64 helpers

// Sum of v over the 64 lanes of the wave, valid in lane 63 (DPP row shifts within each row of
// 16 lanes, then row broadcasts 15 and 31 across rows).
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_add(float x) {
    int r = __builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, kRowMask, 0xf, false);
    return x + __int_as_float(r);
}

// Must be called with all 64 lanes active.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v = dpp_add<0x111, 0xf>(v);  // row_shr:1
    v = dpp_add<0x112, 0xf>(v);  // row_shr:2
    v = dpp_add<0x114, 0xf>(v);  // row_shr:4
    v = dpp_add<0x118, 0xf>(v);  // row_shr:8
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Minimum (kMax: maximum) of an unsigned value over the 64 lanes, valid in lane 63: the same DPP
// row shifts and row broadcasts, lanes without a source reading the identity.
template <bool kMax, int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_minmax_step(uint32_t x) {
    const uint32_t id = kMax ? 0u : 0xffffffffu;
    const uint32_t y = (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)x, kCtrl, kRowMask, 0xf,
                                                            false);
    return kMax ? (y > x ? y : x) : (y < x ? y : x);
}
template <bool kMax>
__device__ __forceinline__ uint32_t wave_minmax_to_lane63(uint32_t x) {
    x = dpp_minmax_step<kMax, 0x111, 0xf>(x);  // row_shr:1
    x = dpp_minmax_step<kMax, 0x112, 0xf>(x);  // row_shr:2
    x = dpp_minmax_step<kMax, 0x114, 0xf>(x);  // row_shr:4
    x = dpp_minmax_step<kMax, 0x118, 0xf>(x);  // row_shr:8
    x = dpp_minmax_step<kMax, 0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
    x = dpp_minmax_step<kMax, 0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
    return x;
}

// x plus the double of the lane DPP control kCtrl names (0 where it names none), in two 32-bit
// halves.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ double dpp_add_f64(double x) {
    const int64_t b = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, kCtrl, kRowMask, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), kCtrl, kRowMask, 0xf,
                                               false);
    return x + __longlong_as_double((int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
// Sum of a double over the 64 lanes in a fixed order, valid in lane 63 (every lane active).
__device__ __forceinline__ double wave_sum_f64_to_lane63(double x) {
    x = dpp_add_f64<0x111, 0xf>(x);  // row_shr:1
    x = dpp_add_f64<0x112, 0xf>(x);  // row_shr:2
    x = dpp_add_f64<0x114, 0xf>(x);  // row_shr:4
    x = dpp_add_f64<0x118, 0xf>(x);  // row_shr:8
    x = dpp_add_f64<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
    x = dpp_add_f64<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
    return x;
}

__device__ __forceinline__ float lane63(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ------------------------------------------------------------------ packed blend records

// Largest sigma a blend accepts: blend_exp(-87) is still a normal float. An intersection with a
// larger sigma is rejected, as the exact alpha would be for opacities below 2.4e35 (the CPU oracle
// applies the same cap).
constexpr float kBlendSigmaCap = 87.0f;

// Packed record of one geometry item, 64 bytes (one aligned segment per staged intersection):
//   r0 = (x, y, a/2, b), r1 = (c/2, o, sigma_max, 1/a), r2 = (red, green, blue, depth),
//   r3 = (ex, ey, cull mode, dy_r) (1/a and dy_r, the height of the 1.01-scaled ellipse's
//   rightmost point, for the forward's tight sub-block test; 0 unless the cull mode is the box).
// They depend only on the rasterizer's inputs, so a forward's records serve its backward.
// sigma_max = log(255 o) + 1e-3 bounds sigma where o e^-sigma can still reach 1/255. The cull mode
// says whether the tile-independent box (+-ex, +-ey) around the centre holds every pixel centre
// with sigma <= sigma_max (kCullBox), or no pixel can pass (kCullNone: sigma_max < 0), or the box
// cannot be trusted and every quadrant is kept (kCullKeep).
enum : uint32_t { kCullBox = 0u, kCullKeep = 1u, kCullNone = 2u };

// The record of one item from its projection outputs (xy, conic a b c, depth), its raw opacity
// o_raw and colour (3 floats); with compensate the blend opacity is o_raw * rho(conic)
// (splax/_render.py:105-110). Written to r[0..3].
__device__ __forceinline__ void pack_record(float x, float y, float a, float b, float c,
                                            float o_raw, int32_t compensate, const float* color,
                                            float depth, float4* r) {
    float o = o_raw;
    if (compensate) {
        float rho2;
        o = o * compensation_rho(a, b, c, rho2);
    }
    // sigma_max is capped at kBlendSigmaCap, where blend_exp's range ends
    float smax;
    if (o > 0.0f) {
        smax = fminf(__logf(o * 255.0f) + 1e-3f, kBlendSigmaCap);
    } else {
        smax = -__builtin_inff();  // o <= 0 or NaN: no pixel accepts it
    }
    uint32_t mode = kCullKeep;
    float ex = 0.0f, ey = 0.0f, inv_a = 0.0f, dy_r = 0.0f;
    if (!(smax >= 0.0f)) {
        mode = kCullNone;  // every pixel rejected
    } else {
        // Points beyond k times the bounding box of {sigma <= smax} have exact
        // sigma >= k^2 smax. The evaluated sigma differs from the exact one by at most
        // ~6e-7 * cond(Q) relative (Q the conic), so with cond(Q) <= (a + c)^2 / det < 1e4
        // and k = 1.01 every point outside the box evaluates above smax.
        // Worse-conditioned conics keep all four quadrants.
        const float det = a * c - b * b;
        const float tr = a + c;
        const float ex2 = 2.0f * smax * c / det, ey2 = 2.0f * smax * a / det;
        if (a > 0.0f && c > 0.0f && det > 0.0f && tr * tr < 1e4f * det && ex2 < 1e30f &&
            ey2 < 1e30f) {
            // half-widths of the ellipse {sigma <= 1.0201 smax} (the 1.01-scaled one), and the box
            const float sx = sqrtf(ex2) * 1.01f, sy = sqrtf(ey2) * 1.01f;
            ex = sx + 0.01f;
            ey = sy + 0.01f;
            // for the forward's tight sub-block test: 1 / a and the height of the scaled
            // ellipse's rightmost point relative to its centre
            inv_a = 1.0f / a;
            dy_r = -(b * sx) / c;
            mode = kCullBox;
        }
    }
    // the blends evaluate sigma = (a/2 dx dx + c/2 dy dy) + b dx dy: halving exactly before
    // the products leaves every rounding where 0.5 (a dx dx + c dy dy) puts it
    r[0] = make_float4(x, y, 0.5f * a, b);
    r[1] = make_float4(0.5f * c, o, smax, inv_a);
    r[2] = make_float4(color[0], color[1], color[2], depth);
    r[3] = make_float4(ex, ey, __uint_as_float(mode), dy_r);
}

}  // namespace splat
