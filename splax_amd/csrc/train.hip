// Training-step kernels of the gfx950 splat library:
//   - the fused multi-tensor Adam update, optax 0.2.8 `adam` (scale_by_adam followed by
//     scale_by_learning_rate, then apply_updates) as the trainers configure it per parameter
//     group (scripts/train_lego.py:203-211), and the moment reset of relocated rows
//     (scripts/train_lego.py:136-146);
//   - the fixed-budget MCMC relocation, splax/mcmc.py:29-131, and the trainers' noise on the
//     means, splax/mcmc.py:134-169.
//
// Adam arithmetic per element (float32, no contraction): mu = c1 g + b1 mu; nu = c2 (g g) + b2 nu;
// u = (mu / bc1) / (sqrt(nu / bc2 + eps_root) + eps); p = p + (-lr) u, with c1 = f32(1 - b1),
// c2 = f32(1 - b2) formed in double as Python does for optax's weakly typed constants, and the
// bias corrections bc = f32(1 - b^count) formed in double on the host.
//
// Relocation (splax/mcmc.py:74-131). A gaussian is dead when sigmoid(logit) <= min_opacity, with
// sigmoid(x) = 1 / (1 + det_expf(-x)). Every dead gaussian draws a source among the alive ones
// with probability proportional to opacity (splax/mcmc.py:107-109). The draw is exact and
// reproducible: the weights are the integers opacity * 2^32 (exact for opacities >= 2^-8), their
// inclusive prefix is an order-free uint64 scan, and a dead gaussian i takes 64 bits r from
// Philox4x32-10 (Salmon et al., SC'11) at counter (i, tag) under the caller's 64-bit seed,
// u = floor(r * total / 2^64), and the first index whose prefix exceeds u. The relocation values
// (compute_relocation, splax/mcmc.py:44-71, after gsplat's relocation kernel) are evaluated in
// double with exact binomial coefficients and rounded to float32 once.
#include <mutex>
#include <string>

#include "../../include/splat_hip.h"
#include "splat_common.hpp"
#include "splat_internal.hpp"

namespace splat {

// ------------------------------------------------------------------ Adam

constexpr int kAdamMaxGroups = 8;
constexpr int kAdamChunk = 1024;  // elements per workgroup (4 per thread)

struct AdamGroupDev {
    float* p; const float* g; float* mu; float* nu;
    int64_t size;
    float neg_lr;
    int32_t map;  // SPLAT_MAP_*: g is the cotangent of the group's mapped value
};

struct AdamParams {
    AdamGroupDev grp[kAdamMaxGroups];
    int64_t block_start[kAdamMaxGroups + 1];  // first workgroup of each group
    int n_groups;
    float b1, c1, b2, c2, eps, eps_root, bc1, bc2;
};

// The update of one workgroup's chunk of group G, with kMap the group's parameter map. Every
// load of the chunk is issued before any update (restrict-qualified pointers: the compiler
// would otherwise keep each element's loads behind the previous element's stores), so a thread
// has its four elements' reads in flight together. The gradient of the stored parameter is the
// reverse-mode rule of render_log's map applied to the mapped value's cotangent
// (log_params_bwd_kernel's float operations), at the parameter before this update.
template <int kMap>
__device__ __forceinline__ void adam_chunk(const AdamParams& P, const AdamGroupDev& G,
                                           int64_t base) {
    constexpr int K = kAdamChunk / 256;
    float* __restrict__ pp = G.p;
    const float* __restrict__ gp = G.g;
    float* __restrict__ mp = G.mu;
    float* __restrict__ np = G.nu;
    const int64_t i0 = base + threadIdx.x;
    float g[K], pv[K], m[K], v[K];
    float q[K][4], vy[K][4];  // kMap == SPLAT_MAP_QUAT: the element's row of the group [rows, 4]
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const int64_t i = i0 + j * 256;
        if (i < G.size) {
            if constexpr (kMap == SPLAT_MAP_QUAT) {
                const int64_t row = i >> 2;  // the group is 16-byte aligned
                const float4 q4 = reinterpret_cast<const float4*>(pp)[row];
                const float4 v4 = reinterpret_cast<const float4*>(gp)[row];
                q[j][0] = q4.x; q[j][1] = q4.y; q[j][2] = q4.z; q[j][3] = q4.w;
                vy[j][0] = v4.x; vy[j][1] = v4.y; vy[j][2] = v4.z; vy[j][3] = v4.w;
            } else {
                g[j] = gp[i];
                pv[j] = pp[i];
            }
            m[j] = mp[i];
            v[j] = np[i];
        }
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const int64_t i = i0 + j * 256;
        if (i >= G.size) break;
        float gg, p0;
        if constexpr (kMap == SPLAT_MAP_QUAT) {
            const int c = (int)(i & 3);
            // whole-row copies, indexed by the component (a dynamic index into q[j] itself
            // would put the arrays in scratch memory)
            const float qa[4] = {q[j][0], q[j][1], q[j][2], q[j][3]};
            const float va[4] = {vy[j][0], vy[j][1], vy[j][2], vy[j][3]};
            gg = map_quat_vjp(qa, va, c);
            p0 = c == 0 ? qa[0] : c == 1 ? qa[1] : c == 2 ? qa[2] : qa[3];
        } else if constexpr (kMap == SPLAT_MAP_EXP) {
            gg = map_exp_vjp(g[j], pv[j]);
            p0 = pv[j];
        } else if constexpr (kMap == SPLAT_MAP_SIGMOID) {
            gg = map_sigmoid_vjp(g[j], pv[j]);
            p0 = pv[j];
        } else {
            gg = g[j];
            p0 = pv[j];
        }
        const float mm = P.c1 * gg + P.b1 * m[j];
        const float vv = P.c2 * (gg * gg) + P.b2 * v[j];
        const float mh = mm / P.bc1;
        const float vh = vv / P.bc2;
        const float u = mh / (sqrtf(vh + P.eps_root) + P.eps);
        mp[i] = mm;
        np[i] = vv;
        pp[i] = p0 + G.neg_lr * u;
    }
}

__global__ void __launch_bounds__(256) adam_step_kernel(AdamParams P) {
    const int64_t b = blockIdx.x;
    int gi = 0;
    while (gi + 1 < P.n_groups && b >= P.block_start[gi + 1]) ++gi;  // uniform per workgroup
    const AdamGroupDev G = P.grp[gi];
    const int64_t base = (b - P.block_start[gi]) * kAdamChunk;
    switch (G.map) {  // uniform per workgroup
    case SPLAT_MAP_EXP: adam_chunk<SPLAT_MAP_EXP>(P, G, base); break;
    case SPLAT_MAP_SIGMOID: adam_chunk<SPLAT_MAP_SIGMOID>(P, G, base); break;
    case SPLAT_MAP_QUAT: adam_chunk<SPLAT_MAP_QUAT>(P, G, base); break;
    default: adam_chunk<SPLAT_MAP_NONE>(P, G, base); break;
    }
}

struct ResetParams {
    float* mu[kAdamMaxGroups];
    float* nu[kAdamMaxGroups];
    int32_t width[kAdamMaxGroups];
    int n_groups;
    const uint8_t* reset;
    int64_t rows;
};

__global__ void __launch_bounds__(256) adam_reset_rows_kernel(ResetParams P) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= P.rows || !P.reset[r]) return;
    // x * keep, as the reference does: a negative moment becomes -0 and NaN stays NaN
    for (int g = 0; g < P.n_groups; ++g) {
        const int32_t w = P.width[g];
        for (int k = 0; k < w; ++k) {
            P.mu[g][r * w + k] = P.mu[g][r * w + k] * 0.0f;
            P.nu[g][r * w + k] = P.nu[g][r * w + k] * 0.0f;
        }
    }
}

// ------------------------------------------------------------------ Philox4x32-10

constexpr uint32_t kPhiloxM0 = 0xD2511F53u, kPhiloxM1 = 0xCD9E8D57u;
constexpr uint32_t kPhiloxW0 = 0x9E3779B9u, kPhiloxW1 = 0xBB67AE85u;
constexpr uint32_t kRelocateTag = 0x4d434d43u;  // counter word 2 of the relocation draws

__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r > 0) {
            k0 += kPhiloxW0;
            k1 += kPhiloxW1;
        }
        const uint64_t p0 = (uint64_t)kPhiloxM0 * c[0];
        const uint64_t p1 = (uint64_t)kPhiloxM1 * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c[0] = n0; c[1] = n1; c[2] = n2; c[3] = n3;
    }
}

// ------------------------------------------------------------------ noise injection
// inject_noise, splax/mcmc.py:134-169: means + Sigma (z sigmoid(100 (min_opacity - o)) scaler),
// Sigma = M M^T with M = R diag(exp(log_scales)), R the rotation of the normalized wxyz
// quaternion (scipy's from_quat normalizes), o = sigmoid(logit) and z three standard normals
// per gaussian: from the caller (noise) or drawn here by Box-Muller on the four words of
// Philox4x32-10 at counter (i, tag) under the caller's seed, each word's top 23 bits giving a
// uniform (k + 1/2) 2^-23 in [2^-24, 1 - 2^-24] (k + 1/2 fits float32's 24-bit significand, so u
// is exact and |z| <= sqrt(48 ln 2) < 5.8). Float32 throughout; the reference draws its normals with
// jax.random.normal, so the distribution is the reference's and the stream the library's.
constexpr uint32_t kNoiseTag = 0x4e4f4953u;  // counter word 2 of the noise draws

struct NoiseParams {
    const float* means; const float* log_scales; const float* quats; const float* logit_opac;
    const float* noise;  // [n, 3] standard normals, or null to draw them
    float* out;
    int64_t n;
    float scaler, min_opacity;
    uint32_t seed_lo, seed_hi;
};

__global__ void __launch_bounds__(256) inject_noise_kernel(NoiseParams P) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= P.n) return;
    float z[3];
    if (P.noise) {
        z[0] = P.noise[3 * i];
        z[1] = P.noise[3 * i + 1];
        z[2] = P.noise[3 * i + 2];
    } else {
        uint32_t c[4] = {(uint32_t)i, (uint32_t)((uint64_t)i >> 32), kNoiseTag, 0u};
        philox4x32_10(c, P.seed_lo, P.seed_hi);
        float u[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) u[k] = ((float)(c[k] >> 9) + 0.5f) * 0x1p-23f;
        const float r0 = sqrtf(-2.0f * logf(u[0])), r1 = sqrtf(-2.0f * logf(u[2]));
        const float t0 = 6.28318530717958647692f * u[1], t1 = 6.28318530717958647692f * u[3];
        z[0] = r0 * cosf(t0);
        z[1] = r0 * sinf(t0);
        z[2] = r1 * cosf(t1);
    }
    const float o = 1.0f / (1.0f + expf(-P.logit_opac[i]));
    const float gate = 1.0f / (1.0f + expf(-(100.0f * (P.min_opacity - o))));
    const float a = gate * P.scaler;
    const float w[3] = {z[0] * a, z[1] * a, z[2] * a};
    const float* q = P.quats + 4 * i;
    const float qn = sqrtf(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
    const float qw = q[0] / qn, qx = q[1] / qn, qy = q[2] / qn, qz = q[3] / qn;
    const float R[9] = {1.0f - 2.0f * (qy * qy + qz * qz), 2.0f * (qx * qy - qw * qz),
                        2.0f * (qx * qz + qw * qy),        2.0f * (qx * qy + qw * qz),
                        1.0f - 2.0f * (qx * qx + qz * qz), 2.0f * (qy * qz - qw * qx),
                        2.0f * (qx * qz - qw * qy),        2.0f * (qy * qz + qw * qx),
                        1.0f - 2.0f * (qx * qx + qy * qy)};
    float s[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = expf(P.log_scales[3 * i + k]);
    // Sigma w = M (M^T w): t = diag(s) R^T w, then R diag(s) t
    float t[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) t[k] = s[k] * ((R[k] * w[0] + R[3 + k] * w[1]) + R[6 + k] * w[2]);
#pragma unroll
    for (int k = 0; k < 3; ++k) t[k] = s[k] * t[k];
#pragma unroll
    for (int r = 0; r < 3; ++r)
        P.out[3 * i + r] = P.means[3 * i + r] + ((R[3 * r] * t[0] + R[3 * r + 1] * t[1]) +
                                                 R[3 * r + 2] * t[2]);
}

// ------------------------------------------------------------------ relocation

constexpr int kRelocChunk = 4096;  // weights per workgroup of the scan (16 per thread)
constexpr int kMaxBinomRows = 62;  // C(r, k) * (r - k) stays below 2^64 for r <= 62

__device__ __forceinline__ float reloc_sigmoid(float x) { return 1.0f / (1.0f + det_expf(-x)); }

// splax/mcmc.py:104 (sigmoid never yields NaN here: det_expf maps NaN to 0).
__device__ __forceinline__ bool reloc_dead(float logit, float min_opacity) {
    return reloc_sigmoid(logit) <= min_opacity;
}

__device__ __forceinline__ uint64_t reloc_weight(float logit, float min_opacity) {
    const float o = reloc_sigmoid(logit);
    if (o <= min_opacity) return 0ull;
    return (uint64_t)(o * 0x1p32f);
}

// compute_relocation for one row (splax/mcmc.py:44-71): new opacity 1 - (1 - o)^(1/r) and the
// scale factor o / sum_{k<r} C(r, k+1) (-1)^k (k+1)^(-1/2) new^(k+1). The reference's
// cumsum(binoms)[r-1, k] equals C(r, k+1).
__device__ __forceinline__ void relocation_values(double o, int r, double& no, double& coeff) {
    no = 1.0 - pow(1.0 - o, 1.0 / (double)r);
    double denom = 0.0, pw = 1.0;
    uint64_t binom = 1;  // C(r, k) before the update, C(r, k+1) after
    for (int k = 0; k < r; ++k) {
        binom = binom * (uint64_t)(r - k) / (uint64_t)(k + 1);
        pw = pw * no;
        const double term = (double)binom * pw / sqrt((double)(k + 1));
        denom = (k & 1) ? denom - term : denom + term;
    }
    coeff = o / denom;
}

struct RelocParams {
    float* means; float* log_scales; float* quats; float* colors; float* logit_opac;
    int64_t n;
    int32_t n_max;
    float min_opacity;
    uint32_t seed_lo, seed_hi;
    uint64_t* cdf;       // [n] inclusive prefix of the weights
    uint64_t* partials;  // [blocks + 1] exclusive prefix per scan workgroup, then the total
    int32_t* counts;     // [n] dead gaussians that drew each source
    int32_t* src;        // [n] dead: drawn source; alive: itself
    float4* newv;        // [n] (logit, log_scale x3) of rows with counts > 0
    int32_t* source_out; // optional [n]
    uint8_t* reset_out;  // optional [n]
    int64_t blocks;
};

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* s_wave) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) s_wave[wave] = v;
    __syncthreads();
    const uint64_t t = s_wave[0] + s_wave[1] + s_wave[2] + s_wave[3];
    __syncthreads();
    return t;
}

// Workgroup sums of the weights; also clears the draw counts of the chunk.
__global__ void __launch_bounds__(256) reloc_partials_kernel(RelocParams P) {
    __shared__ uint64_t s_wave[4];
    const int64_t base = (int64_t)blockIdx.x * kRelocChunk;
    uint64_t acc = 0;
#pragma unroll
    for (int j = 0; j < kRelocChunk / 256; ++j) {
        const int64_t i = base + j * 256 + threadIdx.x;
        if (i < P.n) {
            acc += reloc_weight(P.logit_opac[i], P.min_opacity);
            P.counts[i] = 0;
        }
    }
    const uint64_t t = block_sum_u64(acc, s_wave);
    if (threadIdx.x == 0) P.partials[blockIdx.x] = t;
}

// One workgroup: exclusive scan of the workgroup sums, total in partials[blocks].
__global__ void __launch_bounds__(256) reloc_scan_partials_kernel(RelocParams P) {
    __shared__ uint64_t s[256];
    uint64_t carry = 0;
    for (int64_t c0 = 0; c0 < P.blocks; c0 += 256) {
        const int64_t i = c0 + threadIdx.x;
        const uint64_t v = i < P.blocks ? P.partials[i] : 0ull;
        s[threadIdx.x] = v;
        __syncthreads();
        for (int off = 1; off < 256; off <<= 1) {  // Hillis-Steele inclusive scan
            const uint64_t add = threadIdx.x >= (unsigned)off ? s[threadIdx.x - off] : 0ull;
            __syncthreads();
            s[threadIdx.x] += add;
            __syncthreads();
        }
        if (i < P.blocks) P.partials[i] = carry + s[threadIdx.x] - v;
        carry += s[255];
        __syncthreads();
    }
    if (threadIdx.x == 0) P.partials[P.blocks] = carry;
}

// Inclusive prefix of the weights: each thread owns 16 consecutive weights. The weights are
// computed from coalesced loads (thread t takes elements t, t + 256, ...) into LDS, where each
// thread then reads its own 16 (rows padded by one word against bank conflicts), and the prefixes
// leave the same way, so every global access is coalesced (config 4's relocation 0.066 -> 0.054
// ms against per-thread runs read and written directly).
constexpr int kCdfPad = 17;  // LDS words per thread row: 16 weights + 1 pad
__global__ void __launch_bounds__(256) reloc_cdf_kernel(RelocParams P) {
    __shared__ uint64_t s_w[256 * kCdfPad];
    __shared__ uint64_t s_wave[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t base = (int64_t)blockIdx.x * kRelocChunk;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int e = j * 256 + tid;  // element of the chunk
        const int64_t i = base + e;
        const uint64_t w = i < P.n ? reloc_weight(P.logit_opac[i], P.min_opacity) : 0ull;
        s_w[(e >> 4) * kCdfPad + (e & 15)] = w;
    }
    __syncthreads();
    uint64_t own = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) own += s_w[tid * kCdfPad + k];
    // exclusive prefix of `own` over the workgroup: wave scan by shuffles, then the waves before
    uint64_t incl = own;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t up = __shfl_up(incl, off, 64);
        if (lane >= off) incl += up;
    }
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    uint64_t run = P.partials[blockIdx.x] + incl - own;
#pragma unroll
    for (int w = 0; w < 4; ++w) run += w < wave ? s_wave[w] : 0ull;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        run += s_w[tid * kCdfPad + k];
        s_w[tid * kCdfPad + k] = run;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int e = j * 256 + tid;
        const int64_t i = base + e;
        if (i < P.n) P.cdf[i] = s_w[(e >> 4) * kCdfPad + (e & 15)];
    }
}

// Draws the source of every dead gaussian (splax/mcmc.py:107-111) and counts the draws.
__global__ void __launch_bounds__(256) reloc_sample_kernel(RelocParams P) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= P.n) return;
    if (!reloc_dead(P.logit_opac[i], P.min_opacity)) {
        P.src[i] = (int32_t)i;
        return;
    }
    const uint64_t total = P.partials[P.blocks];
    int64_t s = 0;  // nothing alive: every logit is -inf and the reference's argmax gives 0
    if (total > 0) {
        uint32_t c[4] = {(uint32_t)i, (uint32_t)((uint64_t)i >> 32), kRelocateTag, 0u};
        philox4x32_10(c, P.seed_lo, P.seed_hi);
        const uint64_t r = ((uint64_t)c[0] << 32) | c[1];
        const uint64_t u = __umul64hi(r, total);
        int64_t lo = 0, hi = P.n - 1;  // first index with cdf > u; cdf[n-1] = total > u
        while (lo < hi) {
            const int64_t mid = (lo + hi) >> 1;
            if (P.cdf[mid] > u) hi = mid; else lo = mid + 1;
        }
        s = lo;
    }
    P.src[i] = (int32_t)s;
    atomicAdd(&P.counts[s], 1);
}

// New (logit, log scales) of every drawn source, from its unmodified row.
__global__ void __launch_bounds__(256) reloc_values_kernel(RelocParams P) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= P.n) return;
    const int32_t cnt = P.counts[i];
    if (cnt <= 0) return;
    const int r = cnt + 1 < P.n_max ? cnt + 1 : P.n_max;  // ratio, clipped to [1, n_max]
    const double o = (double)reloc_sigmoid(P.logit_opac[i]);
    double no, coeff;
    relocation_values(o, r, no, coeff);
    const double lo_clip = (double)P.min_opacity, hi_clip = 1.0 - 0x1p-23;
    no = no < lo_clip ? lo_clip : no;
    no = no > hi_clip ? hi_clip : no;
    float4 v;
    v.x = (float)log(no / (1.0 - no));
    v.y = (float)log(coeff * (double)det_expf(P.log_scales[3 * i]));
    v.z = (float)log(coeff * (double)det_expf(P.log_scales[3 * i + 1]));
    v.w = (float)log(coeff * (double)det_expf(P.log_scales[3 * i + 2]));
    P.newv[i] = v;
}

// Writes the relocated rows (splax/mcmc.py:119-131). Dead rows copy mean, quaternion and colour
// of their source, which is alive and keeps those, and take the source's new values.
__global__ void __launch_bounds__(256) reloc_apply_kernel(RelocParams P) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= P.n) return;
    const int32_t s = P.src[i];
    const bool dead = reloc_dead(P.logit_opac[i], P.min_opacity);  // own row, read before writing
    const bool reset = dead || P.counts[i] > 0;
    if (dead) {
        const float m0 = P.means[3 * s], m1 = P.means[3 * s + 1], m2 = P.means[3 * s + 2];
        const float q0 = P.quats[4 * s], q1 = P.quats[4 * s + 1], q2 = P.quats[4 * s + 2],
                    q3 = P.quats[4 * s + 3];
        const float c0 = P.colors[3 * s], c1 = P.colors[3 * s + 1], c2 = P.colors[3 * s + 2];
        P.means[3 * i] = m0; P.means[3 * i + 1] = m1; P.means[3 * i + 2] = m2;
        P.quats[4 * i] = q0; P.quats[4 * i + 1] = q1; P.quats[4 * i + 2] = q2;
        P.quats[4 * i + 3] = q3;
        P.colors[3 * i] = c0; P.colors[3 * i + 1] = c1; P.colors[3 * i + 2] = c2;
    }
    if (reset) {
        const float4 v = P.newv[dead ? s : (int32_t)i];
        P.logit_opac[i] = v.x;
        P.log_scales[3 * i] = v.y;
        P.log_scales[3 * i + 1] = v.z;
        P.log_scales[3 * i + 2] = v.w;
    }
    if (P.source_out) P.source_out[i] = s;
    if (P.reset_out) P.reset_out[i] = reset ? 1 : 0;
}

struct ComputeRelocParams {
    const float* opac; const float* scales; const float* ratios;
    int64_t n;
    int32_t n_max;
    float* new_opac; float* new_scales;
};

// compute_relocation alone (splax/mcmc.py:44-71): ratio rounded and clipped to [1, n_max].
__global__ void __launch_bounds__(256) compute_relocation_kernel(ComputeRelocParams P) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= P.n) return;
    const float rf = rintf(P.ratios[i]);
    int r = rf >= (float)P.n_max ? P.n_max : (rf >= 1.0f ? (int)rf : 1);
    double no, coeff;
    relocation_values((double)P.opac[i], r, no, coeff);
    P.new_opac[i] = (float)no;
    for (int k = 0; k < 3; ++k) P.new_scales[3 * i + k] = (float)(coeff * (double)P.scales[3 * i + k]);
}

// ------------------------------------------------------------------ scratch

struct RelocScratch {
    std::mutex mu;
    int64_t cap = 0;
    uint64_t* cdf = nullptr;
    uint64_t* partials = nullptr;
    int32_t* counts = nullptr;
    int32_t* src = nullptr;
    float4* newv = nullptr;

    void release() {
        if (cap) (void)hipDeviceSynchronize();
        (void)hipFree(cdf); (void)hipFree(partials); (void)hipFree(counts);
        (void)hipFree(src); (void)hipFree(newv);
        cdf = nullptr; partials = nullptr; counts = nullptr; src = nullptr; newv = nullptr;
        cap = 0;
    }
    int ensure(int64_t n) {
        if (n <= cap) return 0;
        release();
        const int64_t c = (int64_t)(n * 1.25) + 1;
        const int64_t nb = (c + kRelocChunk - 1) / kRelocChunk + 1;
        if (hipMalloc((void**)&cdf, c * sizeof(uint64_t)) != hipSuccess ||
            hipMalloc((void**)&partials, nb * sizeof(uint64_t)) != hipSuccess ||
            hipMalloc((void**)&counts, c * sizeof(int32_t)) != hipSuccess ||
            hipMalloc((void**)&src, c * sizeof(int32_t)) != hipSuccess ||
            hipMalloc((void**)&newv, c * sizeof(float4)) != hipSuccess) {
            release();
            return fail(kErrAlloc, "relocate: scratch allocation failed");
        }
        cap = c;
        return 0;
    }
};

constexpr int kRelocMaxDevices = 64;
static RelocScratch g_reloc[kRelocMaxDevices];

void release_train_scratch() {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return;
    for (int d = 0; d < kRelocMaxDevices; ++d) {
        std::lock_guard<std::mutex> lock(g_reloc[d].mu);
        if (!g_reloc[d].cap) continue;
        if (hipSetDevice(d) != hipSuccess) continue;
        g_reloc[d].release();
    }
    (void)hipSetDevice(cur);
}

static unsigned grid_for(int64_t n, int64_t per) { return (unsigned)((n + per - 1) / per); }

static int launched(const char* what) {
    return hipGetLastError() == hipSuccess ? 0 : fail(kErrLaunch, std::string(what) + " launch failed");
}

}  // namespace splat

using namespace splat;

extern "C" {

int splat_adam_step(splat_stream_t stream, const splat_adam_group* groups, int32_t num_groups,
                    double b1, double b2, double eps, double eps_root, int64_t count) {
    return splat_adam_step_mapped(stream, groups, num_groups, nullptr, b1, b2, eps, eps_root,
                                  count);
}

int splat_adam_step_mapped(splat_stream_t stream, const splat_adam_group* groups,
                           int32_t num_groups, const int32_t* maps, double b1, double b2,
                           double eps, double eps_root, int64_t count) {
    if (num_groups < 0 || num_groups > kAdamMaxGroups || (num_groups > 0 && !groups))
        return fail(kErrArgs, "adam_step: between 0 and 8 parameter groups");
    if (count < 1) return fail(kErrArgs, "adam_step: count (the incremented step) must be >= 1");
    AdamParams P;
    P.n_groups = num_groups;
    int64_t blocks = 0;
    for (int g = 0; g < num_groups; ++g) {
        const splat_adam_group& s = groups[g];
        if (s.size < 0 || (s.size > 0 && (!s.params || !s.grads || !s.mu || !s.nu)))
            return fail(kErrArgs, "adam_step: group " + std::to_string(g) + " has no buffers");
        const int32_t map = maps ? maps[g] : SPLAT_MAP_NONE;
        if (map < SPLAT_MAP_NONE || map > SPLAT_MAP_QUAT)
            return fail(kErrArgs, "adam_step: group " + std::to_string(g) +
                                      " has an unknown parameter map");
        if (map == SPLAT_MAP_QUAT &&
            (s.size % 4 != 0 || (((uintptr_t)s.params | (uintptr_t)s.grads) & 15)))
            return fail(kErrArgs, "adam_step: a quaternion group holds rows of 4 floats, "
                                  "16-byte aligned");
        P.grp[g] = AdamGroupDev{s.params, s.grads, s.mu, s.nu, s.size, (float)(-s.lr), map};
        P.block_start[g] = blocks;
        blocks += (s.size + kAdamChunk - 1) / kAdamChunk;
    }
    P.block_start[num_groups] = blocks;
    P.b1 = (float)b1;
    P.c1 = (float)(1.0 - b1);
    P.b2 = (float)b2;
    P.c2 = (float)(1.0 - b2);
    P.eps = (float)eps;
    P.eps_root = (float)eps_root;
    P.bc1 = (float)(1.0 - pow(b1, (double)count));
    P.bc2 = (float)(1.0 - pow(b2, (double)count));
    if (blocks == 0) return 0;
    if (blocks > 0x7fffffff) return fail(kErrArgs, "adam_step: too many elements");
    hipLaunchKernelGGL(adam_step_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), P);
    return launched("adam_step");
}

int splat_adam_reset_rows(splat_stream_t stream, const splat_adam_group* groups,
                          int32_t num_groups, const uint8_t* reset, int64_t num_rows) {
    if (num_groups < 0 || num_groups > kAdamMaxGroups || (num_groups > 0 && !groups))
        return fail(kErrArgs, "adam_reset_rows: between 0 and 8 parameter groups");
    if (num_rows < 0 || (num_rows > 0 && !reset))
        return fail(kErrArgs, "adam_reset_rows: missing reset mask");
    ResetParams P;
    P.n_groups = num_groups;
    P.reset = reset;
    P.rows = num_rows;
    for (int g = 0; g < num_groups; ++g) {
        const splat_adam_group& s = groups[g];
        if (num_rows == 0) break;
        if (s.size % num_rows != 0 || (s.size > 0 && (!s.mu || !s.nu)))
            return fail(kErrArgs, "adam_reset_rows: group " + std::to_string(g) +
                                      " is not a whole number of rows");
        P.mu[g] = s.mu;
        P.nu[g] = s.nu;
        P.width[g] = (int32_t)(s.size / num_rows);
    }
    if (num_rows == 0 || num_groups == 0) return 0;
    hipLaunchKernelGGL(adam_reset_rows_kernel, dim3(grid_for(num_rows, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), P);
    return launched("adam_reset_rows");
}

int splat_mcmc_relocate(splat_stream_t stream, float* means3d, float* log_scales, float* quats,
                        float* logit_colors, float* logit_opacities, int64_t num_gaussians,
                        int32_t n_max, float min_opacity, uint64_t seed, int32_t* source,
                        uint8_t* reset) {
    if (num_gaussians < 0 || num_gaussians > 0x7fffffff)
        return fail(kErrArgs, "relocate: gaussian count outside [0, 2^31)");
    if (n_max < 1 || n_max > kMaxBinomRows)
        return fail(kErrArgs, "relocate: binomial table size must be in [1, 62]");
    if (num_gaussians == 0) return 0;
    if (!means3d || !log_scales || !quats || !logit_colors || !logit_opacities)
        return fail(kErrArgs, "relocate: missing parameter arrays");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kRelocMaxDevices)
        return fail(kErrRuntime, "relocate: no current device");
    RelocScratch& sc = g_reloc[dev];
    std::lock_guard<std::mutex> lock(sc.mu);
    int rc = sc.ensure(num_gaussians);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    RelocParams P;
    P.means = means3d; P.log_scales = log_scales; P.quats = quats; P.colors = logit_colors;
    P.logit_opac = logit_opacities;
    P.n = num_gaussians;
    P.n_max = n_max;
    P.min_opacity = min_opacity;
    P.seed_lo = (uint32_t)seed;
    P.seed_hi = (uint32_t)(seed >> 32);
    P.cdf = sc.cdf; P.partials = sc.partials; P.counts = sc.counts; P.src = sc.src;
    P.newv = sc.newv;
    P.source_out = source;
    P.reset_out = reset;
    P.blocks = (num_gaussians + kRelocChunk - 1) / kRelocChunk;
    const unsigned rows = grid_for(num_gaussians, 256);
    hipLaunchKernelGGL(reloc_partials_kernel, dim3((unsigned)P.blocks), dim3(256), 0, s, P);
    if ((rc = launched("relocate partials"))) return rc;
    hipLaunchKernelGGL(reloc_scan_partials_kernel, dim3(1), dim3(256), 0, s, P);
    if ((rc = launched("relocate scan"))) return rc;
    hipLaunchKernelGGL(reloc_cdf_kernel, dim3((unsigned)P.blocks), dim3(256), 0, s, P);
    if ((rc = launched("relocate cdf"))) return rc;
    hipLaunchKernelGGL(reloc_sample_kernel, dim3(rows), dim3(256), 0, s, P);
    if ((rc = launched("relocate sample"))) return rc;
    hipLaunchKernelGGL(reloc_values_kernel, dim3(rows), dim3(256), 0, s, P);
    if ((rc = launched("relocate values"))) return rc;
    hipLaunchKernelGGL(reloc_apply_kernel, dim3(rows), dim3(256), 0, s, P);
    return launched("relocate apply");
}

int splat_mcmc_inject_noise(splat_stream_t stream, const float* means3d, const float* log_scales,
                            const float* quats, const float* logit_opacities,
                            int64_t num_gaussians, float scaler, float min_opacity,
                            uint64_t seed, const float* noise, float* out_means) {
    if (num_gaussians < 0) return fail(kErrArgs, "inject_noise: negative count");
    if (num_gaussians == 0) return 0;
    if (!means3d || !log_scales || !quats || !logit_opacities || !out_means)
        return fail(kErrArgs, "inject_noise: missing arrays");
    NoiseParams P{means3d, log_scales, quats, logit_opacities, noise, out_means,
                  num_gaussians, scaler, min_opacity, (uint32_t)seed, (uint32_t)(seed >> 32)};
    hipLaunchKernelGGL(inject_noise_kernel, dim3(grid_for(num_gaussians, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), P);
    return launched("inject_noise");
}

int splat_mcmc_compute_relocation(splat_stream_t stream, const float* opacities,
                                  const float* scales, const float* ratios, int64_t n,
                                  int32_t n_max, float* new_opacities, float* new_scales) {
    if (n < 0) return fail(kErrArgs, "compute_relocation: negative count");
    if (n_max < 1 || n_max > kMaxBinomRows)
        return fail(kErrArgs, "compute_relocation: binomial table size must be in [1, 62]");
    if (n == 0) return 0;
    if (!opacities || !scales || !ratios || !new_opacities || !new_scales)
        return fail(kErrArgs, "compute_relocation: missing arrays");
    ComputeRelocParams P{opacities, scales, ratios, n, n_max, new_opacities, new_scales};
    hipLaunchKernelGGL(compute_relocation_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), P);
    return launched("compute_relocation");
}

}  // extern "C"
