// Elementwise stages around the render in a training step, each one pass over HBM:
//   - the log / logit parameter map of render_log (splax/_render.py:161-164) and its reverse-mode
//     rule: scales = exp(log_scales), quats / (|quats| + 1e-8), sigmoid of the colour and opacity
//     logits;
//   - the L1 loss mean |img - target| of the trainers (scripts/train_lego.py:111) and its
//     cotangent sign(img - target) * g / count.
//
// The map and its reverse-mode rules are the device functions of splat_common.hpp (map_sigmoid,
// quat_norm, map_*_vjp): exp is det_expf, so the CPU oracle reproduces every bit.
#include <string>

#include "../../include/splat_hip.h"
#include "splat_common.hpp"
#include "splat_internal.hpp"

namespace splat {

struct LogParams {
    const float* log_scales; const float* quats; const float* logit_colors;
    const float* logit_opac;
    int64_t n;
    float* scales; float* quats_out; float* colors; float* opac;              // forward
    const float* v_scales; const float* v_quats; const float* v_colors;       // backward
    const float* v_opac;
    float* v_log_scales; float* v_quats_in; float* v_logit_colors; float* v_logit_opac;
};

// Both map kernels read every input of their item before they store anything: a load placed
// after a store to another array stays behind it (the compiler cannot rule out aliasing), and the
// interleaved form made each item several dependent memory round trips.
__global__ void __launch_bounds__(256) log_params_fwd_kernel(LogParams P) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= P.n) return;
    float ls[3], lc[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        ls[k] = P.log_scales[3 * i + k];
        lc[k] = P.logit_colors[3 * i + k];
    }
    const float4 q4 = reinterpret_cast<const float4*>(P.quats)[i];
    const float lo = P.logit_opac[i];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        P.scales[3 * i + k] = det_expf(ls[k]);
        P.colors[3 * i + k] = map_sigmoid(lc[k]);
    }
    const float q[4] = {q4.x, q4.y, q4.z, q4.w};
    const float s = quat_norm(q) + kQuatEps;
    reinterpret_cast<float4*>(P.quats_out)[i] =
        make_float4(q[0] / s, q[1] / s, q[2] / s, q[3] / s);
    P.opac[i] = map_sigmoid(lo);
}

// A null cotangent is a zero one.
__device__ __forceinline__ float cot(const float* v, int64_t j) { return v ? v[j] : 0.0f; }

__global__ void __launch_bounds__(256) log_params_bwd_kernel(LogParams P) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= P.n) return;
    float vs[3], ls[3], vc[3], lc[3], vy[4];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int64_t j = 3 * i + k;
        vs[k] = cot(P.v_scales, j);
        ls[k] = P.log_scales[j];
        vc[k] = cot(P.v_colors, j);
        lc[k] = P.logit_colors[j];
    }
    const float vo = cot(P.v_opac, i), lo = P.logit_opac[i];
    const float4 q4 = reinterpret_cast<const float4*>(P.quats)[i];
#pragma unroll
    for (int k = 0; k < 4; ++k) vy[k] = cot(P.v_quats, 4 * i + k);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int64_t j = 3 * i + k;
        P.v_log_scales[j] = map_exp_vjp(vs[k], ls[k]);
        P.v_logit_colors[j] = map_sigmoid_vjp(vc[k], lc[k]);
    }
    P.v_logit_opac[i] = map_sigmoid_vjp(vo, lo);
    const float q[4] = {q4.x, q4.y, q4.z, q4.w};
    float vq[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) vq[k] = map_quat_vjp(q, vy, k);
    reinterpret_cast<float4*>(P.v_quats_in)[i] = make_float4(vq[0], vq[1], vq[2], vq[3]);
}

// ------------------------------------------------------------------ L1 and MSE losses

constexpr int kL1Chunk = 4096;  // elements per workgroup (16 per thread)

// Workgroup sums of |img - target| (kSquare: (img - target)^2, exact in double) in double, in a
// fixed order: per thread sequential over its 16 elements, then the wave's 64 sums by DPP row
// shifts and broadcasts into lane 63, then the four waves in order.
template <bool kSquare>
__global__ void __launch_bounds__(256) loss_partials_kernel(const float* img, const float* tgt,
                                                            int64_t count, double* partials) {
    __shared__ double s[4];
    const int64_t base = (int64_t)blockIdx.x * kL1Chunk;
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < kL1Chunk / 256; ++j) {
        const int64_t i = base + j * 256 + threadIdx.x;
        if (i < count) {
            const float d = img[i] - tgt[i];
            acc += kSquare ? (double)d * (double)d : (double)fabsf(d);
        }
    }
    acc = wave_sum_f64_to_lane63(acc);
    if ((threadIdx.x & 63) == 63) s[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) partials[blockIdx.x] = ((s[0] + s[1]) + s[2]) + s[3];
}

// One workgroup: thread t adds partials t, t + 256, t + 512, ... in that order (loads issued
// sixteen at a time; the padding adds +0.0 to a sum of non-negative terms, which changes no bit),
// then a fixed tree over the 256 sums, divided by the count.
constexpr int kFinalLoads = 16;
__global__ void __launch_bounds__(256) l1_final_kernel(const double* partials, int64_t blocks,
                                                       int64_t count, float* loss) {
    __shared__ double s[256];
    double acc = 0.0;
    for (int64_t b0 = threadIdx.x; b0 < blocks; b0 += 256 * kFinalLoads) {
        double v[kFinalLoads];
#pragma unroll
        for (int k = 0; k < kFinalLoads; ++k) {
            const int64_t b = b0 + 256 * k;
            v[k] = b < blocks ? partials[b] : 0.0;
        }
#pragma unroll
        for (int k = 0; k < kFinalLoads; ++k) acc += v[k];
    }
    s[threadIdx.x] = acc;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) s[threadIdx.x] += s[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) *loss = (float)(s[0] / (double)count);
}

// v_img = sign(img - target) * (g / count) (kSquare: 2 (img - target) * (g / count)), g read
// from device memory (the loss cotangent).
template <bool kSquare>
__global__ void __launch_bounds__(256) loss_bwd_kernel(const float* img, const float* tgt,
                                                       int64_t count, const float* g, float* v) {
    const float scale = *g / (float)count;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * 256) {
        const float d = img[i] - tgt[i];
        if (kSquare) {
            v[i] = (d + d) * scale;
        } else {
            const float sg = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : d);  // sign: +-0 and NaN pass
            v[i] = sg * scale;
        }
    }
}

static int glue_launched(const char* what) {
    return hipGetLastError() == hipSuccess ? 0
                                           : fail(kErrLaunch, std::string(what) + " launch failed");
}

template <bool kSquare>
static int loss_fwd(hipStream_t s, const float* img, const float* target, int64_t count,
                    double* partials, float* loss, const char* name) {
    if (count <= 0 || !img || !target || !partials || !loss)
        return fail(kErrArgs, std::string(name) + ": empty input or missing arrays");
    const int64_t blocks = (count + kL1Chunk - 1) / kL1Chunk;
    hipLaunchKernelGGL(loss_partials_kernel<kSquare>, dim3((unsigned)blocks), dim3(256), 0, s,
                       img, target, count, partials);
    int rc = glue_launched(name);
    if (rc) return rc;
    hipLaunchKernelGGL(l1_final_kernel, dim3(1), dim3(256), 0, s, partials, blocks, count, loss);
    return glue_launched(name);
}

template <bool kSquare>
static int loss_bwd(hipStream_t s, const float* img, const float* target, int64_t count,
                    const float* v_loss, float* v_img, const char* name) {
    if (count <= 0 || !img || !target || !v_loss || !v_img)
        return fail(kErrArgs, std::string(name) + ": empty input or missing arrays");
    int64_t blocks = (count + 255) / 256;
    blocks = blocks < 8192 ? blocks : 8192;
    hipLaunchKernelGGL(loss_bwd_kernel<kSquare>, dim3((unsigned)blocks), dim3(256), 0, s, img,
                       target, count, v_loss, v_img);
    return glue_launched(name);
}

int launch_loss_final(const double* partials, int64_t blocks, int64_t count, float* loss,
                      hipStream_t stream) {
    hipLaunchKernelGGL(l1_final_kernel, dim3(1), dim3(256), 0, stream, partials, blocks, count,
                       loss);
    return hipGetLastError() == hipSuccess ? 0 : kErrLaunch;
}

}  // namespace splat

using namespace splat;

extern "C" {

int splat_log_params_fwd(splat_stream_t stream, const float* log_scales, const float* quats,
                         const float* logit_colors, const float* logit_opacities, int64_t n,
                         float* scales, float* quats_out, float* colors, float* opacities) {
    if (n < 0) return fail(kErrArgs, "log_params_fwd: negative count");
    if (n == 0) return 0;
    if (!log_scales || !quats || !logit_colors || !logit_opacities || !scales || !quats_out ||
        !colors || !opacities)
        return fail(kErrArgs, "log_params_fwd: missing arrays");
    if (((uintptr_t)quats | (uintptr_t)quats_out) & 15)
        return fail(kErrArgs, "log_params_fwd: quaternion arrays must be 16-byte aligned");
    LogParams P{};
    P.log_scales = log_scales; P.quats = quats; P.logit_colors = logit_colors;
    P.logit_opac = logit_opacities; P.n = n;
    P.scales = scales; P.quats_out = quats_out; P.colors = colors; P.opac = opacities;
    hipLaunchKernelGGL(log_params_fwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), P);
    return glue_launched("log_params_fwd");
}

int splat_log_params_bwd(splat_stream_t stream, const float* log_scales, const float* quats,
                         const float* logit_colors, const float* logit_opacities, int64_t n,
                         const float* v_scales, const float* v_quats, const float* v_colors,
                         const float* v_opacities, float* v_log_scales, float* v_quats_in,
                         float* v_logit_colors, float* v_logit_opacities) {
    if (n < 0) return fail(kErrArgs, "log_params_bwd: negative count");
    if (n == 0) return 0;
    if (!log_scales || !quats || !logit_colors || !logit_opacities || !v_log_scales ||
        !v_quats_in || !v_logit_colors || !v_logit_opacities)
        return fail(kErrArgs, "log_params_bwd: missing arrays");
    if (((uintptr_t)quats | (uintptr_t)v_quats_in) & 15)
        return fail(kErrArgs, "log_params_bwd: quaternion arrays must be 16-byte aligned");
    LogParams P{};
    P.log_scales = log_scales; P.quats = quats; P.logit_colors = logit_colors;
    P.logit_opac = logit_opacities; P.n = n;
    P.v_scales = v_scales; P.v_quats = v_quats; P.v_colors = v_colors; P.v_opac = v_opacities;
    P.v_log_scales = v_log_scales; P.v_quats_in = v_quats_in;
    P.v_logit_colors = v_logit_colors; P.v_logit_opac = v_logit_opacities;
    hipLaunchKernelGGL(log_params_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), P);
    return glue_launched("log_params_bwd");
}

int splat_l1_loss_fwd(splat_stream_t stream, const float* img, const float* target,
                      int64_t count, double* partials, float* loss) {
    return loss_fwd<false>(static_cast<hipStream_t>(stream), img, target, count, partials, loss,
                           "l1_loss_fwd");
}

int splat_l1_loss_bwd(splat_stream_t stream, const float* img, const float* target,
                      int64_t count, const float* v_loss, float* v_img) {
    return loss_bwd<false>(static_cast<hipStream_t>(stream), img, target, count, v_loss, v_img,
                           "l1_loss_bwd");
}

int splat_mse_loss_fwd(splat_stream_t stream, const float* img, const float* target,
                       int64_t count, double* partials, float* loss) {
    return loss_fwd<true>(static_cast<hipStream_t>(stream), img, target, count, partials, loss,
                          "mse_loss_fwd");
}

int splat_mse_loss_bwd(splat_stream_t stream, const float* img, const float* target,
                       int64_t count, const float* v_loss, float* v_img) {
    return loss_bwd<true>(static_cast<hipStream_t>(stream), img, target, count, v_loss, v_img,
                          "mse_loss_bwd");
}

}  // extern "C"
