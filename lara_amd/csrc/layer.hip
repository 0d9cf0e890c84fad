// Layer input stage of run_layer (sw/attn_driver.py:552-576): the host RMSNorm, RoPE and
// head reshaping that the reference does in numpy before each attention transaction, here
// as two small HBM-bound kernels around the QKV projection GEMM.
//
// rms_norm_kernel: y = x / sqrt(mean(x^2) + eps) * gamma per token row
//   (hw/rtl/ext/rms_norm/rms_norm.sv:7-8, 42-45: sum of squares, inverse square root, two
//   products), sums and products in fp32, one RNE rounding to bf16.
// rope_scatter_kernel: rotation of each (2p, 2p+1) pair of a Q or K head by
//   pos * theta[p] (hw/rtl/core/rope_engine.sv:4-10, 135-155: phase = fp32(pos * theta), then
//   a*cos - b*sin and a*sin + b*cos, each product and sum rounded to fp32), cos/sin of the
//   fp32 phase evaluated in double and rounded to fp32, output rounded to bf16 (RNE).  Q is
//   written head-major [H_q][n_tokens][D] (reshape_to_heads), K and V rows go straight into
//   the sequence's cache rows.
#include "gqa_internal.h"

namespace lara {
namespace {

__device__ __forceinline__ float bf16_to_f32(uint32_t w) { return __uint_as_float(w << 16); }

constexpr int kNormThreads = 256;

// One work-group per token row; 8 bf16 (16 bytes) per thread and step when hidden % 8 == 0.
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(NormArgs a) {
    const int row = blockIdx.x;
    const uint16_t* x = a.x + (size_t)row * a.hidden;
    uint16_t* y = a.y + (size_t)row * a.hidden;
    const bool vec = (a.hidden & 7) == 0 && ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.gamma) |
                                               reinterpret_cast<uintptr_t>(a.y)) & 15) == 0;
    float ss = 0.f;
    if (vec) {
        for (int i = threadIdx.x * 8; i < a.hidden; i += kNormThreads * 8) {
            const u32x4 w = *(const u32x4*)(x + i);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = bf16_to_f32(w[j] & 0xFFFFu), hi = bf16_to_f32(w[j] >> 16);
                ss += lo * lo;
                ss += hi * hi;
            }
        }
    } else {
        for (int i = threadIdx.x; i < a.hidden; i += kNormThreads) {
            const float f = bf16_to_f32(x[i]);
            ss += f * f;
        }
    }
    // Wave sum, then the four waves through LDS.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    __shared__ float part[kNormThreads / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kNormThreads / 64; ++w) total += part[w];
    const float inv = 1.0f / sqrtf(total / (float)a.hidden + a.eps);
    if (vec) {
        for (int i = threadIdx.x * 8; i < a.hidden; i += kNormThreads * 8) {
            const u32x4 w = *(const u32x4*)(x + i);
            const u32x4 g = *(const u32x4*)(a.gamma + i);
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = __fmul_rn(__fmul_rn(bf16_to_f32(w[j] & 0xFFFFu), inv), bf16_to_f32(g[j] & 0xFFFFu));
                const float hi = __fmul_rn(__fmul_rn(bf16_to_f32(w[j] >> 16), inv), bf16_to_f32(g[j] >> 16));
                o[j] = (uint32_t)f32_to_bf16_rne(lo) | ((uint32_t)f32_to_bf16_rne(hi) << 16);
            }
            *(u32x4*)(y + i) = o;
        }
    } else {
        for (int i = threadIdx.x; i < a.hidden; i += kNormThreads)
            y[i] = f32_to_bf16_rne(__fmul_rn(__fmul_rn(bf16_to_f32(x[i]), inv), bf16_to_f32(a.gamma[i])));
    }
}

// grid (n_tokens, H_q + 2 H_kv), one thread per (2p, 2p+1) pair of one head of one token.
__global__ __launch_bounds__(kMaxRopePairs) void rope_scatter_kernel(RopeArgs a) {
    const int t = blockIdx.x, h = blockIdx.y, p = threadIdx.x;
    const int D = a.head_dim;
    const uint32_t w = *(const uint32_t*)(a.qkv + (size_t)t * a.ld + (size_t)h * D + 2 * p);
    uint32_t out = w;
    const bool is_q = h < a.n_q_heads, is_k = !is_q && h < a.n_q_heads + a.n_kv_heads;
    if (a.rope && (is_q || is_k)) {
        // Each product and sum is rounded to fp32 on its own: no fused multiply-add.
#pragma clang fp contract(off)
        const int pos = (is_q ? a.q_pos_base : a.kv_pos_base) + t;
        const float phase = (float)pos * a.theta[p];
        double sd, cd;
        sincos((double)phase, &sd, &cd);
        const float s = (float)sd, c = (float)cd;
        const float x0 = bf16_to_f32(w & 0xFFFFu), x1 = bf16_to_f32(w >> 16);
        const float r0 = x0 * c - x1 * s;
        const float r1 = x0 * s + x1 * c;
        out = (uint32_t)f32_to_bf16_rne(r0) | ((uint32_t)f32_to_bf16_rne(r1) << 16);
    }
    uint16_t* dst;
    if (is_q) {
        dst = a.q_out + ((size_t)h * a.n_tokens + t) * D;
    } else {
        const int g = is_k ? h - a.n_q_heads : h - a.n_q_heads - a.n_kv_heads;
        dst = (is_k ? a.kc : a.vc) + ((size_t)g * a.l_cap + a.row0 + t) * D;
    }
    *(uint32_t*)(dst + 2 * p) = out;
}

}  // namespace

hipError_t launch_rms_norm(const NormArgs& a, hipStream_t s) {
    if (a.n_tokens < 1) return hipSuccess;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(a.n_tokens), dim3(kNormThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_rope_scatter(const RopeArgs& a, hipStream_t s) {
    if (a.n_tokens < 1) return hipSuccess;
    if (a.head_dim < 2 || a.head_dim > 2 * kMaxRopePairs || (a.head_dim & 1)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_scatter_kernel, dim3(a.n_tokens, a.n_q_heads + 2 * a.n_kv_heads), dim3(a.head_dim / 2), 0,
                       s, a);
    return hipGetLastError();
}

}  // namespace lara
