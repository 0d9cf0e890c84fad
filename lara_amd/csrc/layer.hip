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

constexpr int kNormCached = 4;  // 16-byte chunks a thread keeps in registers (hidden <= 8192)

__device__ __forceinline__ float sum_squares(const u32x4& w) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float lo = bf16_to_f32(w[j] & 0xFFFFu), hi = bf16_to_f32(w[j] >> 16);
        ss += lo * lo;
        ss += hi * hi;
    }
    return ss;
}

__device__ __forceinline__ u32x4 scale_row(const u32x4& w, const u32x4& g, float inv) {
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float lo = __fmul_rn(__fmul_rn(bf16_to_f32(w[j] & 0xFFFFu), inv), bf16_to_f32(g[j] & 0xFFFFu));
        const float hi = __fmul_rn(__fmul_rn(bf16_to_f32(w[j] >> 16), inv), bf16_to_f32(g[j] >> 16));
        o[j] = (uint32_t)f32_to_bf16_rne(lo) | ((uint32_t)f32_to_bf16_rne(hi) << 16);
    }
    return o;
}

// One work-group per token row.  With hidden % 8 == 0 and 16-byte aligned rows each thread
// moves 16-byte chunks and keeps its first kNormCached chunks in registers between the sum
// of squares and the scaling pass; otherwise one bf16 per thread and step.
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(NormArgs a) {
    const int row = blockIdx.x;
    const uint16_t* x = a.x + (size_t)row * a.hidden;
    uint16_t* y = a.y + (size_t)row * a.hidden;
    const bool vec = (a.hidden & 7) == 0 && ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.gamma) |
                                               reinterpret_cast<uintptr_t>(a.y)) & 15) == 0;
    constexpr int kStep = kNormThreads * 8;
    float ss = 0.f;
    u32x4 cache[kNormCached], gcache[kNormCached];  // x and gamma chunks, gamma loaded with x
    if (vec) {
#pragma unroll
        for (int c = 0; c < kNormCached; ++c) {
            const int i = c * kStep + threadIdx.x * 8;
            cache[c] = i < a.hidden ? __builtin_nontemporal_load((const u32x4*)(x + i)) : u32x4{0u, 0u, 0u, 0u};
            gcache[c] = i < a.hidden ? *(const u32x4*)(a.gamma + i) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int c = 0; c < kNormCached; ++c) ss += sum_squares(cache[c]);
        for (int i = kNormCached * kStep + threadIdx.x * 8; i < a.hidden; i += kStep)
            ss += sum_squares(*(const u32x4*)(x + i));
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
#pragma unroll
        for (int c = 0; c < kNormCached; ++c) {
            const int i = c * kStep + threadIdx.x * 8;
            if (i < a.hidden) *(u32x4*)(y + i) = scale_row(cache[c], gcache[c], inv);
        }
        for (int i = kNormCached * kStep + threadIdx.x * 8; i < a.hidden; i += kStep)
            *(u32x4*)(y + i) = scale_row(*(const u32x4*)(x + i), *(const u32x4*)(a.gamma + i), inv);
    } else {
        for (int i = threadIdx.x; i < a.hidden; i += kNormThreads)
            y[i] = f32_to_bf16_rne(__fmul_rn(__fmul_rn(bf16_to_f32(x[i]), inv), bf16_to_f32(a.gamma[i])));
    }
}

constexpr int kRopeThreads = 256;

// grid (n_tokens, ceil((H_q + 2 H_kv) / 8)); one wave per block, one lane per (2p, 2p+1)
// pair.  A lane evaluates cos/sin once for the Q position and once for the K position, loads
// its pair of all 8 heads (each head row is D*2 contiguous bytes across the wave) before
// rotating and storing them.
// One work-group per token: the (position, pair) cos/sin values are computed once into LDS,
// then the token's H_q + 2 H_kv head rows move in 16-byte chunks (four pairs per thread and
// chunk; a thread's pairs are the same in every head, as 256 is a multiple of D / 8).
__global__ __launch_bounds__(kRopeThreads) void rope_scatter_kernel(RopeArgs a) {
    __shared__ float cs[2][kMaxRopePairs][2];  // [Q position | K position][pair][cos, sin]
    const int t = blockIdx.x;
    const int D = a.head_dim, P = D / 2, CPH = D / 8;  // pairs and 16-byte chunks per head row
    const int H = a.n_q_heads + 2 * a.n_kv_heads;
    const bool same_pos = a.kv_pos_base == a.q_pos_base;
    if (a.rope) {
        for (int i = threadIdx.x; i < 2 * P; i += kRopeThreads) {
            const int which = i / P, p = i - which * P;  // 0: the Q position, 1: the K position
            if (which == 1 && same_pos) continue;
            {
#pragma clang fp contract(off)
                double sd, cd;
                sincos((double)((float)((which ? a.kv_pos_base : a.q_pos_base) + t) * a.theta[p]), &sd, &cd);
                cs[which][p][0] = (float)cd;
                cs[which][p][1] = (float)sd;
            }
        }
        __syncthreads();
    }
    const u32x4* src = reinterpret_cast<const u32x4*>(a.qkv + (size_t)t * a.ld);
    for (int ci = threadIdx.x; ci < H * CPH; ci += kRopeThreads) {
        const int h = ci / CPH, cw = ci - h * CPH;
        u32x4 w = __builtin_nontemporal_load(src + ci);
        const bool is_q = h < a.n_q_heads, is_k = !is_q && h < a.n_q_heads + a.n_kv_heads;
        if (a.rope && (is_q || is_k)) {
            const int which = (is_k && !same_pos) ? 1 : 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma clang fp contract(off)
                // Each product and sum is rounded to fp32 on its own: no fused multiply-add.
                const float c = cs[which][4 * cw + j][0], s = cs[which][4 * cw + j][1];
                const float x0 = bf16_to_f32(w[j] & 0xFFFFu), x1 = bf16_to_f32(w[j] >> 16);
                const float r0 = x0 * c - x1 * s;
                const float r1 = x0 * s + x1 * c;
                w[j] = (uint32_t)f32_to_bf16_rne(r0) | ((uint32_t)f32_to_bf16_rne(r1) << 16);
            }
        }
        uint16_t* dst;
        if (is_q) {
            dst = a.q_out + ((size_t)h * a.n_tokens + t) * D;
        } else {
            const int g = is_k ? h - a.n_q_heads : h - a.n_q_heads - a.n_kv_heads;
            int64_t r = (int64_t)g * a.l_cap + a.row0 + t;
            if (a.block_table != nullptr) {
                r = paged_row(a.block_table, a.page_shift, a.n_kv_heads, g, a.row0 + t);
                if (r < 0) continue;  // unmapped page: nothing to write
            }
            dst = (is_k ? a.kc : a.vc) + (size_t)r * D;
        }
        *reinterpret_cast<u32x4*>(dst + 8 * cw) = w;
    }
}

}  // namespace

hipError_t launch_rms_norm(const NormArgs& a, const Launch& l) {
    if (a.n_tokens < 1) return hipSuccess;
    return launch_kernel(rms_norm_kernel, dim3(a.n_tokens), dim3(kNormThreads), l, a);
}

hipError_t launch_rope_scatter(const RopeArgs& a, const Launch& l) {
    if (a.n_tokens < 1) return hipSuccess;
    if (a.head_dim < 8 || a.head_dim > 2 * kMaxRopePairs || (a.head_dim & 7) || kRopeThreads % (a.head_dim / 8))
        return hipErrorInvalidValue;
    return launch_kernel(rope_scatter_kernel, dim3(a.n_tokens), dim3(kRopeThreads), l, a);
}

}  // namespace lara
