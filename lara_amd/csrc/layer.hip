// Layer input stage of run_layer (sw/attn_driver.py:552-576): the host RMSNorm, RoPE and
// head reshaping that the reference does in numpy before each attention transaction, here
// as two small HBM-bound kernels around the QKV projection GEMM.
//
// rms_norm_*_kernel: y = x / sqrt(mean(x^2) + eps) * gamma per token row
//   (hw/rtl/ext/rms_norm/rms_norm.sv:7-8, 42-45: sum of squares, inverse square root, two
//   products), sums and products in fp32, one RNE rounding to bf16.  The same launch fills the
//   RoPE cos/sin table in extra work-groups: the norm is memory-bound, so the double-precision
//   sin/cos run on otherwise idle ALUs, off the RoPE kernel's path.
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

__host__ __device__ inline bool norm_vectorised(const NormArgs& a) {
    return (a.hidden & 7) == 0 &&
           ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.gamma) | reinterpret_cast<uintptr_t>(a.y)) &
            15) == 0;
}

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

// Work-group `wg` (< table_wgs) of a norm launch: one table entry per thread.
__device__ __forceinline__ void fill_rope_table(const RopeTable& t, int wg) {
    const int i = wg * kNormThreads + threadIdx.x;
    if (i >= t.sets * t.n_tokens * t.pairs) return;
    const int p = i % t.pairs, tok = (i / t.pairs) % t.n_tokens, set = i / (t.pairs * t.n_tokens);
    {
#pragma clang fp contract(off)
        double sd, cd;
        sincos((double)((float)((set ? t.kv_pos_base : t.q_pos_base) + tok) * t.theta[p]), &sd, &cd);
        reinterpret_cast<float2*>(t.cs)[i] = make_float2((float)cd, (float)sd);
    }
}

// Row-per-wave form for hidden = CPL * 512 (16-byte aligned rows): each wave owns one token
// row, holds its CPL chunks of x and of gamma in registers (chunk c * 64 + lane, so every load
// instruction covers 1 KiB of the row), sums the squares with a wave reduction (no LDS, no
// barrier) and writes the scaled row.  Rows are independent, so a wave whose loads return
// early computes and stores while other waves' loads are still in flight.
template <int CPL>
__global__ __launch_bounds__(kNormThreads) void rms_norm_wave_kernel(NormArgs a) {
    if ((int)blockIdx.x < a.table_wgs) {
        fill_rope_table(a.table, blockIdx.x);
        return;
    }
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x - a.table_wgs) * (kNormThreads / 64) + (threadIdx.x >> 6);
    if (row >= a.n_tokens) return;
    const u32x4* x = reinterpret_cast<const u32x4*>(a.x + (size_t)row * a.hidden);
    const u32x4* g = reinterpret_cast<const u32x4*>(a.gamma);
    u32x4 v[CPL], gv[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) v[c] = __builtin_nontemporal_load(x + c * 64 + lane);
#pragma unroll
    for (int c = 0; c < CPL; ++c) gv[c] = g[c * 64 + lane];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) ss += sum_squares(v[c]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float inv = 1.0f / sqrtf(ss / (float)a.hidden + a.eps);
    u32x4* y = reinterpret_cast<u32x4*>(a.y + (size_t)row * a.hidden);
#pragma unroll
    for (int c = 0; c < CPL; ++c) y[c * 64 + lane] = scale_row(v[c], gv[c], inv);  // the projection reads y next
}

// General form: one work-group per token row.  With hidden % 8 == 0 and 16-byte aligned rows each
// thread moves 16-byte chunks and keeps its first kNormCached chunks in registers between the sum
// of squares and the scaling pass; otherwise one bf16 per thread and step.  With gamma == nullptr
// the launch only fills the table.
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(NormArgs a) {
    if ((int)blockIdx.x < a.table_wgs) {
        fill_rope_table(a.table, blockIdx.x);
        return;
    }
    const int row = blockIdx.x - a.table_wgs;
    const uint16_t* x = a.x + (size_t)row * a.hidden;
    uint16_t* y = a.y + (size_t)row * a.hidden;
    const bool vec = norm_vectorised(a);
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

// Rotate the four (2p, 2p+1) pairs of one 16-byte chunk of head h by the (cos, sin) values cs
// (two pairs per float4) and store the chunk at its destination.
__device__ __forceinline__ void rope_store_chunk(const RopeArgs& a, int t, int h, int cw, u32x4 w, const float4* cq,
                                                 const float4* ck) {
    const int D = a.head_dim;
    const bool is_q = h < a.n_q_heads, is_k = !is_q && h < a.n_q_heads + a.n_kv_heads;
    if (a.rope && (is_q || is_k)) {
        const float4* csp = is_q ? cq : ck;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma clang fp contract(off)
            // Each product and sum is rounded to fp32 on its own: no fused multiply-add.
            const float4 pair2 = csp[j >> 1];
            const float c = (j & 1) ? pair2.z : pair2.x, s = (j & 1) ? pair2.w : pair2.y;
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
            if (r < 0) return;  // unmapped page: nothing to write
        }
        dst = (is_k ? a.kc : a.vc) + (size_t)r * D;
    }
    *reinterpret_cast<u32x4*>(dst + 8 * cw) = w;
}

// One work-group per token: the token's H_q + 2 H_kv head rows move in 16-byte chunks of four
// (2p, 2p+1) pairs, one chunk per thread and step (three steps for a 32 + 2 x 8 head, D = 128
// token; 128, 512 and 768 threads measured slower at 2048 tokens).  kRopeThreads is a multiple of
// D / 8, so a thread's pairs are the same in every head: it loads their cos/sin from the table
// once per position set.  No LDS and no barrier: every chunk streams independently.
__global__ __launch_bounds__(kRopeThreads) void rope_scatter_kernel(RopeArgs a) {
    const int t = blockIdx.x;
    const int D = a.head_dim, P = D / 2, CPH = D / 8;  // pairs and 16-byte chunks per head row
    const int n_chunks = (a.n_q_heads + 2 * a.n_kv_heads) * CPH;
    const int cw = threadIdx.x % CPH;
    const u32x4* src = reinterpret_cast<const u32x4*>(a.qkv + (size_t)t * a.ld);
    float4 cq[2] = {}, ck[2] = {};  // (cos, sin) of pairs 4cw .. 4cw+3 at the Q and the K position
    if (a.rope) {
        const float4* tq = reinterpret_cast<const float4*>(a.cs + ((size_t)t * P + 4 * cw) * 2);
        cq[0] = tq[0];
        cq[1] = tq[1];
        const float4* tk = reinterpret_cast<const float4*>(a.cs + (((size_t)a.cs_k_set * a.n_tokens + t) * P + 4 * cw) * 2);
        ck[0] = tk[0];
        ck[1] = tk[1];
    }
    for (int ci = threadIdx.x; ci < n_chunks; ci += kRopeThreads)
        rope_store_chunk(a, t, ci / CPH, cw, __builtin_nontemporal_load(src + ci), cq, ck);
}

}  // namespace

hipError_t launch_rms_norm(const NormArgs& args, const Launch& l) {
    NormArgs a = args;
    const int entries = a.table.cs ? a.table.sets * a.table.n_tokens * a.table.pairs : 0;
    a.table_wgs = (entries + kNormThreads - 1) / kNormThreads;
    const int rows = a.gamma ? a.n_tokens : 0;
    if (rows < 1 && a.table_wgs == 0) return hipSuccess;
    constexpr int rows_per_wg = kNormThreads / 64;
    const dim3 block(kNormThreads);
    if (rows > 0 && norm_vectorised(a)) {
        const dim3 grid(a.table_wgs + (rows + rows_per_wg - 1) / rows_per_wg);
        switch (a.hidden) {
            case 512: return launch_kernel(rms_norm_wave_kernel<1>, grid, block, l, a);
            case 1024: return launch_kernel(rms_norm_wave_kernel<2>, grid, block, l, a);
            case 2048: return launch_kernel(rms_norm_wave_kernel<4>, grid, block, l, a);
            case 4096: return launch_kernel(rms_norm_wave_kernel<8>, grid, block, l, a);
            case 8192: return launch_kernel(rms_norm_wave_kernel<16>, grid, block, l, a);
            default: break;
        }
    }
    return launch_kernel(rms_norm_kernel, dim3(a.table_wgs + rows), block, l, a);
}

hipError_t launch_rope_scatter(const RopeArgs& a, const Launch& l) {
    if (a.n_tokens < 1) return hipSuccess;
    if (a.head_dim < 8 || a.head_dim > 2 * kMaxRopePairs || (a.head_dim & 7) || kRopeThreads % (a.head_dim / 8) ||
        (a.rope && a.cs == nullptr))
        return hipErrorInvalidValue;
    return launch_kernel(rope_scatter_kernel, dim3(a.n_tokens), dim3(kRopeThreads), l, a);
}

}  // namespace lara
