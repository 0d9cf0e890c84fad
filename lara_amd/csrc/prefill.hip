// Chunked prefill / full-transaction attention for CDNA4 (gfx950) on bf16 MFMA.
//
// Arithmetic contract (the KV260 datapath, restated for a block of query rows):
//   S[r, j] = sum_d q[r, d] * k[j, d]          (Phase A, attn_tile.sv:176-248)
//   key j valid iff j < kv_len and, causal, kv_pos_base + j <= q_pos_base + r
//                                               (attn_core.sv:138-154, softmax_engine.sv:865-871)
//   online softmax over key blocks: running max m, correction exp(m_old - m_new),
//   running sum l                               (softmax_engine.sv:858-1073)
//   O = sum_j p_j v_j, out = bf16_rne(O / l), 0 for a row with no valid key
//                                               (attn_top.sv:462-625, output_buffer.sv:226-286)
// Like the RTL (attn_top.sv:656), P enters the PV product as bf16 while l sums the fp32 p.
//
// Work decomposition.  A wave owns 32 query rows of one query head; the four waves of a
// work-group own four (row block, head) tasks of one KV head, heads fastest, so for a GQA
// group of 4 the whole group shares every K/V tile the work-group stages in LDS.  Keys are
// processed in blocks of 64:
//   S^T [64 keys x 32 rows] = K [64 x D] . Q^T [D x 32]   two v_mfma_f32_32x32x16_bf16 chains;
//                                                          K from LDS (A), Q^T from VGPRs (B)
//   O^T [D x 32 rows]      += V^T [D x 64] . P^T [64 x 32] D/32 chains of four MFMAs;
//                                                          V^T from LDS (A), P^T from VGPRs (B)
// Computing the transposed products keeps every lane on one query row (column l % 32 of the
// MFMA result), so the softmax state of a row and its O accumulator live in the same lane
// and no cross-lane shuffle is needed between the two products.
//
// Fused chunk append.  With k_new/v_new the launch also places the chunk's own K/V rows at
// cache rows new_begin .. new_begin + n_new - 1: the work-groups with blockIdx.x == 0 copy
// them (spread over kv heads and segments), and every work-group staging one of those rows
// reads it from k_new/v_new instead of the cache, so no work-group waits for the copy.
//
// KV segments.  A chunk of a few hundred query rows gives only tens of work-groups per KV
// head, too few for 256 CUs, so the key range is cut into segments (grid z): each
// work-group attends one segment and writes an fp32 partial (O, m, l) per row, and
// prefill_combine_kernel merges a row's segments with log-sum-exp weights.
//
// MFMA 32x32x16 operand layout used below: lane l supplies row (A) / column (B) l % 32 and
// the eight k-values 8*(l/32)..8*(l/32)+7 of the step; result register i of lane l holds
// row 8*(i/4) + 4*(l/32) + (i%4), column l % 32.  The products only require A and B to
// agree on which k-values a lane holds, so the PV step feeds the P values in the order
// the S^T result leaves them, and V^T is stored in LDS with the matching key order.
#include "gqa_internal.h"

#include <math.h>

namespace lara {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBN = 64;     // keys per block
constexpr int kRows = 32;   // query rows per wave
constexpr int kWaves = 4;
constexpr float kLn2 = 0.693147180559945309f;

__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};  // v_cvt_pk_bf16_f32, round to nearest even
    return __builtin_bit_cast(uint32_t, v);
}

// Key order inside the V^T tile: bits 2 and 3 of the key index are swapped, so the eight
// keys one lane feeds to a PV step are contiguous (one 16-byte LDS read).
__device__ __forceinline__ int vt_pos(int key) {
    return (key & ~0xC) | ((key & 4) << 1) | ((key & 8) >> 1);
}

// 16-byte chunk swizzles (bank-conflict-free MFMA operand reads).
template <int NCH>
__device__ __forceinline__ int k_swz(int row) {
    return NCH == 16 ? (row & 15) : ((row >> 1) & 7);
}
__device__ __forceinline__ int vt_swz(int dim) { return (dim >> 1) & 7; }

template <int D, int G>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(
    PrefillArgs a) {
    constexpr int NCH = D / 8;                 // 16-byte chunks per K/V row
    constexpr int KSTEPS = D / 16;             // QK k-steps
    constexpr int MT = D / 32;                 // PV result tiles (32 dims each)
    constexpr int KLD = kBN * NCH / (kWaves * 64);  // K chunks staged per thread
    constexpr int KPT = NCH / 4;               // V keys staged per thread (same chunk)
    static_assert(KLD >= 1 && KPT >= 1 && KPT <= 4, "tile shape");

    __shared__ __attribute__((aligned(16))) u32x4 lds_k[2][kBN * NCH];
    __shared__ __attribute__((aligned(16))) u32x4 lds_vt[2][D * (kBN / 8)];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = blockIdx.y;  // kv head
    const int n_rb = (a.q_len + kRows - 1) / kRows;
    const int n_tasks = n_rb * G;
    const int task = blockIdx.x * kWaves + wave;
    const bool active = task < n_tasks;
    const int g = task % G;
    const int rb = task / G;
    const int hq = h * G + g;

    // Keys this wave needs: [0, kv_hi) (causal rows stop at their diagonal).
    auto kv_limit = [&](int row_block) {
        int hi = a.kv_len;
        if (a.causal) {
            const int last_row = min(a.q_len, (row_block + 1) * kRows) - 1;
            hi = min(hi, a.q_pos_base + last_row - a.kv_pos_base + 1);
        }
        return max(hi, 0);
    };
    // Fused append: the copy into the cache, before any early exit.
    const bool has_new = a.k_new != nullptr && a.n_new > 0;
    if (has_new && blockIdx.x == 0) {
        const u32x4* ks = reinterpret_cast<const u32x4*>(a.k_new) + (size_t)h * a.n_new * (D / 8);
        const u32x4* vs = reinterpret_cast<const u32x4*>(a.v_new) + (size_t)h * a.n_new * (D / 8);
        u32x4* kd = reinterpret_cast<u32x4*>(a.kc + ((size_t)h * a.l_cap + a.new_begin) * D);
        u32x4* vd = reinterpret_cast<u32x4*>(a.vc + ((size_t)h * a.l_cap + a.new_begin) * D);
        const int words = a.n_new * (D / 8);
        for (int i = blockIdx.z * (kWaves * 64) + threadIdx.x; i < words; i += gridDim.z * (kWaves * 64)) {
            kd[i] = ks[i];
            vd[i] = vs[i];
        }
    }
    const int last_task = min(n_tasks, (int)(blockIdx.x + 1) * kWaves) - 1;
    const int wg_hi = kv_limit(last_task / G);  // row blocks grow with the task index
    const int wave_hi = active ? kv_limit(rb) : 0;
    const int seg_begin = blockIdx.z * a.seg_len;
    // With several segments, one that no row of this work-group reaches is not read by the
    // merge; a single segment always reaches the epilogue (rows without keys output 0).
    if (a.n_segs > 1 && seg_begin >= wg_hi) return;
    const int seg_end = min(wg_hi, seg_begin + a.seg_len);
    const int n_blocks = seg_end > seg_begin ? (seg_end - seg_begin + kBN - 1) / kBN : 0;

    const int col = lane & 31;   // query row within the wave's block (MFMA column)
    const int half = lane >> 5;  // which 8 k-values of a step this lane carries
    const int row = rb * kRows + col;
    const bool row_ok = active && row < a.q_len;
    const int q_pos = a.q_pos_base + row;

    // Q^T operand: row `row`, dims 16*ks + 8*half .. +7.
    u32x4 qb[KSTEPS];
    {
        const u32x4* qp = reinterpret_cast<const u32x4*>(a.q + ((size_t)hq * a.q_len + row) * D);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) qb[ks] = row_ok ? qp[2 * ks + half] : u32x4{0u, 0u, 0u, 0u};
    }

    f32x16 o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[mt][i] = 0.f;
    float m_run = -INFINITY;  // running max (log2 units) of this lane's row
    float l_lane = 0.f;       // this lane's half of the running sum

    // Staging roles: K chunk (key tid / NCH + 256/NCH * i, chunk tid % NCH);
    // V keys KPT*(tid / NCH) .. +KPT-1 of chunk tid % NCH.
    const int sc = tid % NCH;
    const int sk = tid / NCH;
    const u32x4* kg = reinterpret_cast<const u32x4*>(a.kc + (size_t)h * a.l_cap * D);
    const u32x4* vg = reinterpret_cast<const u32x4*>(a.vc + (size_t)h * a.l_cap * D);
    const u32x4* kn = has_new ? reinterpret_cast<const u32x4*>(a.k_new) + (size_t)h * a.n_new * NCH : nullptr;
    const u32x4* vn = has_new ? reinterpret_cast<const u32x4*>(a.v_new) + (size_t)h * a.n_new * NCH : nullptr;
    // Row `row` of this thread's chunk: from the cache, or from this launch's new rows.
    auto k_src = [&](int row) {
        const unsigned r = (unsigned)(row - a.new_begin);
        return (has_new && r < (unsigned)a.n_new) ? kn + (size_t)r * NCH + sc : kg + (size_t)row * NCH + sc;
    };
    auto v_src = [&](int row) {
        const unsigned r = (unsigned)(row - a.new_begin);
        return (has_new && r < (unsigned)a.n_new) ? vn + (size_t)r * NCH + sc : vg + (size_t)row * NCH + sc;
    };

    u32x4 kr[KLD], vr[KPT];
    auto load_block = [&](int j0) {
#pragma unroll
        for (int i = 0; i < KLD; ++i) {
            const int key = sk + i * (kWaves * 64 / NCH);
            kr[i] = *k_src(j0 + key);
        }
#pragma unroll
        for (int b = 0; b < KPT; ++b) {
            const int key = KPT * sk + b;
            // Rows past kv_len may hold stale words: P is 0 there, V must be finite.
            vr[b] = (j0 + key < a.kv_len) ? *v_src(j0 + key) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store_block = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KLD; ++i) {
            const int key = sk + i * (kWaves * 64 / NCH);
            lds_k[buf][key * NCH + (sc ^ k_swz<NCH>(key))] = kr[i];
        }
        // Transpose: dims 8*sc .. 8*sc+7, keys KPT*sk .. +KPT-1 -> V^T rows.
        const int pos = vt_pos(KPT * sk);
        uint16_t* vt = reinterpret_cast<uint16_t*>(&lds_vt[buf][0]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int dim = 8 * sc + e;
            uint16_t w[KPT];
#pragma unroll
            for (int b = 0; b < KPT; ++b) w[b] = (uint16_t)(vr[b][e >> 1] >> (16 * (e & 1)));
            const int elem = (dim * 8 + ((pos >> 3) ^ vt_swz(dim))) * 8 + (pos & 7);
            if constexpr (KPT == 4) {
                uint2 pk;
                pk.x = (uint32_t)w[0] | ((uint32_t)w[1] << 16);
                pk.y = (uint32_t)w[2] | ((uint32_t)w[3] << 16);
                *reinterpret_cast<uint2*>(vt + elem) = pk;
            } else {
                *reinterpret_cast<uint32_t*>(vt + elem) = (uint32_t)w[0] | ((uint32_t)w[1] << 16);
            }
        }
    };

    if (n_blocks > 0) load_block(seg_begin);
    for (int blk = 0; blk < n_blocks; ++blk) {
        const int buf = blk & 1;
        const int j0 = seg_begin + blk * kBN;
        store_block(buf);
        __syncthreads();
        if (blk + 1 < n_blocks) load_block(j0 + kBN);
        if (j0 >= wave_hi) continue;  // this wave's rows see no key of the block

        // ---- S^T = K . Q^T ----
        f32x16 st[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) st[kt][i] = 0.f;
            const int key = kt * 32 + col;
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                const u32x4 kw = lds_k[buf][key * NCH + ((2 * ks + half) ^ k_swz<NCH>(key))];
                st[kt] = mfma32(kw, qb[ks], st[kt]);
            }
        }

        // ---- online softmax (log2 domain) on this lane's row ----
        const bool need_mask =
            (j0 + kBN > a.kv_len) || (a.causal && a.kv_pos_base + j0 + kBN - 1 > a.q_pos_base + rb * kRows);
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float s = st[kt][i] * a.scale_log2;
                if (need_mask) {
                    const int j = j0 + kt * 32 + 8 * (i >> 2) + 4 * half + (i & 3);
                    const bool ok = row_ok && j < a.kv_len && (!a.causal || a.kv_pos_base + j <= q_pos);
                    s = ok ? s : -INFINITY;
                }
                st[kt][i] = s;
                mx = fmaxf(mx, s);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const bool none = (m_new == -INFINITY);
        const float corr = none ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
        float psum = 0.f;
        u32x4 pb[4];  // P^T operand of the four PV k-steps (kt, a2)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int a2 = 0; a2 < 2; ++a2) {
                float p[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float s = st[kt][8 * a2 + j];
                    p[j] = (s == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(s - m_new);
                    psum += p[j];
                }
                pb[2 * kt + a2] = u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                        pack_bf16x2(p[6], p[7])};
            }
        l_lane = l_lane * corr + psum;
        m_run = m_new;

        // ---- O^T = O^T * corr + V^T . P^T ----
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) o[mt][i] *= corr;
            const int dim = mt * 32 + col;
#pragma unroll
            for (int st_i = 0; st_i < 4; ++st_i) {
                const u32x4 vw = lds_vt[buf][dim * 8 + ((st_i * 2 + half) ^ vt_swz(dim))];
                o[mt] = mfma32(vw, pb[st_i], o[mt]);
            }
        }
    }

    if (!row_ok) return;
    const float l_row = l_lane + __shfl_xor(l_lane, 32);
    if (a.n_segs > 1) {
        // Rows this wave never reached in the segment are not read by the merge.
        if (seg_begin >= wave_hi) return;
        const size_t prow = ((size_t)blockIdx.z * a.n_q_heads + hq) * a.q_len + row;
        float* po = a.part_o + prow * D;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                *reinterpret_cast<float4*>(po + mt * 32 + 8 * r4 + 4 * half) =
                    make_float4(o[mt][4 * r4 + 0], o[mt][4 * r4 + 1], o[mt][4 * r4 + 2], o[mt][4 * r4 + 3]);
        if (half == 0) *reinterpret_cast<float2*>(a.part_ml + prow * 2) = make_float2(m_run, l_row);
        return;
    }
    const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
    uint16_t* orow = a.out + ((size_t)hq * a.q_len + row) * D;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            uint2 w;
            w.x = (uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 0] * inv) | ((uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 1] * inv) << 16);
            w.y = (uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 2] * inv) | ((uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 3] * inv) << 16);
            *reinterpret_cast<uint2*>(orow + mt * 32 + 8 * r4 + 4 * half) = w;
        }
    if (half == 0 && a.lse != nullptr)
        a.lse[(size_t)hq * a.q_len + row] = l_row > 0.f ? (m_run + log2f(l_row)) * kLn2 : -INFINITY;
}

// Merge of a row's KV segments: one work-group per (query row, query head), one thread per
// dim.  Segment s holds keys [s*seg_len, (s+1)*seg_len); a row reads the segments below its
// own key limit, which are exactly the ones prefill_kernel wrote for it.
template <int D>
__global__ __launch_bounds__(D) void prefill_combine_kernel(PrefillArgs a) {
    const int row = blockIdx.x;
    const int hq = blockIdx.y;
    const int d = threadIdx.x;
    int hi = a.kv_len;
    if (a.causal) hi = min(hi, a.q_pos_base + row - a.kv_pos_base + 1);
    hi = max(hi, 0);
    const int n_valid = min(a.n_segs, (hi + a.seg_len - 1) / a.seg_len);
    const size_t seg_stride = (size_t)a.n_q_heads * a.q_len;
    const size_t prow = (size_t)hq * a.q_len + row;
    float M = -INFINITY;
    for (int sp = 0; sp < n_valid; ++sp) M = fmaxf(M, a.part_ml[(sp * seg_stride + prow) * 2]);
    float O = 0.f, Ls = 0.f;
    if (M != -INFINITY) {
        for (int sp = 0; sp < n_valid; ++sp) {
            const size_t pr = sp * seg_stride + prow;
            const float w = __builtin_amdgcn_exp2f(a.part_ml[pr * 2] - M);
            O = fmaf(w, a.part_o[pr * D + d], O);
            Ls = fmaf(w, a.part_ml[pr * 2 + 1], Ls);
        }
    }
    a.out[prow * D + d] = f32_to_bf16_rne(Ls > 0.f ? O / Ls : 0.f);
    if (d == 0 && a.lse != nullptr) a.lse[prow] = Ls > 0.f ? (M + log2f(Ls)) * kLn2 : -INFINITY;
}

template <int D, int G>
hipError_t launch_prefill_t(const PrefillArgs& a, hipStream_t s) {
    const int n_rb = (a.q_len + kRows - 1) / kRows;
    const int n_tasks = n_rb * G;
    dim3 grid((n_tasks + kWaves - 1) / kWaves, a.n_kv_heads, a.n_segs);
    hipLaunchKernelGGL((prefill_kernel<D, G>), grid, dim3(kWaves * 64), 0, s, a);
    return hipGetLastError();
}

}  // namespace

PrefillPlan plan_prefill(int q_len, int kv_span, int group, int n_kv_heads, int target_wgs, int max_segs) {
    const int n_rb = (q_len + kRows - 1) / kRows;
    const int base = ((n_rb * group + kWaves - 1) / kWaves) * n_kv_heads;
    const int blocks = (kv_span + kBN - 1) / kBN;
    int segs = (target_wgs + base - 1) / base;
    segs = min(segs, max_segs);
    segs = min(segs, blocks);
    if (segs <= 1) return PrefillPlan{blocks > 0 ? blocks * kBN : kBN, 1};
    const int seg_blocks = (blocks + segs - 1) / segs;
    const int seg_len = seg_blocks * kBN;
    return PrefillPlan{seg_len, (blocks + seg_blocks - 1) / seg_blocks};
}

size_t prefill_workspace_floats(const PrefillPlan& p, int q_len, int n_q_heads, int head_dim) {
    if (p.n_segs <= 1) return 0;
    return (size_t)p.n_segs * n_q_heads * q_len * (head_dim + 2);
}

hipError_t launch_prefill_combine(int head_dim, const PrefillArgs& a, hipStream_t s) {
    if (head_dim == 128) {
        hipLaunchKernelGGL(prefill_combine_kernel<128>, dim3(a.q_len, a.n_q_heads), dim3(128), 0, s, a);
    } else if (head_dim == 64) {
        hipLaunchKernelGGL(prefill_combine_kernel<64>, dim3(a.q_len, a.n_q_heads), dim3(64), 0, s, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool prefill_supported(int head_dim, int group) {
    return (head_dim == 64 || head_dim == 128) && (group == 1 || group == 2 || group == 4 || group == 8 || group == 16);
}

hipError_t launch_prefill(int head_dim, int group, const PrefillArgs& a, hipStream_t s) {
    if (head_dim == 128) {
        if (group == 4) return launch_prefill_t<128, 4>(a, s);
        if (group == 8) return launch_prefill_t<128, 8>(a, s);
        if (group == 2) return launch_prefill_t<128, 2>(a, s);
        if (group == 1) return launch_prefill_t<128, 1>(a, s);
        if (group == 16) return launch_prefill_t<128, 16>(a, s);
    } else if (head_dim == 64) {
        if (group == 4) return launch_prefill_t<64, 4>(a, s);
        if (group == 8) return launch_prefill_t<64, 8>(a, s);
        if (group == 2) return launch_prefill_t<64, 2>(a, s);
        if (group == 1) return launch_prefill_t<64, 1>(a, s);
        if (group == 16) return launch_prefill_t<64, 16>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace lara
