// KV260 RTL-exact numerics mode: the board's bit-level arithmetic on gfx950.
//
// The deployed KV260 datapath does not compute IEEE-exact softmax attention; it computes
// (hw/rtl/pkg/attn_pkg.sv:341-626, hw/rtl/core/softmax_engine.sv:570-1334,
//  hw/rtl/attn_top.sv:653-658, hw/rtl/mem/output_buffer.sv:192-286):
//   S      = sequential fp32 sum over d of exact bf16 products (bf16 exponent 0 reads as 0)
//   s'     = fp32 RNE product with the scale; masked keys -inf
//   per 16-key sub-block and row: row max by bit-pattern compare, m_new = max(m_old, row max),
//   corr   = 0 on the first sub-block, else E(m_old - m_new); p = masked ? 0 : E(s' - m_new),
//   where E is a 1024-entry exp table on [-8, 0] with fixed-point index math and linear
//   interpolation; l = first ? sum p : l*corr + sum p (left to right)
//   dO     = sequential sum over the sub-block's keys of exact products of the UPPER 16 BITS of
//            p (truncation) with V; O = O*corr + dO
//   out    = l == 0 ? 0 : O * R(l), R from a 256-entry reciprocal-mantissa table; bf16 RNE
// over 32-row Q tiles and 64-key KV tiles of four sub-blocks, with the causal KV-tile limit of
// hw/rtl/core/attn_core.sv:138-154.  This kernel reproduces that bit for bit so outputs can be
// compared with board results exactly.
//
// Arithmetic: the RTL's fp32 add and multiply round like IEEE round-to-nearest-even for normal
// operands and results, so the common case runs on native v_add_f32 / v_mul_f32 (with
// contraction off); zero operands, exponent-range edges, inf and NaN take the bit-level path
// that restates the RTL's rules (a zero operand returns the other operand unchanged, 8-bit
// exponent wrap, canonical NaN).
//
// Work decomposition: one lane owns one query row of one query head and walks that row's
// sub-blocks in the board's order; a wave holds 64 consecutive rows of one head, so every
// lane reads the same K/V word at the same time.  Scores and the O accumulator live in LDS
// columns private to each lane.
#include "gqa_internal.h"
#include "rtl_luts.inc"  // kRtlExpLut[1024], kRtlRecipLut[256]: the board's ROM images

#include <math.h>

#pragma clang fp contract(off)

namespace lara {
namespace {

constexpr uint32_t kNan = 0x7FC00000u;
constexpr uint32_t kNegInf = 0xFF800000u;
constexpr uint32_t kOne = 0x3F800000u;
constexpr uint32_t kNegEight = 0xC1000000u;

__device__ __forceinline__ uint32_t ex(uint32_t a) { return (a >> 23) & 0xFFu; }
__device__ __forceinline__ bool zero_b(uint32_t a) { return (a & 0x7FFFFFFFu) == 0u; }
__device__ __forceinline__ bool nan_b(uint32_t a) { return ex(a) == 0xFFu && (a & 0x7FFFFFu) != 0u; }
__device__ __forceinline__ bool inf_b(uint32_t a) { return ex(a) == 0xFFu && (a & 0x7FFFFFu) == 0u; }
__device__ __forceinline__ bool normal_b(uint32_t a) { return ex(a) - 1u < 254u; }
__device__ __forceinline__ float f_(uint32_t a) { return __uint_as_float(a); }
__device__ __forceinline__ uint32_t b_(float a) { return __float_as_uint(a); }

// ---- bit-level paths (operands or results outside the normal range) ----------------------

__device__ __noinline__ uint32_t add_bits(uint32_t a, uint32_t b) {
    // 56-bit aligned significands with a sticky bit, leading-zero count limited to 24,
    // round to nearest even, 8-bit exponent arithmetic; exponent 0 reads as 1 without the
    // hidden bit, exponent 255 as an ordinary value.
    const uint32_t ea0 = ex(a), eb0 = ex(b);
    const uint32_t ma = (ea0 ? 0x800000u : 0u) | (a & 0x7FFFFFu);
    const uint32_t mb = (eb0 ? 0x800000u : 0u) | (b & 0x7FFFFFu);
    const uint32_t ea = ea0 ? ea0 : 1u, eb = eb0 ? eb0 : 1u;
    const bool a_big = ea > eb || (ea == eb && ma >= mb);
    const uint32_t e_big = a_big ? ea : eb;
    const uint32_t diff = a_big ? ea - eb : eb - ea;
    const uint64_t big = (uint64_t)(a_big ? ma : mb) << 32;
    const uint64_t small = (uint64_t)(a_big ? mb : ma) << 32;
    uint64_t sh;
    if (diff >= 56u) {
        sh = small != 0 ? 1u : 0u;
    } else {
        sh = small >> diff;
        if (diff != 0u && (small & ((1ull << diff) - 1u)) != 0) sh |= 1u;
    }
    const bool sub = ((a ^ b) >> 31) != 0u;
    const uint64_t sum = sub ? big - sh : big + sh;
    if (sum == 0) return 0u;
    uint32_t e = e_big;
    uint64_t n;
    if (sum >> 56) {
        e = (e + 1u) & 0xFFu;
        n = (sum >> 1) | (sum & 1u);
    } else {
        const uint32_t top = (uint32_t)(sum >> 32) & 0xFFFFFFu;
        const uint32_t lz = top ? (uint32_t)(__clz(top) - 8) : 24u;
        n = (sum << lz) & ((1ull << 56) - 1);
        e = (e - lz) & 0xFFu;
    }
    const uint32_t keep = (uint32_t)(n >> 32) & 0xFFFFFFu;
    const bool guard = (n >> 31) & 1u;
    const bool rest = (n & 0x7FFFFFFFull) != 0;
    uint32_t r = keep + ((guard && (rest || (keep & 1u))) ? 1u : 0u);
    uint32_t frac = r & 0x7FFFFFu;
    if (r >> 24) {
        e = (e + 1u) & 0xFFu;
        frac = 0u;
    }
    return ((a_big ? a : b) & 0x80000000u) | (e << 23) | frac;
}

__device__ __noinline__ uint32_t mul_bits(uint32_t a, uint32_t b) {
    // both significands carry the hidden bit whatever the exponent; 8-bit exponent wrap
    const uint64_t p = (uint64_t)(0x800000u | (a & 0x7FFFFFu)) * (0x800000u | (b & 0x7FFFFFu));
    const uint32_t top = (uint32_t)(p >> 47) & 1u;
    uint32_t e = (ex(a) + ex(b) - 127u + top) & 0xFFu;
    const uint32_t keep = 0x800000u | ((uint32_t)(p >> (23 + top)) & 0x7FFFFFu);
    const bool guard = (p >> (22 + top)) & 1u;
    const bool rest = (p & ((1ull << (22 + top)) - 1u)) != 0;
    uint32_t r = keep + ((guard && (rest || (keep & 1u))) ? 1u : 0u);
    if (r >> 24) {
        e = (e + 1u) & 0xFFu;
        r = 0x800000u;
    }
    return ((a ^ b) & 0x80000000u) | (e << 23) | (r & 0x7FFFFFu);
}

// ---- the board's operators -------------------------------------------------------------

__device__ __forceinline__ uint32_t add(uint32_t a, uint32_t b) {
    if (normal_b(a) && normal_b(b)) {
        const uint32_t r = b_(f_(a) + f_(b));
        if (normal_b(r)) return r;
        if (r == 0u && a == (b ^ 0x80000000u)) return 0u;  // exact cancellation
        return add_bits(a, b);
    }
    if (nan_b(a) || nan_b(b)) return kNan;
    if (zero_b(a)) return b;
    if (zero_b(b)) return a;
    return add_bits(a, b);
}

__device__ __forceinline__ uint32_t sub(uint32_t a, uint32_t b) { return add(a, b ^ 0x80000000u); }

__device__ __forceinline__ uint32_t mul(uint32_t a, uint32_t b) {
    if (normal_b(a) && normal_b(b)) {
        const uint32_t r = b_(f_(a) * f_(b));
        if (normal_b(r)) return r;
        return mul_bits(a, b);
    }
    if (nan_b(a) || nan_b(b)) return kNan;
    if (zero_b(a) || zero_b(b)) return (a ^ b) & 0x80000000u;
    if (inf_b(a) || inf_b(b)) return ((a ^ b) & 0x80000000u) | 0x7F800000u;
    return mul_bits(a, b);
}

// exact product of two bf16 words
__device__ __forceinline__ uint32_t bmul(uint32_t a16, uint32_t b16) {
    const uint32_t ea = (a16 >> 7) & 0xFFu, eb = (b16 >> 7) & 0xFFu;
    const uint32_t s = ((a16 ^ b16) & 0x8000u) << 16;
    if (ea - 1u < 254u && eb - 1u < 254u && ea + eb - 128u < 253u)  // result exponent 1..254
        return b_(f_(a16 << 16) * f_(b16 << 16));
    const bool az = ea == 0u, bz = eb == 0u;
    const bool ainf = ea == 0xFFu && (a16 & 0x7Fu) == 0u, binf = eb == 0xFFu && (b16 & 0x7Fu) == 0u;
    if ((ea == 0xFFu && !ainf) || (eb == 0xFFu && !binf)) return kNan;
    if ((ainf && bz) || (az && binf)) return kNan;
    if (ainf || binf) return s | 0x7F800000u;
    if (az || bz) return s;
    const uint32_t p = (0x80u | (a16 & 0x7Fu)) * (0x80u | (b16 & 0x7Fu));
    const uint32_t top = p >> 15;
    const uint32_t e = (ea + eb - 127u + top) & 0xFFu;
    return s | (e << 23) | ((p << (9 - top)) & 0x7FFFFFu);
}

__device__ __forceinline__ bool gt(uint32_t a, uint32_t b) {
    if (a == b) return false;
    if ((a ^ b) >> 31) return (b >> 31) != 0u;
    return (a >> 31) ? (a & 0x7FFFFFFFu) < (b & 0x7FFFFFFFu) : (a & 0x7FFFFFFFu) > (b & 0x7FFFFFFFu);
}

__device__ __forceinline__ uint32_t mx(uint32_t a, uint32_t b) { return gt(a, b) ? a : b; }

// E(x): the interpolated exp table (softmax_engine.sv:570-706)
__device__ uint32_t exp_table(uint32_t x) {
    if (gt(kNegEight, x)) return 0u;
    if (gt(x, 0u)) return kOne;
    int64_t xq = 0;
    if (!zero_b(x)) {
        const int sh = (int)ex(x) - 127;
        const int64_t m = 0x800000 | (x & 0x7FFFFF);
        xq = sh >= 0 ? (m << sh) : (sh < -40 ? 0 : (m >> (-sh)));
        if (x >> 31) xq = -xq;
    }
    int64_t n = xq + (1ll << 26);
    n = n < 0 ? 0 : (n > (1ll << 26) ? (1ll << 26) : n);
    const int64_t num = n * 1023;
    const int idx = (int)(num >> 26);
    if (idx >= 1023) return kRtlExpLut[1023];
    const int64_t rem = num & ((1ll << 26) - 1);
    uint32_t frac = 0u;  // rem as fp32, mantissa truncated
    if (rem > 0) {
        const int bit = 63 - __clzll(rem);
        const uint64_t res = (uint64_t)rem - (1ull << bit);
        const uint32_t mant = bit < 23 ? (uint32_t)(res << (23 - bit)) : (uint32_t)(res >> (bit - 23));
        frac = ((uint32_t)(127 + bit - 26) << 23) | (mant & 0x7FFFFFu);
    }
    const uint32_t lo = kRtlExpLut[idx], hi = kRtlExpLut[idx + 1];
    return add(lo, mul(sub(hi, lo), frac));
}

// R(l): reciprocal from the mantissa table (output_buffer.sv:192-224)
__device__ __forceinline__ uint32_t recip_table(uint32_t l) {
    const uint32_t s = l & 0x80000000u, e = ex(l), f = l & 0x7FFFFFu;
    if (nan_b(l)) return kNan;
    if (zero_b(l)) return s | 0x7F800000u;
    if (inf_b(l)) return s;
    if (f == 0u) return s | (((254u - e) & 0xFFu) << 23);
    return s | (((253u - e) & 0xFFu) << 23) | kRtlRecipLut[f >> 15];
}

__device__ __forceinline__ uint16_t to_bf16(uint32_t a) {
    const uint32_t up = ((a >> 15) & 1u) && ((a & 0x7FFFu) || ((a >> 16) & 1u));
    return (uint16_t)((a >> 16) + up);
}

constexpr int kLanes = 64;

template <int D>
__global__ __launch_bounds__(kLanes) void rtl_transaction_kernel(RtlArgs a) {
    __shared__ uint32_t o_lds[D][kLanes];   // O accumulator, one column per lane
    __shared__ uint32_t s_lds[16][kLanes];  // scaled scores of the current sub-block

    const int lane = threadIdx.x;
    const int r = blockIdx.x * kLanes + lane;  // query row within the transaction
    const int hq = blockIdx.y;
    if (r >= a.q_len) return;  // no barriers below: lanes only touch their own LDS columns
    const int G = a.n_q_heads / a.n_kv_heads;
    const int hk = hq / G;
    const uint16_t* kb = a.kc + (size_t)hk * a.l_cap * D;
    const uint16_t* vb = a.vc + (size_t)hk * a.l_cap * D;

    uint32_t qw[D / 2];
    {
        const uint32_t* qp = reinterpret_cast<const uint32_t*>(a.q + ((size_t)hq * a.q_len + r) * D);
#pragma unroll
        for (int i = 0; i < D / 2; ++i) qw[i] = qp[i];
    }

    // Tile walk of the row's 32-row Q tile.
    const int t = r / 32;
    const int rows = min(32, a.q_len - 32 * t);
    const int q_end = a.q_pos_base + 32 * t + rows - 1;
    const int n_kv_tiles = (a.kv_len + 63) / 64;
    int last_tile = n_kv_tiles - 1;
    if (a.causal) last_tile = q_end < a.kv_pos_base ? 0 : min((q_end - a.kv_pos_base) / 64, n_kv_tiles - 1);
    const int q_pos = a.q_pos_base + r;

    for (int d = 0; d < D; ++d) o_lds[d][lane] = 0u;
    uint32_t m = kNegInf, l = 0u;
    bool first = true;
    for (int jt = 0; jt <= last_tile; ++jt) {
        for (int sb = 0; sb < 4; ++sb) {
            const int c0 = jt * 64 + sb * 16;
            if (c0 >= a.kv_len) break;
            uint32_t row_max = kNegInf;
            uint32_t live = 0u;  // bit c: key c0 + c is attended
            for (int c = 0; c < 16; ++c) {
                const int key = c0 + c;
                const bool ok = key < a.kv_len && !(a.causal && q_pos < a.kv_pos_base + key);
                uint32_t val = kNegInf;
                if (ok) {
                    const uint32_t* kr = reinterpret_cast<const uint32_t*>(kb + (size_t)key * D);
                    uint32_t acc = 0u;
#pragma unroll
                    for (int i = 0; i < D / 2; ++i) {
                        const uint32_t kw = kr[i];
                        acc = add(acc, bmul(qw[i] & 0xFFFFu, kw & 0xFFFFu));
                        acc = add(acc, bmul(qw[i] >> 16, kw >> 16));
                    }
                    val = mul(acc, a.scale_bits);
                    live |= 1u << c;
                }
                s_lds[c][lane] = val;
                row_max = mx(row_max, val);
            }
            const uint32_t m_old = first ? kNegInf : m;
            const uint32_t m_new = mx(m_old, row_max);
            const uint32_t corr = first ? 0u : exp_table(sub(m_old, m_new));
            uint32_t row_sum = 0u;
            uint32_t p16[16];
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const uint32_t p = ((live >> c) & 1u) ? exp_table(sub(s_lds[c][lane], m_new)) : 0u;
                row_sum = add(row_sum, p);
                p16[c] = p >> 16;  // the PV product takes the upper half of p (truncation)
            }
            l = first ? row_sum : add(mul(l, corr), row_sum);
            m = m_new;
            for (int d = 0; d < D; ++d) {
                uint32_t delta = 0u;
#pragma unroll
                for (int c = 0; c < 16; ++c) {
                    const int key = c0 + c;
                    const uint32_t vw = key < a.kv_len ? vb[(size_t)key * D + d] : 0u;
                    delta = add(delta, bmul(p16[c], vw));
                }
                o_lds[d][lane] = add(mul(o_lds[d][lane], corr), delta);
            }
            first = false;
        }
    }

    uint16_t* orow = a.out + ((size_t)hq * a.q_len + r) * D;
    const uint32_t rl = recip_table(l);
    for (int d = 0; d < D; d += 2) {
        const uint32_t w0 = zero_b(l) ? 0u : to_bf16(mul(o_lds[d][lane], rl));
        const uint32_t w1 = zero_b(l) ? 0u : to_bf16(mul(o_lds[d + 1][lane], rl));
        *reinterpret_cast<uint32_t*>(orow + d) = w0 | (w1 << 16);
    }
    if (a.lse != nullptr) {
        // natural-log LSE of the board's (m, l): m is in scaled-score units
        a.lse[(size_t)hq * a.q_len + r] = zero_b(l) ? -INFINITY : f_(m) + logf(f_(l));
    }
}

}  // namespace

hipError_t launch_rtl_transaction(int head_dim, const RtlArgs& a, const Launch& l) {
    dim3 grid((a.q_len + kLanes - 1) / kLanes, a.n_q_heads);
    if (head_dim == 128) return launch_kernel(rtl_transaction_kernel<128>, grid, dim3(kLanes), l, a);
    if (head_dim == 64) return launch_kernel(rtl_transaction_kernel<64>, grid, dim3(kLanes), l, a);
    return hipErrorInvalidValue;
}

}  // namespace lara
