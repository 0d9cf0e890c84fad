/*
 * rtl_exact.c -- CPU restatement of the KV260 datapath's bit-level arithmetic (TEST INFRASTRUCTURE).
 *
 * Only tests/ (through ctypes) use this library, as the oracle of the engine's RTL-exact
 * numerics mode; the product never links or loads it.
 *
 * It restates, bit for bit, the synthesis path of the reference RTL (paths relative to the
 * reference repository):
 *   fp32_gt / fp32_max ................. hw/rtl/pkg/attn_pkg.sv:357-368
 *   fp32_add (56-bit align + sticky, RNE, lz capped at 24)   attn_pkg.sv:371-496
 *   fp32_mul (RNE, 8-bit exponent wrap) .. attn_pkg.sv:502-544
 *   bf16_mul_to_fp32 (exact, bf16 exponent 0 -> 0) attn_pkg.sv:546-597
 *   fp32_to_bf16 (RNE, no NaN case) ....... attn_pkg.sv:618-626
 *   fp32_to_q8_23, q26_to_fp32, exp LUT interpolation (quantize/index/finish stages)
 *                                       hw/rtl/core/softmax_engine.sv:523-567, 570-706
 *   online softmax per 16x16 sub-block (scale, mask, row max, correction, p, row sum, l)
 *                                       softmax_engine.sv:826-1334
 *   P -> PV input as the upper 16 bits of the fp32 word (truncation) attn_top.sv:653-658
 *   O = O*corr + dO per sub-block; normalise with the reciprocal LUT; bf16 RNE
 *                                       hw/rtl/mem/output_buffer.sv:192-286, 873-885
 *   tile walk (32-row Q tiles, 64-key KV tiles of four 16-key sub-blocks, causal KV-tile
 *   limit, first sub-block of the first KV tile) hw/rtl/core/attn_core.sv:107-154,
 *   hw/rtl/attn_top.sv:785
 *
 * Pinning: the LUT tables against their closed forms and the board ROM images' SHA-256, the exp
 * lookup at its 1024 knots and across every index boundary, the reciprocal lookup at powers of
 * two and at its 256 bin centres; fp32_add / fp32_mul against IEEE float32 (numpy) on normal
 * operands, where the RTL's rounding is IEEE round-to-nearest-even; hand-derived special cases.
 * The composition (P truncated to its upper half, key-0-first sums, one O delta and one rescale
 * per 16-key sub-block, the R(l) normalise, dimension-0-first Q.K, the exp interpolation fraction
 * truncated to 24 significant bits) is pinned word for word by
 * constructed transactions whose words follow from a few float32 operations and differ under
 * each alternative; rtl_attention_planted applies those alternatives so the tests can show that
 * each is rejected.  Whole transactions are also held to the float64 exact model within the
 * LUT's and the truncated P's error, and to the known answers of one key (output = V exactly)
 * and zero input (output +0).  No board vector exists in the reference snapshot, so agreement
 * with the board itself is not pinned.
 * Parity unpinned: the corners where the RTL departs from IEEE (subnormal operands or
 * results, the leading-zero cap of fp32_add, the 8-bit exponent wrap of fp32_mul) follow the
 * RTL source alone; no independent check covers them.
 */
#include <stdint.h>
#include <string.h>

#define NAN_BITS 0x7FC00000u
#define NEG_INF_BITS 0xFF800000u
#define ONE_BITS 0x3F800000u
#define NEG_EIGHT_BITS 0xC1000000u

static int is_zero(uint32_t a) { return (a & 0x7FFFFFFFu) == 0; }
static int is_inf(uint32_t a) { return ((a >> 23) & 0xFF) == 0xFF && (a & 0x7FFFFF) == 0; }
static int is_nan(uint32_t a) { return ((a >> 23) & 0xFF) == 0xFF && (a & 0x7FFFFF) != 0; }

int rtl_fp32_gt(uint32_t a, uint32_t b) {
    if (a == b) return 0;
    if ((a >> 31) != (b >> 31)) return (int)(b >> 31);
    if (!(a >> 31)) return (a & 0x7FFFFFFFu) > (b & 0x7FFFFFFFu);
    return (a & 0x7FFFFFFFu) < (b & 0x7FFFFFFFu);
}

uint32_t rtl_fp32_max(uint32_t a, uint32_t b) { return rtl_fp32_gt(a, b) ? a : b; }

static int lzd8(uint32_t v) {
    for (int i = 7; i >= 0; --i)
        if (v & (1u << i)) return 7 - i;
    return 8;
}

/* leading zeros of a 56-bit value, looked for only in bits 55..32 (24 at most) */
static int lzd24(uint64_t v) {
    if ((v >> 48) & 0xFF) return lzd8((uint32_t)(v >> 48) & 0xFF);
    if ((v >> 40) & 0xFF) return 8 + lzd8((uint32_t)(v >> 40) & 0xFF);
    if ((v >> 32) & 0xFF) return 16 + lzd8((uint32_t)(v >> 32) & 0xFF);
    return 24;
}

uint32_t rtl_fp32_add(uint32_t a, uint32_t b) {
    const uint64_t M56 = (1ull << 56) - 1;
    if (is_nan(a) || is_nan(b)) return NAN_BITS;
    if (is_zero(a)) return b;
    if (is_zero(b)) return a;
    uint32_t sa = a >> 31, sb = b >> 31;
    uint32_t ea = (a >> 23) & 0xFF, eb = (b >> 23) & 0xFF;
    uint32_t ma = ea ? (0x800000u | (a & 0x7FFFFF)) : (a & 0x7FFFFF);
    uint32_t mb = eb ? (0x800000u | (b & 0x7FFFFF)) : (b & 0x7FFFFF);
    if (ea == 0) ea = 1;
    if (eb == 0) eb = 1;
    int a_larger = (ea > eb) || (ea == eb && ma >= mb);
    uint32_t e_large = a_larger ? ea : eb;
    uint64_t m_large = (uint64_t)(a_larger ? ma : mb) << 32;
    uint64_t m_small = (uint64_t)(a_larger ? mb : ma) << 32;
    uint32_t s_large = a_larger ? sa : sb;
    int eff_sub = (int)(sa ^ sb);
    int shift = a_larger ? (int)ea - (int)eb : (int)eb - (int)ea;
    uint64_t sticky_mask = shift <= 0 ? 0 : (shift >= 56 ? M56 : (M56 >> (56 - shift)));
    int sticky = (m_small & sticky_mask) != 0;
    uint64_t m_small_sh;
    if (shift >= 56) {
        m_small_sh = sticky ? 1 : 0;
    } else {
        m_small_sh = m_small >> shift;
        if (sticky) m_small_sh |= 1;
    }
    uint64_t sum = eff_sub ? (m_large - m_small_sh) : (m_large + m_small_sh); /* 57 bits */
    if (sum == 0) return 0;
    uint32_t e_res;
    uint64_t norm;
    if ((sum >> 56) & 1) {
        e_res = (e_large + 1) & 0xFF;
        norm = (sum >> 1) & M56;
        if (sum & 1) norm |= 1;
    } else {
        int lz = lzd24(sum & M56);
        norm = (sum << lz) & M56;
        e_res = (e_large - (uint32_t)lz) & 0xFF;
    }
    uint32_t keep = (uint32_t)(norm >> 32) & 0xFFFFFF;
    int guard = (int)((norm >> 31) & 1);
    int rnd = (int)((norm >> 30) & 1);
    int st = (norm & ((1ull << 30) - 1)) != 0;
    int up = guard && (rnd || st || (keep & 1));
    uint32_t mr = keep + (uint32_t)up; /* 25 bits */
    uint32_t frac;
    if ((mr >> 24) & 1) {
        e_res = (e_res + 1) & 0xFF;
        frac = 0;
    } else {
        frac = mr & 0x7FFFFF;
    }
    return (s_large << 31) | (e_res << 23) | frac;
}

uint32_t rtl_fp32_sub(uint32_t a, uint32_t b) { return rtl_fp32_add(a, b ^ 0x80000000u); }

uint32_t rtl_fp32_mul(uint32_t a, uint32_t b) {
    if (is_nan(a) || is_nan(b)) return NAN_BITS;
    uint32_t sp = (a ^ b) & 0x80000000u;
    if (is_zero(a) || is_zero(b)) return sp;
    if (is_inf(a) || is_inf(b)) return sp | 0x7F800000u;
    uint32_t ea = (a >> 23) & 0xFF, eb = (b >> 23) & 0xFF;
    uint64_t ma = 0x800000u | (a & 0x7FFFFF), mb = 0x800000u | (b & 0x7FFFFF);
    uint64_t prod = ma * mb; /* 48 bits */
    uint32_t ep, keep;
    int guard, rnd, st;
    if ((prod >> 47) & 1) {
        ep = (ea + eb - 126) & 0xFF;
        keep = 0x800000u | ((uint32_t)(prod >> 24) & 0x7FFFFF);
        guard = (int)((prod >> 23) & 1);
        rnd = (int)((prod >> 22) & 1);
        st = (prod & ((1ull << 22) - 1)) != 0;
    } else {
        ep = (ea + eb - 127) & 0xFF;
        keep = 0x800000u | ((uint32_t)(prod >> 23) & 0x7FFFFF);
        guard = (int)((prod >> 22) & 1);
        rnd = (int)((prod >> 21) & 1);
        st = (prod & ((1ull << 21) - 1)) != 0;
    }
    int up = guard && (rnd || st || (keep & 1));
    uint32_t mr = keep + (uint32_t)up;
    if ((mr >> 24) & 1) {
        ep = (ep + 1) & 0xFF;
        mr = 1u << 23;
    }
    return sp | (ep << 23) | (mr & 0x7FFFFF);
}

uint32_t rtl_bf16_mul(uint16_t a, uint16_t b) {
    uint32_t sp = ((uint32_t)(a ^ b) & 0x8000u) << 16;
    uint32_t ea = (a >> 7) & 0xFF, eb = (b >> 7) & 0xFF;
    uint32_t fa = a & 0x7F, fb = b & 0x7F;
    int a_zero = ea == 0, b_zero = eb == 0;
    int a_inf = ea == 0xFF && fa == 0, b_inf = eb == 0xFF && fb == 0;
    int a_nan = ea == 0xFF && fa != 0, b_nan = eb == 0xFF && fb != 0;
    if (a_nan || b_nan) return NAN_BITS;
    if ((a_inf && b_zero) || (a_zero && b_inf)) return NAN_BITS;
    if (a_inf || b_inf) return sp | 0x7F800000u;
    if (a_zero || b_zero) return sp;
    uint32_t prod = (0x80u | fa) * (0x80u | fb); /* 16 bits */
    uint32_t e_prod = (ea + eb - 127) & 0x1FF;
    uint32_t e_norm, mant;
    if ((prod >> 15) & 1) {
        e_norm = (e_prod + 1) & 0xFF;
        mant = (prod & 0x7FFF) << 8;
    } else {
        e_norm = e_prod & 0xFF;
        mant = (prod & 0x3FFF) << 9;
    }
    return sp | (e_norm << 23) | mant;
}

uint16_t rtl_fp32_to_bf16(uint32_t a) {
    uint32_t upper = a >> 16;
    int up = ((a >> 15) & 1) && ((a & 0x7FFF) || (upper & 1));
    return (uint16_t)((upper + (uint32_t)up) & 0xFFFF);
}

static int64_t fp32_to_q8_23(uint32_t v) {
    if (is_zero(v)) return 0;
    int e = (int)((v >> 23) & 0xFF) - 127;
    int64_t m = 0x800000 | (v & 0x7FFFFF);
    int64_t s = e >= 0 ? (m << e) : (e < -40 ? 0 : (m >> (-e)));
    return (v >> 31) ? -s : s;
}

static uint32_t q26_to_fp32(int64_t value) {
    if (value <= 0) return 0;
    int bit = 25;
    while (bit > 0 && !((value >> bit) & 1)) --bit;
    int64_t residual = value - ((int64_t)1 << bit);
    uint32_t mant = bit < 23 ? (uint32_t)(residual << (23 - bit)) : (uint32_t)(residual >> (bit - 23));
    uint32_t e = (uint32_t)(127 + bit - 26);
    return ((e & 0xFF) << 23) | (mant & 0x7FFFFF);
}

/* The same conversion rounded to nearest even instead of truncated (only for the planted mistake
 * PLANT_FRAC_RNE below): what a conversion written with an ordinary int-to-float cast would give. */
static uint32_t q26_to_fp32_rne(int64_t value) {
    float f = (float)((double)value / 67108864.0);
    uint32_t r;
    memcpy(&r, &f, 4);
    return r;
}

static uint32_t exp_lookup_impl(uint32_t x, const uint32_t* lut, int round_fraction) {
    if (rtl_fp32_gt(NEG_EIGHT_BITS, x)) return 0;
    if (rtl_fp32_gt(x, 0)) return ONE_BITS;
    int64_t xq = fp32_to_q8_23(x);
    int64_t n = xq + 67108864;
    if (n < 0) n = 0;
    if (n > 67108864) n = 67108864;
    int64_t num = (n << 10) - n;
    int64_t idx = num >> 26;
    int64_t rem = num - (idx << 26);
    if (idx >= 1023) return lut[1023];
    uint32_t frac = round_fraction ? q26_to_fp32_rne(rem) : q26_to_fp32(rem);
    uint32_t lo = lut[idx], hi = lut[idx + 1];
    return rtl_fp32_add(lo, rtl_fp32_mul(rtl_fp32_sub(hi, lo), frac));
}

uint32_t rtl_exp_lookup(uint32_t x, const uint32_t* lut) { return exp_lookup_impl(x, lut, 0); }

uint32_t rtl_recip_lookup(uint32_t l, const uint32_t* recip_lut) {
    uint32_t s = l & 0x80000000u, e = (l >> 23) & 0xFF, f = l & 0x7FFFFF;
    if (is_nan(l)) return NAN_BITS;
    if (is_zero(l)) return s | 0x7F800000u;
    if (is_inf(l)) return s;
    if (f == 0) return s | (((254 - e) & 0xFF) << 23);
    return s | (((253 - e) & 0xFF) << 23) | (recip_lut[f >> 15] & 0x7FFFFF);
}

/* Mistakes planted on purpose (test infrastructure): each flag swaps one composition step for a
 * plausible alternative, so the tests can show that their word-level checks reject it. */
enum {
    PLANT_P_RNE = 1,            /* P rounded to bf16 to nearest even instead of truncated       */
    PLANT_SUM_REVERSED = 2,     /* row sum and PV sum of a sub-block taken from key 15 down     */
    PLANT_FLAT_ACCUMULATE = 4,  /* O accumulated key by key instead of one delta per sub-block  */
    PLANT_TILE_RESCALE = 8,     /* running max taken per 64-key tile instead of per sub-block   */
    PLANT_EXACT_DIVIDE = 16,    /* O divided by l (IEEE) instead of multiplied by R(l)          */
    PLANT_QK_REVERSED = 32,     /* Q.K summed from the last dimension down                      */
    PLANT_FRAC_RNE = 64,        /* exp interpolation fraction rounded to nearest, not truncated */
};

static uint32_t exp_planted(uint32_t x, const uint32_t* lut, int plant) {
    return exp_lookup_impl(x, lut, plant & PLANT_FRAC_RNE);
}

static uint32_t f32_div_bits(uint32_t a, uint32_t b) {
    float x, y;
    memcpy(&x, &a, 4);
    memcpy(&y, &b, 4);
    x = x / y;
    uint32_t r;
    memcpy(&r, &x, 4);
    return r;
}

/* Scaled score of one key (hw/rtl/core/attn_tile.sv: sequential fp32 sum over d, then x scale),
 * or -inf for a key that is masked or past the sequence. */
static uint32_t key_score(const uint16_t* qr, const uint16_t* kr, int D, int live, uint32_t scale_bits, int plant) {
    if (!live) return NEG_INF_BITS;
    uint32_t acc = 0;
    if (plant & PLANT_QK_REVERSED)
        for (int d = D - 1; d >= 0; --d) acc = rtl_fp32_add(acc, rtl_bf16_mul(qr[d], kr[d]));
    else
        for (int d = 0; d < D; ++d) acc = rtl_fp32_add(acc, rtl_bf16_mul(qr[d], kr[d]));
    return rtl_fp32_mul(acc, scale_bits);
}

static void attention_impl(const uint16_t* q, const uint16_t* k, const uint16_t* v, int n_q_heads, int n_kv_heads,
                           int head_dim, int seq_len, int q_pos_base, int kv_pos_base, int causal,
                           uint32_t scale_bits, const uint32_t* exp_lut, const uint32_t* recip_lut, uint16_t* out,
                           uint32_t* m_out, uint32_t* l_out, int plant) {
    const int D = head_dim, L = seq_len, G = n_q_heads / n_kv_heads;
    const int n_kv_tiles = (L + 63) / 64;
    uint32_t O[512];
    uint32_t s[16], p[16];
    for (int hq = 0; hq < n_q_heads; ++hq) {
        const int hk = hq / G;
        for (int r = 0; r < L; ++r) {
            /* the row's Q tile decides which KV tiles the transaction visits (attn_core.sv:138-154) */
            const int t = r / 32;
            const int rows = (L - t * 32) < 32 ? (L - t * 32) : 32;
            const int q_end = q_pos_base + t * 32 + rows - 1;
            int last_tile = n_kv_tiles - 1;
            if (causal) {
                last_tile = q_end < kv_pos_base ? 0 : (q_end - kv_pos_base) / 64;
                if (last_tile > n_kv_tiles - 1) last_tile = n_kv_tiles - 1;
            }
            const int q_pos = q_pos_base + r;
            const uint16_t* qr = q + ((size_t)hq * L + r) * D;
            uint32_t m = NEG_INF_BITS, l = 0;
            for (int d = 0; d < D; ++d) O[d] = 0;
            int first = 1;
            for (int jt = 0; jt <= last_tile; ++jt) {
                uint32_t tile_max = NEG_INF_BITS;
                if (plant & PLANT_TILE_RESCALE)
                    for (int key = jt * 64; key < jt * 64 + 64 && key < L; ++key)
                        tile_max = rtl_fp32_max(tile_max, key_score(qr, k + ((size_t)hk * L + key) * D, D,
                                                                    !(causal && q_pos < kv_pos_base + key),
                                                                    scale_bits, plant));
                for (int sb = 0; sb < 4; ++sb) {
                    const int c0 = jt * 64 + sb * 16;
                    if (c0 >= L) break; /* sub-blocks past the sequence are not issued */
                    uint32_t row_max = tile_max;
                    int masked[16];
                    for (int c = 0; c < 16; ++c) {
                        const int key = c0 + c;
                        masked[c] = key >= L || (causal && q_pos < kv_pos_base + key);
                        s[c] = key < L ? key_score(qr, k + ((size_t)hk * L + key) * D, D, !masked[c], scale_bits,
                                                   plant)
                                       : NEG_INF_BITS;
                        row_max = rtl_fp32_max(row_max, s[c]);
                    }
                    const uint32_t m_old = first ? NEG_INF_BITS : m;
                    const uint32_t l_old = first ? 0u : l;
                    const uint32_t m_new = rtl_fp32_max(m_old, row_max);
                    const uint32_t corr = first ? 0u : exp_planted(rtl_fp32_sub(m_old, m_new), exp_lut, plant);
                    uint32_t row_sum = 0;
                    for (int c = 0; c < 16; ++c)
                        p[c] = masked[c] ? 0u : exp_planted(rtl_fp32_sub(s[c], m_new), exp_lut, plant);
                    for (int i = 0; i < 16; ++i) row_sum = rtl_fp32_add(row_sum, p[plant & PLANT_SUM_REVERSED ? 15 - i : i]);
                    l = first ? row_sum : rtl_fp32_add(rtl_fp32_mul(l_old, corr), row_sum);
                    m = m_new;
                    /* the PV operand is the upper half of the fp32 P word (attn_top.sv:653-658) */
                    uint16_t pv[16];
                    for (int c = 0; c < 16; ++c)
                        pv[c] = (plant & PLANT_P_RNE) ? rtl_fp32_to_bf16(p[c]) : (uint16_t)(p[c] >> 16);
                    for (int d = 0; d < D; ++d) {
                        if (plant & PLANT_FLAT_ACCUMULATE) {
                            uint32_t o = rtl_fp32_mul(O[d], corr);
                            for (int c = 0; c < 16; ++c) {
                                const int key = c0 + c;
                                const uint16_t vw = key < L ? v[((size_t)hk * L + key) * D + d] : 0;
                                o = rtl_fp32_add(o, rtl_bf16_mul(pv[c], vw));
                            }
                            O[d] = o;
                            continue;
                        }
                        uint32_t delta = 0;
                        for (int i = 0; i < 16; ++i) {
                            const int c = plant & PLANT_SUM_REVERSED ? 15 - i : i;
                            const int key = c0 + c;
                            const uint16_t vw = key < L ? v[((size_t)hk * L + key) * D + d] : 0;
                            delta = rtl_fp32_add(delta, rtl_bf16_mul(pv[c], vw));
                        }
                        O[d] = rtl_fp32_add(rtl_fp32_mul(O[d], corr), delta);
                    }
                    first = 0;
                }
            }
            uint16_t* orow = out + ((size_t)hq * L + r) * D;
            const uint32_t rl = rtl_recip_lookup(l, recip_lut);
            for (int d = 0; d < D; ++d) {
                const uint32_t o = (plant & PLANT_EXACT_DIVIDE) ? f32_div_bits(O[d], l) : rtl_fp32_mul(O[d], rl);
                orow[d] = is_zero(l) ? 0 : rtl_fp32_to_bf16(o);
            }
            if (m_out) m_out[(size_t)hq * L + r] = m;
            if (l_out) l_out[(size_t)hq * L + r] = l;
        }
    }
}

/*
 * One KV260 transaction: q [H_q][L][D], k/v [H_kv][L][D] bf16 words, query head h reads kv
 * head h / (H_q / H_kv).  Writes out [H_q][L][D] bf16 words and, if non-NULL, the final
 * running max m (scaled-score units) and sum l of every row as fp32 bits.
 */
void rtl_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int n_q_heads, int n_kv_heads,
                   int head_dim, int seq_len, int q_pos_base, int kv_pos_base, int causal, uint32_t scale_bits,
                   const uint32_t* exp_lut, const uint32_t* recip_lut, uint16_t* out, uint32_t* m_out,
                   uint32_t* l_out) {
    attention_impl(q, k, v, n_q_heads, n_kv_heads, head_dim, seq_len, q_pos_base, kv_pos_base, causal, scale_bits,
                   exp_lut, recip_lut, out, m_out, l_out, 0);
}

/* The same transaction with the PLANT_* mistakes of `plant` applied (tests only). */
void rtl_attention_planted(const uint16_t* q, const uint16_t* k, const uint16_t* v, int n_q_heads, int n_kv_heads,
                           int head_dim, int seq_len, int q_pos_base, int kv_pos_base, int causal,
                           uint32_t scale_bits, const uint32_t* exp_lut, const uint32_t* recip_lut, uint16_t* out,
                           uint32_t* m_out, uint32_t* l_out, int plant) {
    attention_impl(q, k, v, n_q_heads, n_kv_heads, head_dim, seq_len, q_pos_base, kv_pos_base, causal, scale_bits,
                   exp_lut, recip_lut, out, m_out, l_out, plant);
}

/* Element-wise batch forms, for the checks that sweep many operands through ctypes. */
void rtl_fp32_add_n(const uint32_t* a, const uint32_t* b, uint32_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = rtl_fp32_add(a[i], b[i]);
}
void rtl_fp32_mul_n(const uint32_t* a, const uint32_t* b, uint32_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = rtl_fp32_mul(a[i], b[i]);
}
void rtl_bf16_mul_n(const uint16_t* a, const uint16_t* b, uint32_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = rtl_bf16_mul(a[i], b[i]);
}
void rtl_exp_lookup_n(const uint32_t* x, const uint32_t* lut, uint32_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = rtl_exp_lookup(x[i], lut);
}
void rtl_recip_lookup_n(const uint32_t* x, const uint32_t* lut, uint32_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = rtl_recip_lookup(x[i], lut);
}
