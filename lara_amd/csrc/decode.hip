// Split-KV GQA decode (flash-decoding) for CDNA4 / gfx950.
//
// Arithmetic contract (what the KV260 datapath computes, restated for one query row):
//   s_k   = scale * sum_d q[d] * k_k[d]          (attn_tile.sv:176-248, attn_pkg.sv:241)
//   p_k   = exp(s_k - m),  m = running max         (softmax_engine.sv:858-1073)
//   O     = sum_k p_k v_k,  l = sum_k p_k            (attn_top.sv:462-625, output_buffer.sv:226-269)
//   out   = bf16_rne(O / l), 0 when no key is valid (output_buffer.sv:271-286, attn_pkg.sv:618-626)
// The KV260 works on 16-key sub-blocks of one Q tile at a time; here one work-group of
// NW waves owns a contiguous chunk of keys of one (sequence, kv head) -- a "split" --
// for all G query heads of the GQA group, so every K/V byte is read from HBM once.
//
// Work decomposition inside a work-group: keys are taken in rounds of 16 rows; wave w owns
// rounds w, w+NW, ...  Per round a wave has the round's K and V rows in registers (coalesced
// 16-byte loads, 1 KiB per wave instruction) and prefetches the next round's rows behind the
// math; the products run on the matrix cores: K and V go to two wave-private LDS tiles;
// S^T [16 keys x 16 heads] = K . Q^T is D/32 v_mfma_f32_16x16x32_bf16 with K read as operand A
// and Q^T held in registers (heads past G are zero); its result leaves lane l the scores of keys
// 4(l/16) .. +3 of head l % 16, so the online softmax (log2 domain, v_exp_f32, the running max
// moved only when a score passes it by 2^8) runs per lane, and its p values are exactly the B
// operand of P^T, rounded to bf16 as on the board (attn_top.sv:653-658); O^T [D x 16] +=
// V^T . P^T is D/16 v_mfma_f32_16x16x16_bf16 with V^T read by the transposing LDS read
// (ds_read_b64_tr_b16).  l sums the fp32 p.  (A VALU form -- v_dot2 dot products over a
// transposed K tile, FMAs for PV -- bounded the kernel at G = 8 and streamed slower at G = 4.)
// At the end the waves merge in LDS.  A sequence that fits in one split writes the
// bf16 output directly; otherwise each split writes an fp32 partial (O, m, l) and the
// splits merge with log-sum-exp weights: inside the launch, by the last split of the
// (sequence, kv head) to arrive (an agent-scope release per split: an L2 write-back of its
// XCD, worth it while the split grid is small and the step short, as for one short sequence), or
// by decode_combine_kernel, a second launch (larger grids, whose write-backs slow the other
// splits' streaming more than the launch costs).
//
// Fused append: when k_new/v_new are given, split 0 of every (sequence, kv head) writes
// the new row to cache row positions[b], and any split whose key range contains that row
// reads it from k_new/v_new instead of the cache, so no split depends on the write.
//
// K/V rows are streamed with nontemporal loads: they are read once per launch and should not
// displace anything from the L2 / Infinity Cache; that streams HBM fastest (7.09 TB/s for 4 GiB
// against 6.28 with plain loads, measured).  A launch whose K/V fit the XCDs' L2s several times over
// (DecodeArgs::cached) uses plain loads instead: a work-group reads the same rows each step on the
// same XCD, whose L2 still holds them from the last launch (16 MiB read back to back: 2.42 us per
// launch plain vs 2.99 nontemporal; 32 MiB: 2.85 vs 5.58).
#include "gqa_internal.h"

#include <math.h>

namespace lara {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr float kLn2 = 0.693147180559945309f;

// Lazy rescaling: the running max a wave's p values are taken against moves only when a
// score exceeds it by more than this (log2 units), so p <= 2^8 and most rounds skip the
// rescale of O.  The result is the same softmax; only fp32 rounding differs.
constexpr float kRescaleSlack = 8.0f;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};  // v_cvt_pk_bf16_f32, round to nearest even
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Orders a wave's LDS writes before its subsequent LDS reads of other lanes' data.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Matrix-core products of the decode rounds.  16x16 outputs: register i of lane l holds row
// 4*(l/16) + i, column l % 16; operand A row / operand B column l % 16 with the k-values
// KPL*(l/16) .. KPL*(l/16) + KPL-1 (KPL = 8 for k = 32, 4 for k = 16).
__device__ __forceinline__ f32x4 mfma_16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x16(const u32x2& a, const u32x2& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, a), __builtin_bit_cast(bf16x4_t, b),
                                                     c, 0, 0, 0);
}
// Transposing LDS read: lane i of each 16-lane group receives element i % 4 of the 8-byte piece
// addressed by lane 4j + i/4 of its group, for j = 0..3.
__device__ __forceinline__ u32x2 lds_read_tr16(const void* p) {
    typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
    const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
    return __builtin_bit_cast(u32x2, v);
}

// LDS swizzles of the round tiles (16 rows of D bf16).  K: the A-operand read covers rows 0..15
// at one 16-byte chunk per 16 lanes, so the chunk is XORed with the row's position inside a
// 256-byte bank period (D = 128: rows are 256 B; D = 64: two rows per period).  V: a transposing
// read covers 8 keys per half-wave at one 32-byte run, so the run is XORed likewise.
template <int D>
__device__ __forceinline__ int mf_kswz(int row) {
    return D == 128 ? (row & 15) : ((row >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int mf_vswz(int row) {
    return D == 128 ? (row & 7) : ((row >> 1) & 3);
}

__device__ __forceinline__ int clamp_len(int len, int l_max) {
    return len < 0 ? 0 : (len > l_max ? l_max : len);
}

template <bool CACHED>
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
    if constexpr (CACHED) return *p;
    else return __builtin_nontemporal_load(p);
}

// The sequence of rank `rank` when the batch is ordered longest first.  Every wave computes it
// for itself from the lengths (no LDS, no barrier); a batch of equal lengths keeps index order.
//  * Up to 64 sequences (one per lane): exact -- by attended length, ties in index order (a wave
//    min/max, then a batch-long loop of lane reads).
//  * More: by length bucket (kBuckets equal slices of 0..l_max), longest bucket first, index
//    order inside a bucket -- a histogram of ballots over 64-sequence chunks, then the rank's
//    bucket and its position among that bucket's members.
constexpr int kBuckets = 16;

__device__ __forceinline__ int length_bucket(const DecodeArgs& a, int s) {
    const int L = clamp_len(a.lens[s], a.l_max);
    return (int)(((int64_t)L * kBuckets) / ((int64_t)a.l_max + 1));
}

// Whether the batch's attended lengths differ (every lane of the wave gets the same answer).
__device__ bool batch_is_ragged(const DecodeArgs& a) {
    const int lane = threadIdx.x & 63;
    int lo = INT_MAX, hi = -1;
    for (int s = lane; s < a.batch; s += 64) {
        const int L = clamp_len(a.lens[s], a.l_max);
        lo = L < lo ? L : lo;
        hi = L > hi ? L : hi;
    }
    return __reduce_min_sync(~0ull, lo) != __reduce_max_sync(~0ull, hi);
}

__device__ int rank_to_sequence(const DecodeArgs& a, int rank) {
    const int lane = threadIdx.x & 63;
    if (a.batch <= 64) {
        const int mine = lane < a.batch ? clamp_len(a.lens[lane], a.l_max) : -1;
        const int lo = __reduce_min_sync(~0ull, lane < a.batch ? mine : INT_MAX);
        const int hi = __reduce_max_sync(~0ull, mine);
        if (lo == hi) return rank;
        int before = 0;  // sequences ordered ahead of this lane's
        for (int j = 0; j < a.batch; ++j) {
            const int other = __builtin_amdgcn_readlane(mine, j);
            before += (other > mine) || (other == mine && j < lane);
        }
        const unsigned long long hit = __ballot(lane < a.batch && before == rank);
        return hit ? (int)__builtin_ctzll(hit) : rank;
    }
    // Bucket histogram (wave-uniform counts).
    int count[kBuckets];
#pragma unroll
    for (int k = 0; k < kBuckets; ++k) count[k] = 0;
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
        const int s = c0 + lane;
        const int kb = s < a.batch ? length_bucket(a, s) : -1;
#pragma unroll
        for (int k = 0; k < kBuckets; ++k) count[k] += __popcll(__ballot(kb == k));
    }
    // The rank's bucket (longest first) and its position among the bucket's members.
    int want = -1, pos = rank;
#pragma unroll
    for (int k = kBuckets - 1; k >= 0; --k) {
        if (want < 0) {
            if (pos < count[k]) want = k;
            else pos -= count[k];
        }
    }
    if (want < 0) return rank;  // rank outside the batch: not reached for grid rows < batch
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
        const int s = c0 + lane;
        const bool member = s < a.batch && length_bucket(a, s) == want;
        const unsigned long long m = __ballot(member);
        const int n = __popcll(m);
        if (pos < n) {
            // the member lane with `pos` members below it
            const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
            const unsigned long long hit = __ballot(member && below == pos);
            return c0 + (int)__builtin_ctzll(hit);
        }
        pos -= n;
    }
    return rank;
}

// Log-sum-exp merge of the split partials of one (sequence, kv head), split-parallel, for its
// GH heads g0 .. g0 + GH - 1: wave w folds splits w, w + NW, ... with lane e (and e + 64, ...)
// owning 8 consecutive dims of one head (16-byte loads of the partial O, one 8-byte load of
// (m, l)), kMergeBatch splits per memory round trip; then the waves' (M, O, l) fold through LDS
// and thread (g, d) writes the output.  Every (head, 8 dims) entry folds the same splits in the
// same order whichever lane holds it and however many heads a work-group takes, so the split
// kernel's fused merge (the last split to arrive merges all G heads, after its acquire of the
// other splits' partials, reusing the LDS of its own wave merge) and decode_combine_kernel (one
// work-group per head) give the same words.
constexpr int kMergeBatch = 4;

template <int D, int G, int NW, int GH>
__device__ __forceinline__ void merge_splits_parallel(const DecodeArgs& a, int unit, int b, int h, int n_splits,
                                                      int g0, float (*lds_o)[GH][D], float (*lds_m)[GH],
                                                      float (*lds_l)[GH]) {
    constexpr int E = GH * D / 8;              // 8-dim entries of the heads' output
    constexpr int EPL = (E + 63) / 64;         // entries per lane
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float4* po = reinterpret_cast<const float4*>(a.part_o);
    const float2* pml = reinterpret_cast<const float2*>(a.part_ml);
    const size_t base = (size_t)unit * a.max_splits * G;  // partial row of (split 0, head 0)
    float M[EPL], L[EPL], O[EPL][8];
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
        M[k] = -INFINITY;
        L[k] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) O[k][i] = 0.f;
    }
    for (int s0 = wave; s0 < n_splits; s0 += NW * kMergeBatch) {
#pragma unroll
        for (int k = 0; k < EPL; ++k) {
            const int e = lane + 64 * k;
            if (e >= E) break;
            const int gl = e / (D / 8), c = e - gl * (D / 8);
            const int g = g0 + gl;
            float2 ml[kMergeBatch];
            float4 lo[kMergeBatch], hi[kMergeBatch];
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                const int sp = s0 + j * NW;
                if (sp < n_splits) {
                    const size_t row = base + (size_t)sp * G + g;
                    ml[j] = pml[row];
                    lo[j] = po[(row * D + 8 * c) / 4];
                    hi[j] = po[(row * D + 8 * c) / 4 + 1];
                } else {
                    ml[j] = make_float2(-INFINITY, 0.f);
                    lo[j] = hi[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
            float bm = M[k];
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) bm = fmaxf(bm, ml[j].x);
            if (bm == -INFINITY) continue;  // no valid key in these splits yet
            const float corr = fast_exp2(M[k] - bm);  // 0 while M = -inf
            L[k] *= corr;
#pragma unroll
            for (int i = 0; i < 8; ++i) O[k][i] *= corr;
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                const float w = fast_exp2(ml[j].x - bm);  // 0 for a split past n_splits
                L[k] = fmaf(w, ml[j].y, L[k]);
                O[k][0] = fmaf(w, lo[j].x, O[k][0]);
                O[k][1] = fmaf(w, lo[j].y, O[k][1]);
                O[k][2] = fmaf(w, lo[j].z, O[k][2]);
                O[k][3] = fmaf(w, lo[j].w, O[k][3]);
                O[k][4] = fmaf(w, hi[j].x, O[k][4]);
                O[k][5] = fmaf(w, hi[j].y, O[k][5]);
                O[k][6] = fmaf(w, hi[j].z, O[k][6]);
                O[k][7] = fmaf(w, hi[j].w, O[k][7]);
            }
            M[k] = bm;
        }
    }
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
        const int e = lane + 64 * k;
        if (e >= E) break;
        const int gl = e / (D / 8), c = e - gl * (D / 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) lds_o[wave][gl][8 * c + i] = O[k][i];
        if (c == 0) {
            lds_m[wave][gl] = M[k];
            lds_l[wave][gl] = L[k];
        }
    }
    __syncthreads();
    const int H_q = a.n_kv_heads * G;
    for (int idx = threadIdx.x; idx < GH * D; idx += NW * 64) {
        const int gl = idx / D, d = idx - gl * D;
        float Mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) Mx = fmaxf(Mx, lds_m[w][gl]);
        float Ov = 0.f, Ls = 0.f;
        if (Mx != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float sc = fast_exp2(lds_m[w][gl] - Mx);  // 0 for a wave without splits
                Ov = fmaf(sc, lds_o[w][gl][d], Ov);
                Ls = fmaf(sc, lds_l[w][gl], Ls);
            }
        }
        const size_t row = (size_t)b * H_q + h * G + g0 + gl;
        a.out[row * D + d] = f32_to_bf16_rne(Ls > 0.f ? Ov / Ls : 0.f);
        if (d == 0 && a.lse != nullptr) a.lse[row] = Ls > 0.f ? (Mx + log2f(Ls)) * kLn2 : -INFINITY;
    }
}

template <int D, int G, int NW, bool PAGED, bool CACHED>
__global__ __launch_bounds__(NW * 64) void decode_split_kernel(DecodeArgs a) {
    constexpr int NCH = D / 8;           // 16-byte words per K/V row
    constexpr int RK = 16;               // keys per wave round
    constexpr int RPL = 64 / NCH;        // rows covered by one wave-wide 1 KiB load
    constexpr int NLD = RK / RPL;        // wave loads per round, for K and for V
    static_assert(NLD >= 1 && G <= 16, "16-key rounds, up to 16 heads per group");

    const int split = blockIdx.x;
    int row = blockIdx.y;  // (rank of the sequence) * H_kv + kv head
    // Equal lengths keep index order (rank_to_sequence would return the rank): then no ticket and no
    // ranking.  Every wave of every work-group reaches the same answer from the same lengths.
    const bool ranked = a.longest_first && batch_is_ragged(a);
    if (a.ticket != nullptr && ranked) {
        // One split per row: the work-group takes the next row in longest-first order as it starts.
        // The counter is zero when a launch starts (cleared with the context, then reset by every
        // launch): the launch's work-groups take one ticket each, 0 .. rows-1, and the one holding
        // rows-1 made the last increment, so its store of zero races with none.  Taking the ticket
        // modulo the row count keeps the row in range even if the counter held something else.
        __shared__ int s_row;
        if (threadIdx.x == 0) {
            const unsigned rows = gridDim.y;
            const unsigned t = (unsigned)__hip_atomic_fetch_add(a.ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (t % rows == rows - 1) __hip_atomic_store(a.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_row = (int)(t % rows);
        }
        __syncthreads();
        row = s_row;
    }
    const int h = row % a.n_kv_heads;
    int b = row / a.n_kv_heads;
    if (ranked) b = rank_to_sequence(a, b);
    const int unit = b * a.n_kv_heads + h;
    const int H_q = a.n_kv_heads * G;
    const int L = clamp_len(a.lens[b], a.l_max);
    const int n_splits = decode_split_count(L, a.chunk);
    if (split >= n_splits) return;  // uniform across the work-group
    const int k_begin = split * a.chunk;
    const int k_end = split == n_splits - 1 ? L : k_begin + a.chunk;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const size_t row0 = (size_t)unit * a.l_cap;

    // Fused append (see the file comment): the appended row, if any, and where it goes.
    const int pos = (a.k_new != nullptr) ? a.positions[b] : -1;
    const bool has_new = pos >= 0 && pos < a.l_max;
    const u32x4* knew = reinterpret_cast<const u32x4*>(a.k_new) + (size_t)unit * NCH;
    const u32x4* vnew = reinterpret_cast<const u32x4*>(a.v_new) + (size_t)unit * NCH;
    const int32_t* trow = PAGED ? a.block_table + (size_t)b * a.max_pages : nullptr;
    if (has_new && split == 0 && threadIdx.x < 2 * NCH) {
        const int c = threadIdx.x % NCH;
        int64_t r;
        if constexpr (PAGED)
            r = paged_row(trow, a.page_shift, a.n_kv_heads, h, pos);  // -1: unmapped, not written
        else
            r = (int64_t)(row0 + pos);
        if (r >= 0) {
            u32x4* dst = reinterpret_cast<u32x4*>(threadIdx.x < NCH ? a.kc : a.vc) + (size_t)r * NCH + c;
            *dst = (threadIdx.x < NCH) ? knew[c] : vnew[c];
        }
    }

    // LDS: a K and a V tile per wave; the merge's O reuses their space once every wave is done.
    constexpr int KV_TILE = RK * NCH;  // 16-byte words of one K (or V) tile
    constexpr size_t O_BYTES = sizeof(float) * NW * G * D;
    constexpr size_t KV_BYTES = 16 * 2 * NW * KV_TILE;
    __shared__ __attribute__((aligned(16))) uint8_t lds_raw[KV_BYTES > O_BYTES ? KV_BYTES : O_BYTES];
    float(*const lds_o)[G][D] = reinterpret_cast<float(*)[G][D]>(lds_raw);
    u32x4* const lds_kv = reinterpret_cast<u32x4*>(lds_raw);
    __shared__ float lds_m[NW][G];
    __shared__ float lds_l[NW][G];

    // Q^T operand: lane l holds dims 32t + 8(l/16) .. +7 of head l % 16 for every t (heads past G
    // are zero).  O^T accumulators: o_acc[t] holds rows (dims) 16t + 4(l/16) + i, column (head)
    // l % 16.  Lane (cpv, rpv) of the loads holds 16-byte chunk cpv of rows rpv, rpv + RPL, ...
    u32x4 qb[D / 32];
    {
        const int hq = lane & 15;
        const u32x4* qp = reinterpret_cast<const u32x4*>(a.q + ((size_t)b * H_q + h * G + (hq < G ? hq : 0)) * D);
#pragma unroll
        for (int t = 0; t < D / 32; ++t) qb[t] = hq < G ? qp[4 * t + (lane >> 4)] : u32x4{0u, 0u, 0u, 0u};
    }
    const int rpv = lane / NCH;
    const int cpv = lane - rpv * NCH;
    f32x4 o_acc[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; ++t) o_acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;  // running max (log2 units) of this lane's head, uniform over its lanes
    float l_lane = 0.f;       // this lane's share of the running sum of its head

    const u32x4* kbase = reinterpret_cast<const u32x4*>(a.kc) + (PAGED ? 0 : row0 * NCH);
    const u32x4* vbase = reinterpret_cast<const u32x4*>(a.vc) + (PAGED ? 0 : row0 * NCH);
    const u32x4* zero = reinterpret_cast<const u32x4*>(a.zero_row);

    // Rounds start at multiples of RK and l_cap (the page size, when paged) is a multiple of
    // 64, so every row a round touches lies inside the sequence's cache region (one page);
    // rows >= k_end are read as the zero row and their scores masked.
    const int n_rounds = (k_end - k_begin + RK - 1) / RK;
    u32x4 kr[NLD], vr[NLD];
    // Rows of a round: first word of row key0 and the row stride (0: an unmapped page, read
    // as the zero row).  key0 is uniform across the wave, so the page lookup is scalar.
    struct RoundSrc {
        const u32x4* k;
        const u32x4* v;
        int stride;
    };
    // Paged: 64 consecutive block-table entries of the sequence, one per lane, from page
    // pc_first on; a round reads its page with v_readlane (no memory access and no wait), and
    // the window moves once every 64 pages.
    int pc_first = -(1 << 30), pc_val = -1;
    auto page_of = [&](int page_idx) -> int {  // page_idx is wave-uniform
        if (page_idx - pc_first >= 64 || page_idx < pc_first) {
            pc_first = page_idx;
            const int i = page_idx + lane;
            pc_val = i < a.max_pages ? trow[i] : -1;
        }
        return __builtin_amdgcn_readlane(pc_val, page_idx - pc_first);
    };
    auto round_src = [&](int key0) -> RoundSrc {
        if constexpr (PAGED) {
            const int k0 = __builtin_amdgcn_readfirstlane(key0);
            const int page = page_of(k0 >> a.page_shift);
            if (page < 0) return {zero, zero, 0};
            const int64_t r = (((int64_t)page * a.n_kv_heads + h) << a.page_shift) + (k0 & ((1 << a.page_shift) - 1));
            return {kbase + (size_t)r * NCH, vbase + (size_t)r * NCH, NCH};
        } else {
            return {kbase + (size_t)key0 * NCH, vbase + (size_t)key0 * NCH, NCH};
        }
    };
    // One round of this wave: rows key0 + j*RPL + rpv of K and V.  A round that ends past k_end
    // or holds the row appended by this launch takes a per-lane path (rows >= k_end read as the
    // zero row, since stale cache words may be NaN and 0 * NaN is NaN; the appended row comes
    // from k_new/v_new); every other round loads straight from the cache.  The test is
    // wave-uniform.
    auto load_round = [&](int key0, u32x4* kd, u32x4* vd) {
        const RoundSrc src = round_src(key0);
        const bool special = key0 + RK > k_end || (has_new && pos >= key0 && pos < key0 + RK);
        if (special) {
#pragma unroll
            for (int j = 0; j < NLD; ++j) {
                const int rel = j * RPL + rpv;
                const int key = key0 + rel;
                const size_t off = (size_t)rel * src.stride + cpv;
                const bool past = key >= k_end;
                const bool fresh = has_new && key == pos;
                kd[j] = ld_stream<CACHED>(past ? zero + cpv : fresh ? knew + cpv : src.k + off);
                vd[j] = ld_stream<CACHED>(past ? zero + cpv : fresh ? vnew + cpv : src.v + off);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NLD; ++j) {
                const size_t off = (size_t)(j * RPL + rpv) * src.stride + cpv;
                kd[j] = ld_stream<CACHED>(src.k + off);
                vd[j] = ld_stream<CACHED>(src.v + off);
            }
        }
    };
    int r = wave;
    if (r < n_rounds) load_round(k_begin + r * RK, kr, vr);
    for (; r < n_rounds; r += NW) {
        const int key0 = k_begin + r * RK;
        // K and V rows of the round into the wave's two LDS tiles: K swizzled so that the
        // A-operand reads below (row l % 16, 16 bytes) are conflict-free, V in 32-byte runs
        // swizzled so that a transposing read's 8 keys of one half-wave hit 8 different runs.
        u32x4* const tk = lds_kv + (size_t)(2 * wave) * KV_TILE;
        u32x4* const tv = tk + KV_TILE;
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
            const int row = j * RPL + rpv;
            tk[row * NCH + (cpv ^ mf_kswz<D>(row))] = kr[j];
            tv[row * NCH + 2 * ((cpv >> 1) ^ mf_vswz<D>(row)) + (cpv & 1)] = vr[j];
        }
        // Prefetch the next round of this wave.
        if (r + NW < n_rounds) load_round(key0 + NW * RK, kr, vr);
        wave_lds_sync();

        // 2. S^T [16 keys x 16 heads] = K [16 x D] . Q^T [D x 16]: lane l gets keys
        //    4(l/16) .. +3 of head l % 16.
        const int m16 = lane & 15, grp = lane >> 4;
        f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < D / 32; ++t)
            sacc = mfma_16x16x32(tk[m16 * NCH + ((4 * t + grp) ^ mf_kswz<D>(m16))], qb[t], sacc);

        // 3. Online softmax of head l % 16 over its 16 keys (4 per lane, 4 lanes), rescaled
        //    lazily as below.
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[i] = (key0 + 4 * grp + i < k_end) ? sacc[i] * a.scale_log2 : -INFINITY;
            mx = fmaxf(mx, sv[i]);
        }
        mx = pair_max32(pair_max16(mx));
        const float m_cand = fmaxf(m_run, mx);
        if (__ballot(m_cand > m_run + kRescaleSlack) != 0) {
            const float corr = (m_cand == -INFINITY) ? 1.f : fast_exp2(m_run - m_cand);
            m_run = m_cand;
            l_lane *= corr;
#pragma unroll
            for (int t = 0; t < D / 16; ++t) o_acc[t] *= corr;
        }
        float pf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pf[i] = (sv[i] == -INFINITY) ? 0.f : fast_exp2(sv[i] - m_run);
            l_lane += pf[i];
        }
        // The S^T result layout is the B-operand layout of P^T (keys 4(l/16) .. +3, head l % 16).
        const u32x2 pb = {pack_bf16x2(pf[0], pf[1]), pack_bf16x2(pf[2], pf[3])};

        // 4. O^T [D x 16 heads] += V^T [D x 16 keys] . P^T: per 16-dim tile, lane l of half-wave
        //    group g addresses key 4g + (l%16)/4, dims 16t + 4(l%4) .. +3 and receives dim
        //    16t + l % 16 of keys 4g .. 4g + 3.
        const int vkey = 4 * grp + (m16 >> 2);
        const uint8_t* const vrow = reinterpret_cast<const uint8_t*>(tv + vkey * NCH) + 8 * (lane & 3);
#pragma unroll
        for (int t = 0; t < D / 16; ++t)
            o_acc[t] = mfma_16x16x16(lds_read_tr16(vrow + 32 * (t ^ mf_vswz<D>(vkey))), pb, o_acc[t]);
    }

    // ---- merge the waves of this work-group ----
    __syncthreads();  // every wave is done with its K/V tiles, whose space lds_o reuses
    {
        const float l_head = pair_sum32(pair_sum16(l_lane));
        const int hq = lane & 15, grp = lane >> 4;
        if (hq < G) {
#pragma unroll
            for (int t = 0; t < D / 16; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) lds_o[wave][hq][16 * t + 4 * grp + i] = o_acc[t][i];
            if (grp == 0) {
                lds_m[wave][hq] = m_run;
                lds_l[wave][hq] = l_head;
            }
        }
    }
    __syncthreads();

    const bool single = (n_splits == 1);
    const bool fused_merge = !single && a.arrivals != nullptr;
    for (int idx = threadIdx.x; idx < G * D; idx += NW * 64) {
        const int g = idx / D;
        const int d = idx - g * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, lds_m[w][g]);
        float O = 0.f, Ls = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float sc = fast_exp2(lds_m[w][g] - M);
                O = fmaf(sc, lds_o[w][g][d], O);
                Ls = fmaf(sc, lds_l[w][g], Ls);
            }
        }
        if (single) {
            const size_t row = (size_t)b * H_q + h * G + g;
            a.out[row * D + d] = f32_to_bf16_rne(Ls > 0.f ? O / Ls : 0.f);
            if (d == 0 && a.lse != nullptr) a.lse[row] = Ls > 0.f ? (M + log2f(Ls)) * kLn2 : -INFINITY;
        } else {
            const size_t pidx = ((size_t)unit * a.max_splits + split) * G + g;
            if (fused_merge) {
                // Agent-scope atomic stores: coherent across the XCDs without an L2 write-back.
                __hip_atomic_store(&a.part_o[pidx * D + d], O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (d == 0) {
                    __hip_atomic_store(&a.part_ml[pidx * 2], M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&a.part_ml[pidx * 2 + 1], Ls, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                a.part_o[pidx * D + d] = O;
                if (d == 0) {
                    a.part_ml[pidx * 2] = M;
                    a.part_ml[pidx * 2 + 1] = Ls;
                }
            }
        }
    }
    if (!fused_merge) return;
    // The last split of this (sequence, kv head) to arrive merges every split's partial.  Every
    // thread's partial stores happen before thread 0's release increment (work-group barrier); the
    // increment that reads n_splits - 1 acquires all of them (release sequence of the counter).
    // That split resets the counter for the next launch.
    __shared__ int is_last;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(&a.arrivals[unit], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        is_last = prev == n_splits - 1;
        if (is_last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the other splits' partials
            __hip_atomic_store(&a.arrivals[unit], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
    if (!is_last) return;
    merge_splits_parallel<D, G, NW, G>(a, unit, b, h, n_splits, 0, lds_o, lds_m, lds_l);
}

// Waves per split work-group: 8 for every group size (at most 150 registers per lane with the
// matrix-core rounds, so two waves per SIMD), which gives one (sequence, kv head) twice the loads in
// flight of a 4-wave work-group: ragged batches finish their long sequences sooner, and a long
// context is cut into half as many splits.

// The merge launch: one work-group per (sequence, kv head, query head of the group), each reading
// one head's share of the partials (G times the work-groups of a per-(sequence, kv head) grid, each
// with 1/G of the loads and LDS).
template <int D, int G, int NW>
__global__ __launch_bounds__(NW * 64) void decode_combine_kernel(DecodeArgs a) {
    const int unit = blockIdx.x / G;
    const int g = blockIdx.x - unit * G;
    const int b = unit / a.n_kv_heads;
    const int h = unit - b * a.n_kv_heads;
    const int L = clamp_len(a.lens[b], a.l_max);
    const int n_splits = decode_split_count(L, a.chunk);
    if (n_splits <= 1) return;  // written directly by the split kernel
    __shared__ float lds_o[NW][1][D];
    __shared__ float lds_m[NW][1];
    __shared__ float lds_l[NW][1];
    merge_splits_parallel<D, G, NW, 1>(a, unit, b, h, n_splits, g, lds_o, lds_m, lds_l);
}

template <int D, int G, int NW>
hipError_t launch_decode_nw(const DecodeArgs& a, const Launch& l) {
    dim3 grid(a.max_splits, a.batch * a.n_kv_heads);
    if (a.cached) {
        if (a.block_table != nullptr)
            return launch_kernel(decode_split_kernel<D, G, NW, true, true>, grid, dim3(NW * 64), l, a);
        return launch_kernel(decode_split_kernel<D, G, NW, false, true>, grid, dim3(NW * 64), l, a);
    }
    if (a.block_table != nullptr)
        return launch_kernel(decode_split_kernel<D, G, NW, true, false>, grid, dim3(NW * 64), l, a);
    return launch_kernel(decode_split_kernel<D, G, NW, false, false>, grid, dim3(NW * 64), l, a);
}

template <int D, int G>
hipError_t launch_decode_t(const DecodeArgs& a, const Launch& l) {
    if (a.waves == kDecodeWavesSmall) return launch_decode_nw<D, G, kDecodeWavesSmall>(a, l);
    if (a.waves == kDecodeWaves) return launch_decode_nw<D, G, kDecodeWaves>(a, l);
    return hipErrorInvalidValue;
}

template <int D, int G>
hipError_t launch_combine_t(const DecodeArgs& a, const Launch& l) {
    const dim3 grid(a.batch * a.n_kv_heads * G);
    if (a.waves == kDecodeWavesSmall)
        return launch_kernel(decode_combine_kernel<D, G, kDecodeWavesSmall>, grid, dim3(kDecodeWavesSmall * 64), l, a);
    if (a.waves == kDecodeWaves)
        return launch_kernel(decode_combine_kernel<D, G, kDecodeWaves>, grid, dim3(kDecodeWaves * 64), l, a);
    return hipErrorInvalidValue;
}

}  // namespace

int decode_round_keys(int) { return 16; }  // RK of decode_split_kernel, every group size

bool decode_supported(int head_dim, int group) {
    return (head_dim == 64 || head_dim == 128) && (group == 2 || group == 4 || group == 8 || group == 16);
}

#define LARA_DISPATCH_DG(FN, D_, G_, ...)                              \
    do {                                                               \
        if ((D_) == 128) {                                             \
            if ((G_) == 4) return FN<128, 4>(__VA_ARGS__);             \
            if ((G_) == 8) return FN<128, 8>(__VA_ARGS__);             \
            if ((G_) == 2) return FN<128, 2>(__VA_ARGS__);             \
            if ((G_) == 16) return FN<128, 16>(__VA_ARGS__);           \
        } else if ((D_) == 64) {                                       \
            if ((G_) == 4) return FN<64, 4>(__VA_ARGS__);              \
            if ((G_) == 8) return FN<64, 8>(__VA_ARGS__);              \
            if ((G_) == 2) return FN<64, 2>(__VA_ARGS__);              \
            if ((G_) == 16) return FN<64, 16>(__VA_ARGS__);            \
        }                                                              \
        return hipErrorInvalidValue;                                   \
    } while (0)

hipError_t launch_decode(int head_dim, int group, const DecodeArgs& a, const Launch& l) {
    LARA_DISPATCH_DG(launch_decode_t, head_dim, group, a, l);
}

hipError_t launch_combine(int head_dim, int group, const DecodeArgs& a, const Launch& l) {
    LARA_DISPATCH_DG(launch_combine_t, head_dim, group, a, l);
}


}  // namespace lara
