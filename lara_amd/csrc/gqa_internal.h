// Internal declarations shared by the libgqa translation units (not part of the ABI).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lara {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Cross-lane reductions over lane pairs (l, l ^ 16) and (l, l ^ 32) without an LDS round trip.
// v_permlane16_swap (v_permlane32_swap) of a register with itself exchanges the odd 16-lane rows
// (the upper 32-lane half) of its first result with the even rows (lower half) of its second, so
// of the two results one holds the lane's own value and the other its partner's: their max (sum)
// is the pair's max (sum), with no select on the lane's position.  (A two-term fp32 sum is the
// same word in either order.)
__device__ __forceinline__ float pair_max16(float x) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float pair_max32(float x) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float pair_sum16(float x) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}
__device__ __forceinline__ float pair_sum32(float x) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Where a kernel goes: its stream and, while profiling, a start/stop event pair that the runtime
// stamps with the launch's own begin and end (hipExtLaunchKernel binds them to the dispatch
// itself, so no marker command sits between timed launches and they run back to back).
struct Launch {
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

template <typename... KArgs, typename... Args>
inline hipError_t launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, const Launch& l, Args... args) {
    if (l.start != nullptr || l.stop != nullptr)
        hipExtLaunchKernelGGL(kernel, grid, block, 0, l.stream, l.start, l.stop, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, 0, l.stream, args...);
    return hipGetLastError();
}

// Split-KV decode launch description.  All pointers are device pointers.
struct DecodeArgs {
    const uint16_t* q;      // [B][H_q][D] bf16
    uint16_t* kc;           // [B][H_kv][L_cap][D] bf16
    uint16_t* vc;           // same layout as kc
    const int32_t* lens;    // [B] keys attended per sequence
    const uint16_t* k_new;  // [B][H_kv][D] rows appended by this launch, or nullptr
    const uint16_t* v_new;  // same layout as k_new
    const int32_t* positions;  // [B] cache row of the appended row (-1: none), or nullptr
    int32_t batch;
    int32_t n_kv_heads;
    int32_t l_cap;          // cache rows per (b, kv head), multiple of 64
    int32_t l_max;          // configured maximum (lens are clamped to it)
    int32_t chunk;          // keys per split work-group, multiple of 256
    int32_t max_splits;     // grid x extent; splits beyond a sequence's length exit
    float scale_log2;       // softmax scale * log2(e)
    float* part_o;          // [B*H_kv][max_splits][G][D] fp32 un-normalised partial O
    float* part_ml;         // [B*H_kv][max_splits][G][2] (running max in log2 units, sum)
    uint16_t* out;          // [B][H_q][D] bf16
    float* lse;             // [B][H_q] natural-log LSE, or nullptr
    // Paged cache (block_table != nullptr): kc/vc are the page pools [n_pages][H_kv][P][D] and
    // row t of (b, h) is row t % P of page block_table[b * max_pages + t / P] (P = 2^page_shift,
    // a multiple of 64); rows of an unmapped page (-1) read as zero_row and are never written.
    const int32_t* block_table;
    int32_t page_shift;
    int32_t max_pages;
    const uint16_t* zero_row;
    // Nonzero: grid row y runs the (y / H_kv)-th longest sequence instead of sequence y / H_kv,
    // so the longest sequences are dispatched first (exact order up to 64 sequences, by length
    // bucket beyond).
    int32_t longest_first;
    // [B*H_kv] split arrival counters, zero between launches: the last split of a (sequence, kv
    // head) to finish merges the partials itself (no merge launch); nullptr = decode_combine_kernel.
    int32_t* arrivals;
    // One split per (sequence, kv head) and several sequences: a counter, zero between launches,
    // from which each work-group takes its grid row as it starts (rows in longest-first order), so
    // the rows left for the second dispatch round go to the work-groups that start first, on
    // whichever XCDs stream fastest; nullptr = row blockIdx.y.
    int32_t* ticket;
    // Nonzero: K/V rows are read with plain (L2-allocating) loads instead of nontemporal ones
    // (decode_cached_loads).
    int32_t cached;
    // Waves per work-group of the split and merge kernels: kDecodeWaves, or kDecodeWavesSmall for
    // launches that are a short latency chain (plan_decode_shape).  Both kernels of a plan use the
    // same count, so the in-launch merge and the merge launch fold in the same order.
    int32_t waves;
};
constexpr int kDecodeWaves = 8;
constexpr int kDecodeWavesSmall = 4;
// Whether a decode launch over `units` (sequence, kv head) units of at most max_len keys reads
// its K/V with plain loads: when they fit the L2s of the XCDs (4 MiB each) several times over, a
// step finds them where the last one left them.
constexpr int64_t kDecodeCachedBytes = 24ll << 20;
inline bool decode_cached_loads(int64_t units, int max_len, int head_dim) {
    return units * (int64_t)max_len * head_dim * 2 * 2 <= kDecodeCachedBytes;
}

// Chunked prefill / full-transaction launch description (one sequence b).
struct PrefillArgs {
    const uint16_t* q;      // [H_q][q_len][D] bf16, head-major
    uint16_t* kc;           // cache base of sequence b: [H_kv][L_cap][D]
    uint16_t* vc;
    const uint16_t* k_new;  // [H_kv][n_new][D] rows placed at cache rows new_begin.. by this launch
    const uint16_t* v_new;  //   (nullptr: none)
    int32_t new_begin;
    int32_t n_new;
    int32_t n_q_heads;
    int32_t n_kv_heads;
    int32_t l_cap;
    int32_t q_len;
    int32_t kv_len;
    int32_t q_pos_base;
    int32_t kv_pos_base;
    int32_t causal;
    float scale_log2;
    uint16_t* out;          // [H_q][q_len][D] bf16
    float* lse;             // [H_q][q_len] or nullptr
    int32_t seg_len;        // keys per KV segment (multiple of 64)
    int32_t n_segs;         // KV segments (grid z); 1 = write the output directly
    uint16_t* part_o;       // [n_segs][H_q][q_len][D] fp16 words: the segment's O divided by 2^e, e the
                            //   exponent of the row's largest |O| (frexp)
    float* part_ml;         // [n_segs][H_q][q_len][4] (running max in log2 units, sum l, e, unused)
    const uint16_t* zero_row;  // >= D zero words: the source of K/V rows past kv_len
    // Paged cache: block_table is sequence b's row of page indices (-1 = unmapped, read as
    // zero_row, never written), kc/vc the pools [n_pages][H_kv][2^page_shift][D]; nullptr =
    // contiguous cache of sequence b as above.
    const int32_t* block_table;
    int32_t page_shift;
    int32_t pair;           // 1: paired causal row blocks (G = 4, one segment; prefill_kernel)
};

// Row index (in units of D elements) of token row t of (sequence-relative) kv head h in a paged
// pool, or -1 when its page is unmapped.
__device__ __forceinline__ int64_t paged_row(const int32_t* table_row, int page_shift, int n_kv_heads, int h, int t) {
    const int page = table_row[t >> page_shift];
    if (page < 0) return -1;
    return (((int64_t)page * n_kv_heads + h) << page_shift) + (t & ((1 << page_shift) - 1));
}

// paged_row for a wave-uniform t: the table entry comes through the scalar cache (s_load, counted by
// lgkmcnt), so the wait for it does not also wait for the vector loads in flight (which a table
// read by a vector load would, since the compiler cannot see the kernels' direct-to-LDS loads).  The
// table is read-only while a kernel runs.
__device__ __forceinline__ int64_t paged_row_uniform(const int32_t* table_row, int page_shift, int n_kv_heads, int h,
                                                     int t) {
    typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
    const const_i32_ptr row = (const_i32_ptr)(uintptr_t)table_row;
    const int page = row[t >> page_shift];
    if (page < 0) return -1;
    return (((int64_t)page * n_kv_heads + h) << page_shift) + (t & ((1 << page_shift) - 1));
}

// KV segmentation of a prefill launch: (seg_len, n_segs) for q_len query rows whose
// attended key span is kv_span, sized so the launch has about target_wgs work-groups.
struct PrefillPlan {
    int32_t seg_len;
    int32_t n_segs;
};
constexpr int kPrefillRows = 32;  // query rows per prefill wave (a row block)
PrefillPlan plan_prefill(int q_len, int kv_span, int group, int n_kv_heads, int target_wgs, int max_segs);
// fp32 words of partial-output workspace a plan needs (O and (m, l) per row, per segment).
size_t prefill_workspace_floats(const PrefillPlan& p, int q_len, int n_q_heads, int head_dim);

// KV260 RTL-exact transaction (one sequence): the board's bit-level arithmetic.
struct RtlArgs {
    const uint16_t* q;      // [H_q][q_len][D] bf16, head-major
    const uint16_t* kc;     // cache base of sequence b: [H_kv][L_cap][D]
    const uint16_t* vc;
    int32_t n_q_heads;
    int32_t n_kv_heads;
    int32_t l_cap;
    int32_t q_len;
    int32_t kv_len;
    int32_t q_pos_base;
    int32_t kv_pos_base;
    int32_t causal;
    uint32_t scale_bits;    // fp32 bits of the score scale (the board's INV_SQRT_D_FP32)
    uint16_t* out;          // [H_q][q_len][D] bf16
    float* lse;             // [H_q][q_len] or nullptr
};
hipError_t launch_rtl_transaction(int head_dim, const RtlArgs& a, const Launch& l);

// Splits of a sequence of L attended keys cut into `chunk`-key splits: a last split of at most
// chunk/4 keys is folded into the one before it (no work-group is left with a handful of keys, such
// as the row a decode step appends); at least one split.  Split s covers keys
// [s*chunk, s == n-1 ? L : (s+1)*chunk).
__host__ __device__ inline int decode_split_count(int L, int chunk) {
    if (L <= chunk) return 1;
    const int n = (L + chunk - 1) / chunk;
    return (L - (n - 1) * chunk <= chunk / 4) ? n - 1 : n;
}

bool decode_supported(int head_dim, int group);
// Keys a wave of the decode kernel takes per round (a divisor of 64) for a group size.
int decode_round_keys(int group);

// Split-KV attention with an optional fused row append; sequences longer than one split
// leave fp32 partials that launch_combine merges.
hipError_t launch_decode(int head_dim, int group, const DecodeArgs& a, const Launch& l);
hipError_t launch_combine(int head_dim, int group, const DecodeArgs& a, const Launch& l);

bool prefill_supported(int head_dim, int group);
hipError_t launch_prefill(int head_dim, int group, const PrefillArgs& a, const Launch& l);
// One work-group per (query head, 32-row block), the waves splitting the keys and merging in LDS:
// for launches whose shared-tile grid (prefill_shared_wgs, no KV segments) is smaller than the GPU.
// Ignores seg_len / n_segs / part_*.
hipError_t launch_prefill_rows(int head_dim, const PrefillArgs& a, const Launch& l);
// Work-groups of launch_prefill for q_len rows without KV segments.
int prefill_shared_wgs(int q_len, int group, int n_kv_heads);
// Merges the KV segments of a prefill launch with n_segs > 1.
hipError_t launch_prefill_combine(int head_dim, const PrefillArgs& a, const Launch& l);

// K/V row append: rows [B][H_kv][D] -> cache row positions[b] (skipped if < 0 or >= l_max, or,
// in a paged cache (block_table != nullptr, [B][max_pages]), if the row's page is unmapped).
hipError_t launch_append(const uint16_t* k_rows, const uint16_t* v_rows, const int32_t* positions,
                         uint16_t* kc, uint16_t* vc, int batch, int n_kv_heads, int head_dim,
                         int l_cap, int l_max, const int32_t* block_table, int page_shift, int max_pages,
                         const Launch& l);

// Layer input stage of run_layer (sw/attn_driver.py:552-576): RMSNorm of the hidden states
// and, after the QKV projection GEMM, RoPE plus the head-major scatter of Q and of K/V into
// the cache.
constexpr int kMaxRopePairs = 64;  // head_dim <= 128

// cos/sin table of the RoPE stage: [sets][n_tokens][pairs][cos, sin] fp32, set 0 for the Q
// positions q_pos_base + t, set 1 for the K positions kv_pos_base + t (only when they differ).
struct RopeTable {
    float* cs;           // nullptr: no table to compute
    int sets, pairs, n_tokens;
    int q_pos_base, kv_pos_base;
    float theta[kMaxRopePairs];  // rotation frequency of pair (2p, 2p+1)
};

struct NormArgs {
    const uint16_t* x;      // [n_tokens][hidden] bf16
    const uint16_t* gamma;  // [hidden] bf16; nullptr: no rows to normalise (the table only)
    uint16_t* y;            // [n_tokens][hidden] bf16
    int n_tokens, hidden;
    float eps;
    int table_wgs;          // the launch's first table_wgs work-groups fill `table`
    RopeTable table;
};
hipError_t launch_rms_norm(const NormArgs& a, const Launch& l);

struct RopeArgs {
    const uint16_t* qkv;   // [n_tokens][ld] bf16: Q heads, then K heads, then V heads, D columns each
    int ld;
    int n_tokens, n_q_heads, n_kv_heads, head_dim;
    int rope;              // rotate Q and K with `cs`
    const float* cs;       // the RopeTable of this call (filled by the RMSNorm launch before it)
    int cs_k_set;          // 1: K positions have their own set, 0: K uses the Q set
    uint16_t* q_out;       // [n_q_heads][n_tokens][D]
    uint16_t* kc;          // cache of one sequence: [n_kv_heads][l_cap][D], rows row0 ..
    uint16_t* vc;          //   (paged: the pools, addressed through block_table)
    int l_cap, row0;
    const int32_t* block_table;  // paged: the sequence's page indices; nullptr = contiguous
    int page_shift;
};
hipError_t launch_rope_scatter(const RopeArgs& a, const Launch& l);

// Streaming-read ceiling probe (probe.hip): reads n_bytes (a multiple of 16) at src with n_wgs
// 512-thread work-groups, `unroll` (1, 2, 4 or 8) 16-byte nontemporal loads in flight per thread.
hipError_t launch_stream_read(const void* src, int64_t n_bytes, int n_wgs, int unroll, uint32_t* sink,
                              const Launch& l);

// fp32 -> bf16 word, round to nearest even on the upper half: the output rounding of
// fp32_to_bf16 in hw/rtl/pkg/attn_pkg.sv:618-626 (no NaN special case).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    uint32_t bits = __float_as_uint(x);
    uint32_t lsb = (bits >> 16) & 1u;
    bits += 0x7FFFu + lsb;
    return (uint16_t)(bits >> 16);
}

}  // namespace lara
