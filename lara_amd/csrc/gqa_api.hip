// C ABI of libgqa.so: context lifetime, validation, staging and the transaction protocol.
// Declarations and the reference interface each entry point replaces are in include/gqa.h.
#include "../../include/gqa.h"
#include "gqa_internal.h"
#include "page_table.h"

#include <math.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <mutex>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

using namespace lara;

namespace {

constexpr int kChunkOptionQuantum = 64;  // GQA_OPT_DECODE_CHUNK: a multiple of every decode round size
constexpr int kMinSplitCap = 256;        // the split workspace holds at least l_cap / this splits
constexpr int kMaxPrefillSegs = 16;
constexpr int32_t kMaxRows = 1 << 30;  // max_seq_len / max_q_len limit: row counts rounded up stay in int32
constexpr int kDecodeWavesPerCu = 8;  // split planner target; one split per (sequence, kv head) once that fills the GPU

struct Txn {
    int valid = 0;     // a transaction has been submitted (configure + Q staged)
    int running = 0;   // launched, completion not yet observed
    int32_t b = 0, q_len = 0, q_pos_base = 0, kv_len = 0, kv_pos_base = 0, causal = 1;
    int layer = 0;     // cache layer active at submission; the transaction reads that layer
    float kernel_us = 0.f, total_us = 0.f, copy_us = 0.f;
};

}  // namespace

// One projection GEMM shape, D[rows x n_tokens] (leading dimension ld) = W^T X with W stored
// [rows][hidden] and X [n_tokens][hidden] (column-major: W is hidden x rows, X hidden x
// n_tokens), bf16 in and out, fp32 accumulation: the hipBLASLt descriptors, the candidates its
// heuristic ranks first (workspace up to kProjectionWorkspace bytes) and the one in use: the
// heuristic's first until the first call outside a graph capture has timed them all.
constexpr int kProjectionCandidates = 8;
constexpr size_t kProjectionWorkspace = 32u << 20;
struct ProjectionPlan {
    int rows = 0, n_tokens = 0, hidden = 0, ld = 0;
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t w = nullptr, x = nullptr, d = nullptr;
    hipblasLtMatmulHeuristicResult_t cand[kProjectionCandidates] = {};
    int n_cand = 0;
    int pick = 0;        // index into cand of the algorithm in use
    bool tuned = false;  // pick chosen by timing
};
constexpr int kProjectionPlans = 8;

struct gqa_ctx {
    gqa_config cfg{};
    int group = 1;
    int l_cap = 0;
    int max_splits_cap = 0;
    float scale = 0.f;
    hipStream_t stream = nullptr;
    uint16_t* k_cache = nullptr;  // the active layer's K pool (k_pool + layer * kv_words)
    uint16_t* v_cache = nullptr;
    uint16_t* k_pool = nullptr;   // the allocations: n_layers pools back to back
    uint16_t* v_pool = nullptr;
    int n_layers = 1, layer = 0;
    float* part_o = nullptr;
    float* part_ml = nullptr;
    int32_t* arrivals = nullptr;  // [B*H_kv] split arrival counters of the fused merge, then the row ticket
                                  // of one-split launches (all zero between launches)
    int decode_merge = GQA_DECODE_MERGE_AUTO;
    int prefill_kernel = GQA_PREFILL_KERNEL_AUTO;
    float* pre_ws = nullptr;     // prefill KV-segment partials (O, then (m, l))
    uint16_t* zero_row = nullptr;  // one zero K/V row: the prefill source of rows past kv_len
    size_t pre_ws_floats = 0;
    uint16_t* q_dev = nullptr;   // staging: max(B*H_q*D, H_q*max_q_len*D) words
    uint16_t* o_dev = nullptr;   // same size as q_dev
    float* lse_dev = nullptr;    // max(B*H_q, H_q*max_q_len)
    int32_t* lens_dev = nullptr; // [B]
    int32_t* pos_dev = nullptr;  // [B] append positions (host fused decode)
    uint16_t* rows_dev = nullptr;  // [2][B][H_kv][D] append staging
    uint16_t* new_dev = nullptr;   // [2][H_kv][max_q_len][D] chunk-append staging
    uint16_t* o_pinned = nullptr;  // transaction output (host, pinned)
    size_t stage_words = 0;
    size_t lse_words = 0;
    int chunk_opt = 0;
    int prefill_wgs_opt = 0;
    int numerics = GQA_NUMERICS_EXACT;
    int profile = 0;
    hipEvent_t ev_begin = nullptr, ev_end = nullptr;
    // Profiling: a pool of event pairs per timer slot, filled launch by launch.
    hipEvent_t* ev_pool[GQA_TIMER_COUNT] = {};
    int ev_count[GQA_TIMER_COUNT] = {};
    hipEvent_t ev_t[4] = {};     // transaction: copy-in start, kernel start, kernel end, done
    float last_us = 0.f;
    double clock_mhz = 0.0;
    int n_cu = 256;  // compute units of the device (the planners' work-group targets scale with it)
    Txn txn;
    // Layer input stage (run_layer): hipBLASLt handle, projection plans and grow-only device
    // workspaces, created on first use; ev_layer brackets RMSNorm, projection and RoPE of the last timed layer call
    // (every host-pointer call; a device call only while profiling is on, since each recorded
    // event leaves the GPU idle for several microseconds between the launches it separates).
    hipblasLtHandle_t lt = nullptr;
    ProjectionPlan proj[kProjectionPlans];  // per GEMM shape, reused in turn
    int proj_next = 0;
    uint8_t* layer_in = nullptr;   // host-entry uploads: x, Wq, Wk, Wv, gamma
    size_t layer_in_bytes = 0;
    uint8_t* layer_tmp = nullptr;  // normalised x, then the [n_tokens][Q|K|V] projection
    size_t layer_tmp_bytes = 0;
    uint8_t* lt_ws = nullptr;      // hipBLASLt workspace of the projection algorithms in use
    size_t lt_ws_bytes = 0;
    hipEvent_t ev_layer[4] = {};
    float layer_us[3] = {};
    bool layer_timed = false;  // ev_layer holds a recorded call
    // Paged cache (gqa_create_paged): k_cache/v_cache are page pools [n_pages][H_kv][P][D], the
    // block tables [B][max_pages] live on the device (table_dev) and in `pages` on the host.
    int paged = 0;
    int page_size = 0, page_shift = 0, n_pages = 0, max_pages = 0;
    int32_t* table_dev = nullptr;
    PageTable pages;
    int last_prefill_kernel = 0;  // decomposition and KV segments of the last prefill launch (gqa_last_prefill_plan)
    int last_prefill_segs = 0;
};

// A prepared decode step (gqa_graph_capture_decode_append): the launch description planned once,
// replayed by direct launches, and the context it reads.
struct gqa_graph {
    gqa_ctx* ctx = nullptr;
    lara::DecodeArgs args{};
    bool combine = false;
};

namespace {

#define HIP_TRY(expr)                          \
    do {                                       \
        hipError_t err__ = (expr);             \
        if (err__ != hipSuccess) {             \
            last_hip_error(err__, #expr);      \
            return GQA_ERR_HIP;                \
        }                                      \
    } while (0)

thread_local char g_last_error[256];

void last_hip_error(hipError_t e, const char* what) {
    snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, hipGetErrorString(e));
}

inline size_t kv_words(const gqa_ctx* c) {
    if (c->paged) return (size_t)c->n_pages * c->cfg.n_kv_heads * c->page_size * c->cfg.head_dim;
    return (size_t)c->cfg.batch * c->cfg.n_kv_heads * c->l_cap * c->cfg.head_dim;
}

// Row (in units of D elements) of token t of (b, h) in the cache, or -1 (unmapped page).
int64_t cache_row(const gqa_ctx* c, int b, int h, int t) {
    if (!c->paged) return ((int64_t)b * c->cfg.n_kv_heads + h) * c->l_cap + t;
    const int page = c->pages.row(b)[t >> c->page_shift];
    if (page < 0) return -1;
    return (((int64_t)page * c->cfg.n_kv_heads + h) << c->page_shift) + (t & (c->page_size - 1));
}

// True when rows [row0, row0 + n) of sequence b are backed (always, for a contiguous cache).
bool rows_backed(const gqa_ctx* c, int b, int64_t row0, int64_t n) {
    return !c->paged || c->pages.covers(b, row0, n, c->page_size);
}

hipStream_t pick_stream(gqa_ctx* c, void* s) { return s ? (hipStream_t)s : c->stream; }

// Device operands the kernels move in 16-byte vectors (Q, appended K/V rows, prefill output)
// must be 16-byte aligned; nullptr passes (optional operands are checked for presence apart).
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Splits per (sequence, kv head) the automatic plan aims for: about kDecodeWavesPerCu waves per CU
// over the batch's units, with `waves` waves per work-group.
int plan_splits(int batch, int n_kv_heads, int n_cu, int waves) {
    const int units = batch * n_kv_heads;
    const int target_wgs = kDecodeWavesPerCu * n_cu / waves;
    const int splits = (target_wgs + units - 1) / units;
    return splits < 1 ? 1 : splits;
}

// Keys per split for max_len attended keys: max_len over plan_splits, in whole rounds of every wave
// of a work-group (128 keys with 8 waves) so the waves of a split share its keys evenly -- rounded
// down when that still gives at most plan_splits splits (a short tail joins the last split), else
// up.  decode_split_count(max_len, chunk) <= plan_splits either way.
// A (sequence, kv head) whose K/V take at most this many bytes is not split: one work-group streams
// it in about a microsecond, less than merging splits costs (8 q / 2 kv heads, D 64, 256 keys = 64 KiB
// per unit: 4.2 us of kernel in one split per unit against 4.8 us in four splits merged in-launch).
constexpr int64_t kDecodeSplitMinBytes = 128 << 10;

int plan_chunk(int batch, int n_kv_heads, int group, int n_cu, int max_len, int waves, int head_dim) {
    const int quantum = waves * decode_round_keys(group);
    if ((int64_t)max_len * head_dim * 2 * 2 <= kDecodeSplitMinBytes)
        return std::max(quantum, (max_len + quantum - 1) / quantum * quantum);
    const int splits = plan_splits(batch, n_kv_heads, n_cu, waves);
    const int even = (max_len + splits - 1) / splits;
    const int down = std::max(quantum, even / quantum * quantum);
    if (decode_split_count(max_len, down) <= splits) return down;
    return (even + quantum - 1) / quantum * quantum;
}

// Whether the last split to arrive merges a sequence's splits inside the decode launch.  Each split
// then ends with an agent-scope release (an L2 write-back of its XCD) and an increment of its
// sequence's arrival counter, and the last one with an acquire (an L2 invalidate): that saves the
// merge launch where the step is a short latency chain, but the L2 maintenance of many work-groups
// slows the streaming of the others.  AUTO fuses up to kFusedMergeSplits splits per sequence while
// the split grid fills at most half the CUs (measured, kernel time per step, fused vs launch: 4
// work-groups (2 splits of 128 keys) 5.1 vs 8.1 us, 64 work-groups (8 splits of 512) 9.4 vs 11.7 us,
// 32 q / 8 kv heads, one sequence of 2049 keys: 128 work-groups (16 splits of 128) 7.5 vs 8.6 us;
// 256 work-groups: 8 splits of 16384 keys 314.1 vs 311.5 us, 4 of 8192 161 vs 160 us, 2 of 4096
// 83-86 vs 81-82 us, 2 of 512 16.7 vs 16.1 us; 32 splits of 128 keys 9.4 vs 8.8 us).
constexpr int kFusedMergeSplits = 16;

bool fuse_merge(int option, int units, int max_splits, int n_cu) {
    if (max_splits <= 1 || option == GQA_DECODE_MERGE_LAUNCH) return false;
    return option == GQA_DECODE_MERGE_FUSED ||
           (2 * (int64_t)units * max_splits <= n_cu && max_splits <= kFusedMergeSplits);
}

// A decode launch's shape: keys per split, splits and waves per work-group.  Work-groups have
// kDecodeWaves waves, except in launches of at most kSmallDecodeGrid work-groups at that size (a
// step that is a short latency chain, such as one sequence of a few hundred keys): those are
// planned with kDecodeWavesSmall waves per work-group, which start and merge sooner (measured,
// 8 q / 2 kv heads, D 64, 256 keys: 4.87 vs 5.04 us of kernel; at 256 work-groups and more the
// 8-wave shape streams faster).  chunk_opt > 0 forces the keys per split.
// Under GQA_DECODE_MERGE_AUTO, a plan of the shortest splits (one round of every wave) whose merge
// would be a launch takes splits twice as long when that lets the merge fuse: the step loses a
// launch's latency for a round per split (measured, 32 q / 8 kv heads: one sequence of 4097 keys,
// 16 fused splits of 256 keys 8.27 us of kernel against 32 of 128 merged by a launch 8.66-8.80; two
// of 2049 keys, 8 fused splits of 256 8.50 against 16 of 128 and a launch 9.00).
constexpr int64_t kSmallDecodeGrid = 8;

struct DecodeShape {
    int chunk;
    int max_splits;
    int waves;
};

DecodeShape plan_decode_shape(int batch, int n_kv_heads, int group, int head_dim, int n_cu, int max_len,
                              int chunk_opt, int merge_option) {
    const int64_t units = (int64_t)batch * n_kv_heads;
    auto shape = [&](int waves) {
        const int chunk =
            chunk_opt > 0 ? chunk_opt : plan_chunk(batch, n_kv_heads, group, n_cu, max_len, waves, head_dim);
        return DecodeShape{chunk, decode_split_count(max_len, chunk), waves};
    };
    const DecodeShape big = shape(kDecodeWaves);
    if (units * big.max_splits <= kSmallDecodeGrid) return shape(kDecodeWavesSmall);
    if (chunk_opt <= 0 && merge_option == GQA_DECODE_MERGE_AUTO && big.max_splits > 1 &&
        big.chunk == kDecodeWaves * decode_round_keys(group) &&
        !fuse_merge(merge_option, (int)units, big.max_splits, n_cu)) {
        const int chunk = 2 * big.chunk;
        const DecodeShape twice{chunk, decode_split_count(max_len, chunk), kDecodeWaves};
        if (fuse_merge(merge_option, (int)units, twice.max_splits, n_cu)) return twice;
    }
    return big;
}

constexpr int kProfileLaunches = 512;  // event pairs kept per timer slot

// Whether work enqueued on s is being recorded into a caller's HIP graph (stream capture): such
// launches take no timer events and the layer stage does not tune on them.
bool stream_capturing(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// A launch on stream s; while profiling (outside a stream capture), with the next event pair of
// the timer slot bound to the launch itself (no marker commands between launches).
Launch timed(gqa_ctx* c, int slot, hipStream_t s) {
    Launch l;
    l.stream = s;
    if (c->profile && c->ev_count[slot] < kProfileLaunches && !stream_capturing(s)) {
        l.start = c->ev_pool[slot][2 * c->ev_count[slot]];
        l.stop = c->ev_pool[slot][2 * c->ev_count[slot] + 1];
        c->ev_count[slot] += 1;
    }
    return l;
}

void timers_reset(gqa_ctx* c) {
    for (int i = 0; i < GQA_TIMER_COUNT; ++i) c->ev_count[i] = 0;
}

int profile_enable(gqa_ctx* c, int on) {
    if (on) {
        for (int i = 0; i < GQA_TIMER_COUNT; ++i) {
            if (c->ev_pool[i]) continue;
            c->ev_pool[i] = (hipEvent_t*)calloc(2 * kProfileLaunches, sizeof(hipEvent_t));
            if (!c->ev_pool[i]) return GQA_ERR_OOM;
            for (int e = 0; e < 2 * kProfileLaunches; ++e) HIP_TRY(hipEventCreate(&c->ev_pool[i][e]));
        }
    }
    timers_reset(c);
    c->profile = on ? 1 : 0;
    return GQA_OK;
}

// The launch description of one decode step (split kernel, plus the merge launch when *combine);
// run_decode launches it, a prepared step (gqa_graph) keeps it for its replays.
int plan_decode(gqa_ctx* c, const void* q, const int32_t* lens, const void* k_new, const void* v_new,
                const int32_t* positions, void* o, float* lse, int max_len, DecodeArgs* out, bool* combine) {
    if (!decode_supported(c->cfg.head_dim, c->group) || c->numerics != GQA_NUMERICS_EXACT) return GQA_ERR_UNSUPPORTED;
    const DecodeShape shape = plan_decode_shape(c->cfg.batch, c->cfg.n_kv_heads, c->group, c->cfg.head_dim, c->n_cu,
                                                max_len, c->chunk_opt, c->decode_merge);
    const int chunk = shape.chunk;
    const int max_splits = shape.max_splits;
    if (max_splits > c->max_splits_cap) return GQA_ERR_RANGE;
    DecodeArgs& a = *out;
    a = DecodeArgs{};
    a.q = (const uint16_t*)q;
    a.kc = c->k_cache;
    a.vc = c->v_cache;
    a.lens = lens;
    a.k_new = (const uint16_t*)k_new;
    a.v_new = (const uint16_t*)v_new;
    a.positions = positions;
    a.batch = c->cfg.batch;
    a.n_kv_heads = c->cfg.n_kv_heads;
    a.l_cap = c->l_cap;
    a.l_max = c->cfg.max_seq_len;
    a.chunk = chunk;
    a.max_splits = max_splits;
    a.scale_log2 = c->scale * 1.4426950408889634f;
    a.part_o = c->part_o;
    a.part_ml = c->part_ml;
    a.out = (uint16_t*)o;
    a.lse = lse;
    a.block_table = c->paged ? c->table_dev : nullptr;
    a.page_shift = c->page_shift;
    a.max_pages = c->max_pages;
    a.zero_row = c->zero_row;
    a.longest_first = c->cfg.batch > 1;
    a.cached = decode_cached_loads((int64_t)c->cfg.batch * c->cfg.n_kv_heads, max_len, c->cfg.head_dim) ? 1 : 0;
    a.waves = shape.waves;
    a.arrivals = fuse_merge(c->decode_merge, c->cfg.batch * c->cfg.n_kv_heads, max_splits, c->n_cu) ? c->arrivals
                                                                                                      : nullptr;
    *combine = max_splits > 1 && a.arrivals == nullptr;
    a.ticket = (c->cfg.batch > 1 && max_splits == 1) ? c->arrivals + (size_t)c->cfg.batch * c->cfg.n_kv_heads : nullptr;
    return GQA_OK;
}

int run_decode(gqa_ctx* c, const void* q, const int32_t* lens, const void* k_new, const void* v_new,
               const int32_t* positions, void* o, float* lse, hipStream_t s, int max_len) {
    DecodeArgs a;
    bool combine = false;
    const int rc = plan_decode(c, q, lens, k_new, v_new, positions, o, lse, max_len, &a, &combine);
    if (rc != GQA_OK) return rc;
    HIP_TRY(launch_decode(c->cfg.head_dim, c->group, a, timed(c, GQA_TIMER_DECODE, s)));
    if (combine) HIP_TRY(launch_combine(c->cfg.head_dim, c->group, a, timed(c, GQA_TIMER_COMBINE, s)));
    return GQA_OK;
}

int check_prefill_args(const gqa_ctx* c, int32_t b, int32_t q_len, int32_t q_pos_base, int32_t kv_len,
                       int32_t kv_pos_base) {
    if (b < 0 || b >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
    if (q_len < 1 || q_len > c->cfg.max_q_len) return GQA_ERR_RANGE;
    if (kv_len < 0 || kv_len > c->cfg.max_seq_len) return GQA_ERR_RANGE;
    if (q_pos_base < 0 || kv_pos_base < 0) return GQA_ERR_RANGE;
    if ((int64_t)q_pos_base + q_len > INT32_MAX || (int64_t)kv_pos_base + kv_len > INT32_MAX)
        return GQA_ERR_RANGE;
    return GQA_OK;
}

int run_prefill(gqa_ctx* c, int32_t b, const void* q, int32_t q_len, int32_t q_pos_base, int32_t kv_len,
                int32_t kv_pos_base, int32_t causal, void* o, float* lse, hipStream_t s,
                const void* k_new = nullptr, const void* v_new = nullptr, int32_t n_new = 0) {
    if (c->paged) c->pages.touch(b);
    if (c->numerics == GQA_NUMERICS_KV260) {
        if (c->paged) return GQA_ERR_UNSUPPORTED;
        const size_t seq = (size_t)b * c->cfg.n_kv_heads * c->l_cap * c->cfg.head_dim;
        if (k_new != nullptr && n_new > 0) {
            const size_t D = c->cfg.head_dim;
            const size_t pitch_dst = (size_t)c->l_cap * D * 2, pitch_src = (size_t)n_new * D * 2;
            const size_t dst = seq + (size_t)(kv_len - n_new) * D;
            HIP_TRY(hipMemcpy2DAsync(c->k_cache + dst, pitch_dst, k_new, pitch_src, pitch_src, c->cfg.n_kv_heads,
                                     hipMemcpyDeviceToDevice, s));
            HIP_TRY(hipMemcpy2DAsync(c->v_cache + dst, pitch_dst, v_new, pitch_src, pitch_src, c->cfg.n_kv_heads,
                                     hipMemcpyDeviceToDevice, s));
        }
        RtlArgs r{};
        r.q = (const uint16_t*)q;
        r.kc = c->k_cache + seq;
        r.vc = c->v_cache + seq;
        r.n_q_heads = c->cfg.n_q_heads;
        r.n_kv_heads = c->cfg.n_kv_heads;
        r.l_cap = c->l_cap;
        r.q_len = q_len;
        r.kv_len = kv_len;
        r.q_pos_base = q_pos_base;
        r.kv_pos_base = kv_pos_base;
        r.causal = causal ? 1 : 0;
        uint32_t sb;
        memcpy(&sb, &c->scale, sizeof(sb));
        r.scale_bits = sb;
        r.out = (uint16_t*)o;
        r.lse = lse;
        HIP_TRY(launch_rtl_transaction(c->cfg.head_dim, r, timed(c, GQA_TIMER_PREFILL, s)));
        c->last_prefill_kernel = 0;
        c->last_prefill_segs = 0;
        return GQA_OK;
    }
    if (!prefill_supported(c->cfg.head_dim, c->group)) return GQA_ERR_UNSUPPORTED;
    int kv_span = kv_len;
    if (causal) kv_span = std::min(kv_len, std::max(0, q_pos_base + q_len - kv_pos_base));
    // Paired causal row blocks (shared kernel, one segment) for a causal prompt without earlier keys
    // (its rows see at most the prompt's own keys) whose shared grid is between half and one
    // work-group per CU: one dispatch round, whose row blocks range from one key block to all of
    // them.  (Measured, one causal launch, 32q/8kv, D 128: 1024 tokens 28.0 us paired vs 30.5 row
    // blocks, 1536: 37.6 vs 52.6, 2048: 48.8 vs 79.6 (64.4 unpaired); 768 tokens, 96 work-groups:
    // 23.5 vs 21.4.)  Earlier keys are read by both row blocks of a pair in step, unpaired, so
    // chunks after a history keep the row-block kernel.
    const int shared_wgs = prefill_shared_wgs(q_len, c->group, c->cfg.n_kv_heads);
    const bool pairable = causal && c->group == 4 && q_len > kPrefillRows;
    const bool pair_auto = c->prefill_kernel == GQA_PREFILL_KERNEL_AUTO && c->prefill_wgs_opt == 0 && pairable &&
                           kv_span <= q_len && 2 * shared_wgs >= c->n_cu && shared_wgs <= c->n_cu;
    // Launches whose shared-tile grid would not fill the GPU without KV segments take the row-block
    // kernel (no segments, no merge launch), unless a segment target is set.
    const bool rows = c->prefill_kernel == GQA_PREFILL_KERNEL_ROWS ||
                      (c->prefill_kernel == GQA_PREFILL_KERNEL_AUTO && c->prefill_wgs_opt == 0 &&
                       shared_wgs < c->n_cu && !pair_auto);
    // A forced PAIRED decomposition plans one KV segment (pairs exist only in one-segment launches);
    // launches it cannot pair (not causal, group != 4, one row block) plan as SHARED.
    const bool pair_forced = c->prefill_kernel == GQA_PREFILL_KERNEL_PAIRED && pairable;
    const int target = (pair_auto || pair_forced) ? 1 : c->prefill_wgs_opt > 0 ? c->prefill_wgs_opt : c->n_cu;
    PrefillPlan plan = plan_prefill(q_len, kv_span, c->group, c->cfg.n_kv_heads, target, kMaxPrefillSegs);
    if (prefill_workspace_floats(plan, q_len, c->cfg.n_q_heads, c->cfg.head_dim) > c->pre_ws_floats)
        plan = plan_prefill(q_len, kv_span, c->group, c->cfg.n_kv_heads, 1, 1);  // one segment
    PrefillArgs a{};
    const size_t seq_off = c->paged ? 0 : (size_t)b * c->cfg.n_kv_heads * c->l_cap * c->cfg.head_dim;
    a.q = (const uint16_t*)q;
    a.kc = c->k_cache + seq_off;
    a.vc = c->v_cache + seq_off;
    a.block_table = c->paged ? c->table_dev + (size_t)b * c->max_pages : nullptr;
    a.page_shift = c->page_shift;
    a.k_new = (const uint16_t*)k_new;
    a.v_new = (const uint16_t*)v_new;
    a.new_begin = kv_len - n_new;
    a.n_new = n_new;
    a.n_q_heads = c->cfg.n_q_heads;
    a.n_kv_heads = c->cfg.n_kv_heads;
    a.l_cap = c->l_cap;
    a.q_len = q_len;
    a.kv_len = kv_len;
    a.q_pos_base = q_pos_base;
    a.kv_pos_base = kv_pos_base;
    a.causal = causal ? 1 : 0;
    a.scale_log2 = c->scale * 1.4426950408889634f;
    a.out = (uint16_t*)o;
    a.lse = lse;
    a.seg_len = plan.seg_len;
    a.n_segs = plan.n_segs;
    a.zero_row = c->zero_row;
    a.part_o = reinterpret_cast<uint16_t*>(c->pre_ws);
    a.part_ml = c->pre_ws + (size_t)plan.n_segs * c->cfg.n_q_heads * q_len * (c->cfg.head_dim / 2);
    if (rows) {
        HIP_TRY(launch_prefill_rows(c->cfg.head_dim, a, timed(c, GQA_TIMER_PREFILL, s)));
        c->last_prefill_kernel = GQA_PREFILL_KERNEL_ROWS;
        c->last_prefill_segs = 1;
        return GQA_OK;
    }
    // Paired causal row blocks: the work of a causal grid grows with the row block, and a grid of one
    // dispatch round (at most one work-group per CU) cannot be balanced by longest-first dispatch.
    a.pair = pairable && plan.n_segs == 1 &&
                     (c->prefill_kernel == GQA_PREFILL_KERNEL_PAIRED || pair_auto ||
                      (c->prefill_kernel == GQA_PREFILL_KERNEL_AUTO && shared_wgs == c->n_cu))
                 ? 1 : 0;
    HIP_TRY(launch_prefill(c->cfg.head_dim, c->group, a, timed(c, GQA_TIMER_PREFILL, s)));
    if (plan.n_segs > 1) HIP_TRY(launch_prefill_combine(c->cfg.head_dim, a, timed(c, GQA_TIMER_COMBINE, s)));
    c->last_prefill_kernel = a.pair ? GQA_PREFILL_KERNEL_PAIRED : GQA_PREFILL_KERNEL_SHARED;
    c->last_prefill_segs = plan.n_segs;
    return GQA_OK;
}

int finish_sync(gqa_ctx* c) {
    HIP_TRY(hipEventRecord(c->ev_end, c->stream));
    HIP_TRY(hipEventSynchronize(c->ev_end));
    float ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&ms, c->ev_begin, c->ev_end));
    c->last_us = ms * 1000.f;
    return GQA_OK;
}

int txn_idle(gqa_ctx* c) {
    // A transaction in flight blocks every other use of the context's staging buffers.
    if (!c->txn.running) return GQA_OK;
    hipError_t e = hipEventQuery(c->ev_t[3]);
    if (e == hipErrorNotReady) return GQA_ERR_BUSY_START;
    if (e != hipSuccess) {
        last_hip_error(e, "hipEventQuery");
        return GQA_ERR_HIP;
    }
    return GQA_OK;
}

// Grow-only device buffer (the old contents are not kept).
int ensure_buffer(uint8_t** buf, size_t* cap, size_t bytes) {
    if (bytes <= *cap) return GQA_OK;
    if (*buf) {
        HIP_TRY(hipDeviceSynchronize());
        (void)hipFree(*buf);
        *buf = nullptr;
        *cap = 0;
    }
    if (hipMalloc(buf, bytes) != hipSuccess) {
        *buf = nullptr;
        return GQA_ERR_OOM;
    }
    *cap = bytes;
    return GQA_OK;
}

constexpr double kRopeBase = 10000.0;  // theta_p = 10000^(-2p/D): hw/data/rope_theta.hex for D = 128

int check_layer_args(const gqa_ctx* c, int32_t b, int32_t n_tokens, int32_t hidden, int32_t q_pos_base,
                     int32_t kv_pos_base, int32_t row0) {
    if (b < 0 || b >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
    if (n_tokens < 1 || n_tokens > c->cfg.max_q_len || hidden < 1) return GQA_ERR_RANGE;
    if (row0 < 0 || (int64_t)row0 + n_tokens > c->cfg.max_seq_len) return GQA_ERR_RANGE;
    if (q_pos_base < 0 || kv_pos_base < 0 || (int64_t)q_pos_base + n_tokens > (1 << 24) ||
        (int64_t)kv_pos_base + n_tokens > (1 << 24))
        return GQA_ERR_RANGE;  // positions are exact in the fp32 phase product below 2^24
    if (c->cfg.head_dim > 2 * kMaxRopePairs || (c->cfg.head_dim & 7)) return GQA_ERR_UNSUPPORTED;
    return GQA_OK;
}

void release_plan(ProjectionPlan& p) {
    if (p.w) (void)hipblasLtMatrixLayoutDestroy(p.w);
    if (p.x) (void)hipblasLtMatrixLayoutDestroy(p.x);
    if (p.d) (void)hipblasLtMatrixLayoutDestroy(p.d);
    if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
    p = ProjectionPlan();
}

// The cached plan for this projection shape, or a new one (replacing the oldest of
// kProjectionPlans): descriptors plus hipBLASLt's heuristic candidates.
int projection_plan(gqa_ctx* c, int rows, int n_tokens, int hidden, int ld, ProjectionPlan** out) {
    for (ProjectionPlan& p : c->proj)
        if (p.desc && p.rows == rows && p.n_tokens == n_tokens && p.hidden == hidden && p.ld == ld) {
            *out = &p;
            return GQA_OK;
        }
    ProjectionPlan& p = c->proj[c->proj_next];
    c->proj_next = (c->proj_next + 1) % kProjectionPlans;
    release_plan(p);
    hipblasLtMatmulPreference_t pref = nullptr;
    const hipblasOperation_t tw = HIPBLAS_OP_T, tx = HIPBLAS_OP_N;
    const uint64_t max_workspace = kProjectionWorkspace;
    int found = 0;
    hipblasStatus_t st = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &tw, sizeof(tw));
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tx, sizeof(tx));
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.w, HIP_R_16BF, hidden, rows, hidden);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.x, HIP_R_16BF, hidden, n_tokens, hidden);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.d, HIP_R_16BF, rows, n_tokens, ld);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatmulPreferenceCreate(&pref);
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_workspace,
                                                   sizeof(max_workspace));
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = hipblasLtMatmulAlgoGetHeuristic(c->lt, p.desc, p.w, p.x, p.d, p.d, pref, kProjectionCandidates, p.cand,
                                             &found);
    if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
    // Keep the usable candidates, in the heuristic's order.
    p.n_cand = 0;
    for (int i = 0; st == HIPBLAS_STATUS_SUCCESS && i < found && i < kProjectionCandidates; ++i)
        if (p.cand[i].state == HIPBLAS_STATUS_SUCCESS && p.cand[i].workspaceSize <= kProjectionWorkspace)
            p.cand[p.n_cand++] = p.cand[i];
    if (st != HIPBLAS_STATUS_SUCCESS || p.n_cand < 1) {
        snprintf(g_last_error, sizeof(g_last_error), "hipBLASLt projection plan %dx%dx%d: status %d, %d algorithms",
                 rows, n_tokens, hidden, (int)st, found);
        release_plan(p);
        return GQA_ERR_HIP;
    }
    p.pick = 0;
    p.tuned = p.n_cand == 1;
    p.rows = rows;
    p.n_tokens = n_tokens;
    p.hidden = hidden;
    p.ld = ld;
    *out = &p;
    return GQA_OK;
}

// Picks the fastest of a plan's candidates on the caller's operands: each runs once untimed,
// then three times between two events; the stream is synchronised once per candidate.  Every
// candidate computes the same product (beta = 0), so the runs leave the destination as the
// final call does.  A candidate that fails to launch is skipped.  Runs once per plan.
template <typename Gemm>
int tune_projection(gqa_ctx* c, ProjectionPlan* p, Gemm&& gemm, hipStream_t s) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    HIP_TRY(hipEventCreate(&e0));
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return GQA_ERR_HIP;
    }
    int best = 0;
    float best_ms = INFINITY;
    hipError_t err = hipSuccess;
    for (int k = 0; k < p->n_cand && err == hipSuccess; ++k) {
        if (gemm(k) != HIPBLAS_STATUS_SUCCESS) continue;
        bool ok = (err = hipEventRecord(e0, s)) == hipSuccess;
        for (int r = 0; ok && r < 3; ++r) ok = gemm(k) == HIPBLAS_STATUS_SUCCESS;
        if (err == hipSuccess) err = hipEventRecord(e1, s);
        if (err == hipSuccess) err = hipEventSynchronize(e1);
        float ms = 0.f;
        if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
        if (ok && err == hipSuccess && ms < best_ms) {
            best_ms = ms;
            best = k;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (err != hipSuccess) {
        last_hip_error(err, "projection tuning");
        return GQA_ERR_HIP;
    }
    p->pick = best;
    p->tuned = true;
    return GQA_OK;
}

// RMSNorm (if gamma) -> [Q|K|V] = x W^T (one fused or three hipBLASLt bf16 GEMMs, fp32
// accumulate) -> RoPE (if rope) and scatter: Q to q_out [H_q][n_tokens][D], K/V to rows
// row0.. of sequence b.
int run_layer_qkv(gqa_ctx* c, int32_t b, const void* x, int32_t n_tokens, int32_t hidden, const void* wq,
                  const void* wk, const void* wv, const void* gamma, float eps, int32_t q_pos_base,
                  int32_t kv_pos_base, int32_t row0, int32_t rope, void* q_out, hipStream_t s, bool stage_events) {
    const int D = c->cfg.head_dim, nq = c->cfg.n_q_heads * D, nkv = c->cfg.n_kv_heads * D;
    const int ld = nq + 2 * nkv;
    const size_t y_bytes = gamma ? ((size_t)n_tokens * hidden * 2 + 255) / 256 * 256 : 0;
    const size_t qkv_bytes = ((size_t)n_tokens * ld * 2 + 255) / 256 * 256;
    const int cs_sets = rope ? (kv_pos_base == q_pos_base ? 1 : 2) : 0;  // RoPE cos/sin table sets
    const size_t cs_bytes = (size_t)cs_sets * n_tokens * (D / 2) * 2 * sizeof(float);
    int rc = ensure_buffer(&c->layer_tmp, &c->layer_tmp_bytes, y_bytes + qkv_bytes + cs_bytes);
    if (rc != GQA_OK) return rc;
    if (!c->lt) {
        const hipblasStatus_t st = hipblasLtCreate(&c->lt);
        if (st != HIPBLAS_STATUS_SUCCESS) {
            c->lt = nullptr;
            snprintf(g_last_error, sizeof(g_last_error), "hipblasLtCreate: status %d", (int)st);
            return GQA_ERR_HIP;
        }
    }
    if (stage_events && !c->ev_layer[0])
        for (int i = 0; i < 4; ++i) HIP_TRY(hipEventCreate(&c->ev_layer[i]));
    c->layer_timed = false;
    auto mark = [&](int i) { return stage_events ? hipEventRecord(c->ev_layer[i], s) : hipSuccess; };
    // While profiling (device calls), the projection's hipBLASLt kernels are bracketed by the next
    // event pair of its timer slot; RMSNorm and RoPE have event pairs bound to their launches.
    const Launch proj_events = stage_events ? Launch{s} : timed(c, GQA_TIMER_PROJECTION, s);
    HIP_TRY(mark(0));
    const uint16_t* src = (const uint16_t*)x;
    float* cs = rope ? reinterpret_cast<float*>(c->layer_tmp + y_bytes + qkv_bytes) : nullptr;
    if (gamma || rope) {
        // The RMSNorm launch also fills the RoPE table (the table alone without normalisation).
        NormArgs na{};
        na.x = (const uint16_t*)x;
        na.gamma = (const uint16_t*)gamma;
        na.y = (uint16_t*)c->layer_tmp;
        na.n_tokens = n_tokens;
        na.hidden = hidden;
        na.eps = eps;
        na.table.cs = cs;
        na.table.sets = cs_sets;
        na.table.pairs = D / 2;
        na.table.n_tokens = n_tokens;
        na.table.q_pos_base = q_pos_base;
        na.table.kv_pos_base = kv_pos_base;
        for (int p = 0; p < D / 2; ++p) na.table.theta[p] = (float)pow(kRopeBase, -2.0 * p / D);
        HIP_TRY(launch_rms_norm(na, stage_events ? Launch{s} : timed(c, GQA_TIMER_NORM, s)));
        if (gamma) src = na.y;
    }
    HIP_TRY(mark(1));
    if (proj_events.start) HIP_TRY(hipEventRecord(proj_events.start, s));  // after the norm launch
    uint16_t* qkv = (uint16_t*)(c->layer_tmp + y_bytes);
    const float one = 1.f, zero = 0.f;
    const void* ws[3] = {wq, wk, wv};
    int rows[3] = {nq, nkv, nkv}, off[3] = {0, nq, nq + nkv};
    int n_gemm = 3;
    // Wq, Wk, Wv stored back to back ([H_q + 2 H_kv][D][hidden]) are one fused projection.
    const size_t row_bytes = (size_t)hidden * 2;
    if ((const uint8_t*)wk == (const uint8_t*)wq + (size_t)nq * row_bytes &&
        (const uint8_t*)wv == (const uint8_t*)wk + (size_t)nkv * row_bytes) {
        rows[0] = ld;
        n_gemm = 1;
    }
    for (int i = 0; i < n_gemm; ++i) {
        ProjectionPlan* p = nullptr;
        rc = projection_plan(c, rows[i], n_tokens, hidden, ld, &p);
        if (rc != GQA_OK) return rc;
        const bool tune = !p->tuned && !stream_capturing(s);
        size_t ws_need = p->cand[p->pick].workspaceSize;
        if (tune)
            for (int k = 0; k < p->n_cand; ++k) ws_need = std::max(ws_need, p->cand[k].workspaceSize);
        rc = ensure_buffer(&c->lt_ws, &c->lt_ws_bytes, std::max<size_t>(ws_need, 256));
        if (rc != GQA_OK) return rc;
        auto gemm = [&](int k) {
            return hipblasLtMatmul(c->lt, p->desc, &one, ws[i], p->w, src, p->x, &zero, qkv + off[i], p->d,
                                   qkv + off[i], p->d, &p->cand[k].algo, c->lt_ws, p->cand[k].workspaceSize, s);
        };
        if (tune) {
            rc = tune_projection(c, p, gemm, s);
            if (rc != GQA_OK) return rc;
        }
        const hipblasStatus_t st = gemm(p->pick);
        if (st != HIPBLAS_STATUS_SUCCESS) {
            snprintf(g_last_error, sizeof(g_last_error), "hipblasLtMatmul: status %d", (int)st);
            return GQA_ERR_HIP;
        }
    }
    if (proj_events.stop) HIP_TRY(hipEventRecord(proj_events.stop, s));
    HIP_TRY(mark(2));
    RopeArgs ra{};
    ra.qkv = qkv;
    ra.ld = ld;
    ra.n_tokens = n_tokens;
    ra.n_q_heads = c->cfg.n_q_heads;
    ra.n_kv_heads = c->cfg.n_kv_heads;
    ra.head_dim = D;
    ra.rope = rope ? 1 : 0;
    ra.cs = cs;
    ra.cs_k_set = cs_sets == 2 ? 1 : 0;
    ra.q_out = (uint16_t*)q_out;
    const size_t seq = c->paged ? 0 : (size_t)b * c->cfg.n_kv_heads * c->l_cap * D;
    ra.kc = c->k_cache + seq;
    ra.vc = c->v_cache + seq;
    ra.block_table = c->paged ? c->table_dev + (size_t)b * c->max_pages : nullptr;
    ra.page_shift = c->page_shift;
    ra.l_cap = c->l_cap;
    ra.row0 = row0;
    HIP_TRY(launch_rope_scatter(ra, stage_events ? Launch{s} : timed(c, GQA_TIMER_ROPE, s)));
    HIP_TRY(mark(3));
    c->layer_timed = stage_events;
    return GQA_OK;
}

int layer_times(gqa_ctx* c) {
    HIP_TRY(hipEventSynchronize(c->ev_layer[3]));
    for (int i = 0; i < 3; ++i) {
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, c->ev_layer[i], c->ev_layer[i + 1]));
        c->layer_us[i] = ms * 1000.f;
    }
    return GQA_OK;
}

// Largest segmented-plan workspace (floats) over every query length up to max_q_len, keys up
// to max_seq_len, for a work-group target.
size_t prefill_workspace_need(const gqa_ctx* c, int target_wgs) {
    const gqa_config& k = c->cfg;
    size_t need = 0;
    for (int q_len = 32; q_len < k.max_q_len + 32; q_len += 32) {
        const int ql = q_len < k.max_q_len ? q_len : k.max_q_len;
        const PrefillPlan p = plan_prefill(ql, k.max_seq_len, c->group, k.n_kv_heads, target_wgs, kMaxPrefillSegs);
        const size_t f = prefill_workspace_floats(p, ql, k.n_q_heads, k.head_dim);
        if (f > need) need = f;
    }
    return need;
}

int create_ctx(const gqa_config* cfg, int32_t page_size, int32_t n_pages, int32_t n_layers, gqa_ctx** out_ctx) {
    if (!cfg || !out_ctx) return GQA_ERR_NULL;
    *out_ctx = nullptr;
    const gqa_config& k = *cfg;
    if (k.batch < 1 || k.n_q_heads < 1 || k.n_kv_heads < 1 || k.n_q_heads % k.n_kv_heads != 0 ||
        k.max_seq_len < 1 || k.max_q_len < 1 || k.max_seq_len > kMaxRows || k.max_q_len > kMaxRows ||
        !(k.scale >= 0.f) || !isfinite(k.scale))
        return GQA_ERR_BAD_CFG;
    const int group = k.n_q_heads / k.n_kv_heads;
    if (!decode_supported(k.head_dim, group) && !prefill_supported(k.head_dim, group)) return GQA_ERR_UNSUPPORTED;

    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) return GQA_ERR_NO_DEVICE;
    if (k.device < 0 || k.device >= n) return GQA_ERR_NO_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, k.device) != hipSuccess) return GQA_ERR_NO_DEVICE;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return GQA_ERR_NO_DEVICE;
    HIP_TRY(hipSetDevice(k.device));

    gqa_ctx* c = new gqa_ctx();
    c->cfg = k;
    c->group = group;
    c->l_cap = ((k.max_seq_len + 63) / 64) * 64;
    // Enough partial slots for any plan: the automatic one at either work-group shape, or forced
    // chunks down to kMinSplitCap keys.
    c->max_splits_cap = std::max((c->l_cap + kMinSplitCap - 1) / kMinSplitCap,
                                 plan_splits(k.batch, k.n_kv_heads,
                                             prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256,
                                             kDecodeWavesSmall));
    c->scale = k.scale > 0.f ? k.scale : (float)(1.0 / sqrt((double)k.head_dim));
    c->cfg.scale = c->scale;
    c->clock_mhz = prop.clockRate / 1000.0;
    if (prop.multiProcessorCount > 0) c->n_cu = prop.multiProcessorCount;
    if (page_size > 0) {
        c->paged = 1;
        c->page_size = page_size;
        while ((1 << c->page_shift) < page_size) ++c->page_shift;
        c->n_pages = n_pages;
        c->max_pages = (k.max_seq_len + page_size - 1) / page_size;
        c->pages = PageTable(k.batch, c->max_pages, n_pages);
    }
    c->n_layers = n_layers;
    const size_t D = (size_t)k.head_dim;
    const size_t units = (size_t)k.batch * k.n_kv_heads;
    c->stage_words = (size_t)k.n_q_heads * D * (size_t)(k.batch > k.max_q_len ? k.batch : k.max_q_len);
    c->lse_words = (size_t)k.n_q_heads * (size_t)(k.batch > k.max_q_len ? k.batch : k.max_q_len);

    int rc = GQA_OK;
    auto alloc = [&](void** p, size_t bytes) {
        if (rc != GQA_OK) return;
        if (hipMalloc(p, bytes) != hipSuccess) rc = GQA_ERR_OOM;
    };
    alloc((void**)&c->k_pool, kv_words(c) * 2 * (size_t)n_layers);
    alloc((void**)&c->v_pool, kv_words(c) * 2 * (size_t)n_layers);
    c->k_cache = c->k_pool;
    c->v_cache = c->v_pool;
    alloc((void**)&c->part_o, units * c->max_splits_cap * group * D * sizeof(float));
    alloc((void**)&c->part_ml, units * c->max_splits_cap * group * 2 * sizeof(float));
    alloc((void**)&c->arrivals, (units + 1) * sizeof(int32_t));
    if (prefill_supported(k.head_dim, group)) {
        c->pre_ws_floats = prefill_workspace_need(c, c->n_cu);
        if (c->pre_ws_floats > 0) alloc((void**)&c->pre_ws, c->pre_ws_floats * sizeof(float));
    }
    alloc((void**)&c->q_dev, c->stage_words * 2);
    alloc((void**)&c->o_dev, c->stage_words * 2);
    alloc((void**)&c->lse_dev, c->lse_words * sizeof(float));
    alloc((void**)&c->lens_dev, (size_t)k.batch * sizeof(int32_t));
    alloc((void**)&c->zero_row, D * 2);
    alloc((void**)&c->pos_dev, (size_t)k.batch * sizeof(int32_t));
    alloc((void**)&c->rows_dev, 2 * units * D * 2);
    alloc((void**)&c->new_dev, 2 * (size_t)k.n_kv_heads * k.max_q_len * D * 2);
    if (c->paged) alloc((void**)&c->table_dev, (size_t)k.batch * c->max_pages * sizeof(int32_t));
    if (rc == GQA_OK && hipHostMalloc((void**)&c->o_pinned, c->stage_words * 2, 0) != hipSuccess) rc = GQA_ERR_OOM;
    // A blocking stream: ordered both ways with the legacy default stream, so a caller that
    // passes NULL (for instance PyTorch's default stream, whose handle is 0) sees its own
    // earlier default-stream work finish before the library reads it, and vice versa.
    if (rc == GQA_OK && hipStreamCreateWithFlags(&c->stream, hipStreamDefault) != hipSuccess) rc = GQA_ERR_HIP;
    if (rc == GQA_OK) {
        bool ok = hipEventCreate(&c->ev_begin) == hipSuccess && hipEventCreate(&c->ev_end) == hipSuccess;
        for (int i = 0; i < 4 && ok; ++i) ok = hipEventCreate(&c->ev_t[i]) == hipSuccess;
        if (!ok) rc = GQA_ERR_HIP;
    }
    // Zero the caches (every layer's pool) once so rows beyond every sequence's length hold finite words.
    if (rc == GQA_OK && (hipMemsetAsync(c->zero_row, 0, D * 2, c->stream) != hipSuccess ||
                         hipMemsetAsync(c->arrivals, 0, (units + 1) * sizeof(int32_t), c->stream) != hipSuccess ||
                         hipMemsetAsync(c->k_pool, 0, kv_words(c) * 2 * (size_t)n_layers, c->stream) != hipSuccess ||
                         hipMemsetAsync(c->v_pool, 0, kv_words(c) * 2 * (size_t)n_layers, c->stream) != hipSuccess ||
                         (c->paged && hipMemsetAsync(c->table_dev, 0xFF, (size_t)k.batch * c->max_pages * 4,
                                                     c->stream) != hipSuccess) ||  // every entry -1: unmapped
                         hipStreamSynchronize(c->stream) != hipSuccess))
        rc = GQA_ERR_HIP;
    if (rc != GQA_OK) {
        gqa_destroy(c);
        return rc;
    }
    *out_ctx = c;
    return GQA_OK;
}


// Uploads sequence b's block-table row (host -> device, synchronous on the context stream).
int upload_table_row(gqa_ctx* c, int b) {
    HIP_TRY(hipMemcpyAsync(c->table_dev + (size_t)b * c->max_pages, c->pages.row(b),
                           (size_t)c->max_pages * sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return GQA_OK;
}

// Copies rows [start, start + n) of [H_kv][n][D] K and V between a caller buffer and a paged
// cache, one strided copy (over the kv heads) per page the range touches.
int copy_rows_paged(gqa_ctx* c, int b, int start, int n, const uint16_t* k_src, const uint16_t* v_src,
                    uint16_t* k_dst, uint16_t* v_dst, hipMemcpyKind kind, hipStream_t s) {
    const size_t D = c->cfg.head_dim;
    const size_t pitch_pool = (size_t)c->page_size * D * 2;  // bytes between kv heads in a page
    const size_t pitch_buf = (size_t)n * D * 2;              // bytes between kv heads in the buffer
    for (int t = start; t < start + n;) {
        const int t1 = std::min(start + n, ((t >> c->page_shift) + 1) << c->page_shift);
        const int64_t row = cache_row(c, b, 0, t);
        if (row < 0) return GQA_ERR_RANGE;
        const size_t width = (size_t)(t1 - t) * D * 2;
        const size_t buf = (size_t)(t - start) * D;
        if (kind == hipMemcpyDeviceToHost) {
            HIP_TRY(hipMemcpy2DAsync(k_dst + buf, pitch_buf, c->k_cache + row * D, pitch_pool, width,
                                     c->cfg.n_kv_heads, kind, s));
            HIP_TRY(hipMemcpy2DAsync(v_dst + buf, pitch_buf, c->v_cache + row * D, pitch_pool, width,
                                     c->cfg.n_kv_heads, kind, s));
        } else {
            HIP_TRY(hipMemcpy2DAsync(c->k_cache + row * D, pitch_pool, k_src + buf, pitch_buf, width,
                                     c->cfg.n_kv_heads, kind, s));
            HIP_TRY(hipMemcpy2DAsync(c->v_cache + row * D, pitch_pool, v_src + buf, pitch_buf, width,
                                     c->cfg.n_kv_heads, kind, s));
        }
        t = t1;
    }
    return GQA_OK;
}

}  // namespace

// ---- decode without allocation (gqa_decode_append_noalloc) ---------------------------------
// Split-KV partials of gqa_decode_append_noalloc: one copy per device, held until the process
// ends.  Its tail holds the split arrival counters of the fused merge (kNoAllocCounters, zero
// between launches: the last split to arrive resets its counter) and, last, the zero K/V row (the
// source of rows past a sequence's length, never written); both are cleared at set-up.  Host code
// uses the per-device address from hipGetSymbolAddress, never this name.
static __device__ __align__(256) uint8_t scratch[GQA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kNoAllocDevices = 64;
constexpr size_t kNoAllocZeroBytes = 256;  // one K/V row of D <= 128 bf16 words
constexpr int kNoAllocCounters = 1024;     // (sequence, kv head) units the fused merge can count
constexpr size_t kNoAllocTailBytes = kNoAllocCounters * sizeof(int32_t) + kNoAllocZeroBytes;
constexpr size_t kNoAllocPartialBytes = GQA_NOALLOC_SCRATCH_BYTES - kNoAllocTailBytes;

struct NoAllocDevice {
    bool ready = false;
    uint8_t* scratch = nullptr;      // device address of `scratch` on this device
    int32_t* arrivals = nullptr;     // its split arrival counters
    const uint16_t* zero = nullptr;  // its zero row
    int n_cu = 0;
};

NoAllocDevice g_noalloc[kNoAllocDevices];
std::mutex g_noalloc_mu;

// Once per device, with that device current and outside any stream capture: the device address of
// `scratch`, the zero row cleared (and finished before any launch that reads it), and the CU count
// the split planner targets.
int noalloc_setup(int device, hipStream_t stream, NoAllocDevice** out) {
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    NoAllocDevice& d = g_noalloc[device];
    if (!d.ready) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        HIP_TRY(hipStreamIsCapturing(stream, &cs));
        if (cs != hipStreamCaptureStatusNone) return GQA_ERR_UNSUPPORTED;  // set-up cannot be captured
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, device) != hipSuccess || strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            return GQA_ERR_NO_DEVICE;
        void* p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        uint8_t* base = static_cast<uint8_t*>(p);
        HIP_TRY(hipMemset(base + kNoAllocPartialBytes, 0, kNoAllocTailBytes));
        HIP_TRY(hipDeviceSynchronize());
        d.scratch = base;
        d.arrivals = reinterpret_cast<int32_t*>(base + kNoAllocPartialBytes);
        d.zero = reinterpret_cast<const uint16_t*>(base + kNoAllocPartialBytes + kNoAllocCounters * sizeof(int32_t));
        d.n_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
        d.ready = true;
    }
    *out = &d;
    return GQA_OK;
}

}  // namespace

extern "C" {

const char* gqa_status_string(int32_t code) {
    switch (code) {
        case GQA_OK: return "ok";
        case GQA_ERR_BAD_CFG: return "bad configuration";
        case GQA_ERR_BUSY_START: return "start while a transaction is running";
        case GQA_ERR_STREAM_LEN: return "payload length does not match the configured shape";
        case GQA_ERR_STREAM_DEST: return "bad destination (sequence index)";
        case GQA_ERR_RESULT_LEN: return "result length does not match the transaction";
        case GQA_ERR_HIP: return g_last_error[0] ? g_last_error : "HIP runtime error";
        case GQA_ERR_OOM: return "out of device or pinned host memory";
        case GQA_ERR_NO_DEVICE: return "no usable gfx950 device";
        case GQA_ERR_NULL: return "required pointer is NULL";
        case GQA_ERR_RANGE: return "length or position outside the configured capacity";
        case GQA_ERR_TIMEOUT: return "timed out waiting for the transaction";
        case GQA_ERR_NO_TRANSACTION: return "no transaction has been submitted";
        case GQA_ERR_UNSUPPORTED: return "no kernel compiled for this head_dim / group size";
        case GQA_ERR_SCRATCH: return "the split plan needs more than the no-allocation scratch (GQA_NOALLOC_SCRATCH_BYTES)";
        default: return "unknown status";
    }
}

int gqa_device_count(int32_t* out_count) {
    if (!out_count) return GQA_ERR_NULL;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *out_count = (e == hipSuccess) ? n : 0;
    return GQA_OK;
}

int gqa_create(const gqa_config* cfg, gqa_ctx** out_ctx) { return create_ctx(cfg, 0, 0, 1, out_ctx); }

int gqa_create_paged(const gqa_config* cfg, int32_t page_size, int32_t n_pages, gqa_ctx** out_ctx) {
    if (!cfg || !out_ctx) return GQA_ERR_NULL;
    *out_ctx = nullptr;
    if (page_size < 64 || page_size > (1 << 16) || (page_size & (page_size - 1)) != 0 || n_pages < 1)
        return GQA_ERR_BAD_CFG;
    return create_ctx(cfg, page_size, n_pages, 1, out_ctx);
}

int gqa_create_paged_layers(const gqa_config* cfg, int32_t page_size, int32_t n_pages, int32_t n_layers,
                            gqa_ctx** out_ctx) {
    if (!cfg || !out_ctx) return GQA_ERR_NULL;
    *out_ctx = nullptr;
    if (page_size < 64 || page_size > (1 << 16) || (page_size & (page_size - 1)) != 0 || n_pages < 1 ||
        n_layers < 1 || n_layers > GQA_MAX_LAYERS)
        return GQA_ERR_BAD_CFG;
    return create_ctx(cfg, page_size, n_pages, n_layers, out_ctx);
}

int gqa_destroy(gqa_ctx* c) {
    if (!c) return GQA_ERR_NULL;
    (void)hipSetDevice(c->cfg.device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    (void)hipFree(c->k_pool);
    (void)hipFree(c->v_pool);
    (void)hipFree(c->part_o);
    (void)hipFree(c->part_ml);
    (void)hipFree(c->arrivals);
    (void)hipFree(c->pre_ws);
    (void)hipFree(c->zero_row);
    (void)hipFree(c->q_dev);
    (void)hipFree(c->o_dev);
    (void)hipFree(c->lse_dev);
    (void)hipFree(c->lens_dev);
    (void)hipFree(c->pos_dev);
    (void)hipFree(c->rows_dev);
    (void)hipFree(c->new_dev);
    (void)hipFree(c->table_dev);
    if (c->o_pinned) (void)hipHostFree(c->o_pinned);
    if (c->ev_begin) (void)hipEventDestroy(c->ev_begin);
    if (c->ev_end) (void)hipEventDestroy(c->ev_end);
    for (int i = 0; i < GQA_TIMER_COUNT; ++i) {
        if (!c->ev_pool[i]) continue;
        for (int e = 0; e < 2 * kProfileLaunches; ++e)
            if (c->ev_pool[i][e]) (void)hipEventDestroy(c->ev_pool[i][e]);
        free(c->ev_pool[i]);
    }
    for (int i = 0; i < 4; ++i)
        if (c->ev_t[i]) (void)hipEventDestroy(c->ev_t[i]);
    for (ProjectionPlan& p : c->proj) release_plan(p);
    if (c->lt) (void)hipblasLtDestroy(c->lt);
    (void)hipFree(c->layer_in);
    (void)hipFree(c->layer_tmp);
    (void)hipFree(c->lt_ws);
    for (int i = 0; i < 4; ++i)
        if (c->ev_layer[i]) (void)hipEventDestroy(c->ev_layer[i]);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return GQA_OK;
}

int gqa_get_config(const gqa_ctx* c, gqa_config* out) {
    if (!c || !out) return GQA_ERR_NULL;
    *out = c->cfg;
    return GQA_OK;
}

int gqa_set_option(gqa_ctx* c, int32_t option, int64_t value) {
    if (!c) return GQA_ERR_NULL;
    switch (option) {
        case GQA_OPT_DECODE_CHUNK:
            if (value < 0 || (value > 0 && (value % kChunkOptionQuantum != 0 || value > c->l_cap + kChunkOptionQuantum ||
                                            decode_split_count(c->cfg.max_seq_len, (int)value) > c->max_splits_cap)))
                return GQA_ERR_RANGE;
            c->chunk_opt = (int)value;
            return GQA_OK;
        case GQA_OPT_PROFILE:
            return profile_enable(c, value ? 1 : 0);
        case GQA_OPT_PREFILL_KERNEL:
            if (value != GQA_PREFILL_KERNEL_AUTO && value != GQA_PREFILL_KERNEL_SHARED &&
                value != GQA_PREFILL_KERNEL_ROWS && value != GQA_PREFILL_KERNEL_PAIRED)
                return GQA_ERR_RANGE;
            c->prefill_kernel = (int)value;
            return GQA_OK;
        case GQA_OPT_DECODE_MERGE:
            if (value != GQA_DECODE_MERGE_AUTO && value != GQA_DECODE_MERGE_FUSED && value != GQA_DECODE_MERGE_LAUNCH)
                return GQA_ERR_RANGE;
            c->decode_merge = (int)value;
            return GQA_OK;
        case GQA_OPT_LAYER: {
            if (value < 0 || value >= c->n_layers) return GQA_ERR_RANGE;
            const size_t off = kv_words(c) * (size_t)value;
            c->layer = (int)value;
            c->k_cache = c->k_pool + off;
            c->v_cache = c->v_pool + off;
            return GQA_OK;
        }
        case GQA_OPT_NUMERICS:
            if (value != GQA_NUMERICS_EXACT && value != GQA_NUMERICS_KV260) return GQA_ERR_RANGE;
            if (value == GQA_NUMERICS_KV260 && ((c->cfg.head_dim != 64 && c->cfg.head_dim != 128) || c->paged))
                return GQA_ERR_UNSUPPORTED;
            c->numerics = (int)value;
            return GQA_OK;
        case GQA_OPT_PREFILL_WGS: {
            if (value < 0 || value > (1 << 20)) return GQA_ERR_RANGE;
            if (!prefill_supported(c->cfg.head_dim, c->group)) {
                c->prefill_wgs_opt = (int)value;
                return GQA_OK;
            }
            // Grow the segment workspace for the new target (kept if it already suffices).
            const size_t need = prefill_workspace_need(c, value > 0 ? (int)value : c->n_cu);
            if (need > c->pre_ws_floats) {
                int rc = txn_idle(c);
                if (rc != GQA_OK) return rc;
                HIP_TRY(hipSetDevice(c->cfg.device));
                HIP_TRY(hipDeviceSynchronize());
                float* ws = nullptr;
                if (hipMalloc(&ws, need * sizeof(float)) != hipSuccess) return GQA_ERR_OOM;
                (void)hipFree(c->pre_ws);
                c->pre_ws = ws;
                c->pre_ws_floats = need;
            }
            c->prefill_wgs_opt = (int)value;
            return GQA_OK;
        }
        default:
            return GQA_ERR_BAD_CFG;
    }
}

int gqa_cache_pointers(gqa_ctx* c, void** k, void** v, int32_t* l_cap) {
    if (!c) return GQA_ERR_NULL;
    if (k) *k = c->k_cache;
    if (v) *v = c->v_cache;
    if (l_cap) *l_cap = c->paged ? c->page_size : c->l_cap;
    return GQA_OK;
}

// ---- paged cache management ------------------------------------------------------------

int gqa_paged_reserve(gqa_ctx* c, int32_t b, int32_t n_rows) {
    if (!c) return GQA_ERR_NULL;
    if (!c->paged) return GQA_ERR_UNSUPPORTED;
    if (b < 0 || b >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
    if (n_rows < 0 || n_rows > c->cfg.max_seq_len) return GQA_ERR_RANGE;
    const int before = c->pages.mapped(b);
    if (!c->pages.reserve(b, n_rows, c->page_size)) return GQA_ERR_OOM;
    if (c->pages.mapped(b) == before) return GQA_OK;
    HIP_TRY(hipSetDevice(c->cfg.device));
    return upload_table_row(c, b);
}

int gqa_paged_release(gqa_ctx* c, int32_t b) {
    if (!c) return GQA_ERR_NULL;
    if (!c->paged) return GQA_ERR_UNSUPPORTED;
    if (b < 0 || b >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipSetDevice(c->cfg.device));
    HIP_TRY(hipStreamSynchronize(c->stream));  // no launch on the context stream still reads the pages
    c->pages.release(b);
    return upload_table_row(c, b);
}

int gqa_paged_evict_lru(gqa_ctx* c, int32_t n_free_pages, const int32_t* pinned, int32_t n_pinned,
                        int32_t* evicted, int32_t max_evicted, int32_t* n_evicted) {
    if (!c || (n_pinned > 0 && !pinned)) return GQA_ERR_NULL;
    if (!c->paged) return GQA_ERR_UNSUPPORTED;
    if (n_free_pages < 0 || n_free_pages > c->n_pages || n_pinned < 0 || max_evicted < 0) return GQA_ERR_RANGE;
    std::vector<char> pin(c->cfg.batch, 0);
    for (int i = 0; i < n_pinned; ++i) {
        if (pinned[i] < 0 || pinned[i] >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
        pin[pinned[i]] = 1;
    }
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipSetDevice(c->cfg.device));
    HIP_TRY(hipStreamSynchronize(c->stream));
    std::vector<int> out;
    if (!c->pages.evict_lru(n_free_pages, pin, &out)) return GQA_ERR_OOM;
    for (int b : out) {
        rc = upload_table_row(c, b);
        if (rc != GQA_OK) return rc;
    }
    if (n_evicted) *n_evicted = (int32_t)out.size();
    for (int i = 0; i < (int)out.size() && i < max_evicted && evicted; ++i) evicted[i] = out[i];
    return GQA_OK;
}

int gqa_paged_info(gqa_ctx* c, int32_t* page_size, int32_t* n_pages, int32_t* n_free, int32_t* max_pages) {
    if (!c) return GQA_ERR_NULL;
    if (!c->paged) return GQA_ERR_UNSUPPORTED;
    if (page_size) *page_size = c->page_size;
    if (n_pages) *n_pages = c->n_pages;
    if (n_free) *n_free = c->pages.free_pages();
    if (max_pages) *max_pages = c->max_pages;
    return GQA_OK;
}

int gqa_paged_layers(gqa_ctx* c, int32_t* n_layers, int32_t* layer) {
    if (!c) return GQA_ERR_NULL;
    if (!c->paged) return GQA_ERR_UNSUPPORTED;
    if (n_layers) *n_layers = c->n_layers;
    if (layer) *layer = c->layer;
    return GQA_OK;
}

int gqa_paged_table(gqa_ctx* c, int32_t b, int32_t* out, int32_t n) {
    if (!c || !out) return GQA_ERR_NULL;
    if (!c->paged) return GQA_ERR_UNSUPPORTED;
    if (b < 0 || b >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
    if (n < 0 || n > c->max_pages) return GQA_ERR_RANGE;
    memcpy(out, c->pages.row(b), (size_t)n * sizeof(int32_t));
    return GQA_OK;
}

int gqa_load_kv(gqa_ctx* c, int32_t b, int32_t start_pos, int32_t n, const uint16_t* k, const uint16_t* v) {
    if (!c || !k || !v) return GQA_ERR_NULL;
    if (b < 0 || b >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
    if (n < 0 || start_pos < 0 || (int64_t)start_pos + n > c->cfg.max_seq_len) return GQA_ERR_RANGE;
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    if (n == 0) return GQA_OK;
    HIP_TRY(hipSetDevice(c->cfg.device));
    if (c->paged) {
        if (!rows_backed(c, b, start_pos, n)) return GQA_ERR_RANGE;
        c->pages.touch(b);
        HIP_TRY(hipEventRecord(c->ev_begin, c->stream));
        rc = copy_rows_paged(c, b, start_pos, n, k, v, nullptr, nullptr, hipMemcpyHostToDevice, c->stream);
        if (rc != GQA_OK) return rc;
        return finish_sync(c);
    }
    const size_t D = c->cfg.head_dim;
    const size_t row_bytes = D * 2;
    HIP_TRY(hipEventRecord(c->ev_begin, c->stream));
    for (int h = 0; h < c->cfg.n_kv_heads; ++h) {
        const size_t dst = (((size_t)b * c->cfg.n_kv_heads + h) * c->l_cap + start_pos) * D;
        const size_t src = (size_t)h * n * D;
        HIP_TRY(hipMemcpyAsync(c->k_cache + dst, k + src, n * row_bytes, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(hipMemcpyAsync(c->v_cache + dst, v + src, n * row_bytes, hipMemcpyHostToDevice, c->stream));
    }
    return finish_sync(c);
}

int gqa_load_kv_device(gqa_ctx* c, int32_t b, int32_t start_pos, int32_t n, const void* k, const void* v,
                       void* stream) {
    if (!c || !k || !v) return GQA_ERR_NULL;
    if (b < 0 || b >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
    if (n < 0 || start_pos < 0 || (int64_t)start_pos + n > c->cfg.max_seq_len) return GQA_ERR_RANGE;
    if (n == 0) return GQA_OK;
    hipStream_t s = pick_stream(c, stream);
    if (c->paged) {
        if (!rows_backed(c, b, start_pos, n)) return GQA_ERR_RANGE;
        c->pages.touch(b);
        return copy_rows_paged(c, b, start_pos, n, (const uint16_t*)k, (const uint16_t*)v, nullptr, nullptr,
                               hipMemcpyDeviceToDevice, s);
    }
    const size_t D = c->cfg.head_dim;
    const size_t pitch_dst = (size_t)c->l_cap * D * 2;   // bytes between kv heads in the cache
    const size_t pitch_src = (size_t)n * D * 2;          // bytes between kv heads in the source
    const size_t dst = ((size_t)b * c->cfg.n_kv_heads * c->l_cap + start_pos) * D;
    HIP_TRY(hipMemcpy2DAsync(c->k_cache + dst, pitch_dst, k, pitch_src, pitch_src, c->cfg.n_kv_heads,
                             hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpy2DAsync(c->v_cache + dst, pitch_dst, v, pitch_src, pitch_src, c->cfg.n_kv_heads,
                             hipMemcpyDeviceToDevice, s));
    return GQA_OK;
}

int gqa_read_kv(gqa_ctx* c, int32_t b, int32_t start_pos, int32_t n, uint16_t* k, uint16_t* v) {
    if (!c || !k || !v) return GQA_ERR_NULL;
    if (b < 0 || b >= c->cfg.batch) return GQA_ERR_STREAM_DEST;
    if (n < 0 || start_pos < 0 || (int64_t)start_pos + n > c->cfg.max_seq_len) return GQA_ERR_RANGE;
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    if (n == 0) return GQA_OK;
    HIP_TRY(hipSetDevice(c->cfg.device));
    if (c->paged) {
        if (!rows_backed(c, b, start_pos, n)) return GQA_ERR_RANGE;
        rc = copy_rows_paged(c, b, start_pos, n, nullptr, nullptr, k, v, hipMemcpyDeviceToHost, c->stream);
        if (rc != GQA_OK) return rc;
        HIP_TRY(hipStreamSynchronize(c->stream));
        return GQA_OK;
    }
    const size_t D = c->cfg.head_dim;
    for (int h = 0; h < c->cfg.n_kv_heads; ++h) {
        const size_t src = (((size_t)b * c->cfg.n_kv_heads + h) * c->l_cap + start_pos) * D;
        const size_t dst = (size_t)h * n * D;
        HIP_TRY(hipMemcpyAsync(k + dst, c->k_cache + src, n * D * 2, hipMemcpyDeviceToHost, c->stream));
        HIP_TRY(hipMemcpyAsync(v + dst, c->v_cache + src, n * D * 2, hipMemcpyDeviceToHost, c->stream));
    }
    HIP_TRY(hipStreamSynchronize(c->stream));
    return GQA_OK;
}

int gqa_append_kv(gqa_ctx* c, const uint16_t* k_rows, const uint16_t* v_rows, const int32_t* positions) {
    if (!c || !k_rows || !v_rows || !positions) return GQA_ERR_NULL;
    for (int b = 0; b < c->cfg.batch; ++b) {
        if (positions[b] < -1 || positions[b] >= c->cfg.max_seq_len) return GQA_ERR_RANGE;
        if (positions[b] >= 0 && !rows_backed(c, b, positions[b], 1)) return GQA_ERR_RANGE;
    }
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipSetDevice(c->cfg.device));
    const size_t row_words = (size_t)c->cfg.batch * c->cfg.n_kv_heads * c->cfg.head_dim;
    HIP_TRY(hipEventRecord(c->ev_begin, c->stream));
    HIP_TRY(hipMemcpyAsync(c->rows_dev, k_rows, row_words * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->rows_dev + row_words, v_rows, row_words * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->lens_dev, positions, c->cfg.batch * sizeof(int32_t), hipMemcpyHostToDevice,
                           c->stream));
    rc = gqa_append_kv_device(c, c->rows_dev, c->rows_dev + row_words, c->lens_dev, nullptr);
    if (rc != GQA_OK) return rc;
    return finish_sync(c);
}

int gqa_append_kv_device(gqa_ctx* c, const void* k_rows, const void* v_rows, const int32_t* positions,
                         void* stream) {
    if (!c || !k_rows || !v_rows || !positions) return GQA_ERR_NULL;
    hipStream_t s = pick_stream(c, stream);
    HIP_TRY(launch_append((const uint16_t*)k_rows, (const uint16_t*)v_rows, positions, c->k_cache, c->v_cache,
                          c->cfg.batch, c->cfg.n_kv_heads, c->cfg.head_dim, c->l_cap, c->cfg.max_seq_len,
                          c->paged ? c->table_dev : nullptr, c->page_shift, c->max_pages,
                          timed(c, GQA_TIMER_APPEND, s)));
    return GQA_OK;
}

int gqa_decode(gqa_ctx* c, const uint16_t* q, const int32_t* ctx_lens, uint16_t* o, float* lse) {
    if (!c || !q || !ctx_lens || !o) return GQA_ERR_NULL;
    int max_len = 0;
    for (int b = 0; b < c->cfg.batch; ++b) {
        if (ctx_lens[b] < 0 || ctx_lens[b] > c->cfg.max_seq_len) return GQA_ERR_RANGE;
        if (!rows_backed(c, b, 0, ctx_lens[b])) return GQA_ERR_RANGE;
        if (ctx_lens[b] > max_len) max_len = ctx_lens[b];
    }
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipSetDevice(c->cfg.device));
    if (c->paged)
        for (int b = 0; b < c->cfg.batch; ++b)
            if (ctx_lens[b] > 0) c->pages.touch(b);
    const size_t qwords = (size_t)c->cfg.batch * c->cfg.n_q_heads * c->cfg.head_dim;
    HIP_TRY(hipEventRecord(c->ev_begin, c->stream));
    HIP_TRY(hipMemcpyAsync(c->q_dev, q, qwords * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->lens_dev, ctx_lens, c->cfg.batch * sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
    rc = run_decode(c, c->q_dev, c->lens_dev, nullptr, nullptr, nullptr, c->o_dev, lse ? c->lse_dev : nullptr,
                    c->stream, max_len);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipMemcpyAsync(o, c->o_dev, qwords * 2, hipMemcpyDeviceToHost, c->stream));
    if (lse)
        HIP_TRY(hipMemcpyAsync(lse, c->lse_dev, (size_t)c->cfg.batch * c->cfg.n_q_heads * sizeof(float),
                               hipMemcpyDeviceToHost, c->stream));
    return finish_sync(c);
}

int gqa_decode_device(gqa_ctx* c, const void* q, const int32_t* ctx_lens, void* o, float* lse, void* stream) {
    if (!c || !q || !ctx_lens || !o) return GQA_ERR_NULL;
    if (!aligned16(q)) return GQA_ERR_RANGE;
    return run_decode(c, q, ctx_lens, nullptr, nullptr, nullptr, o, lse, pick_stream(c, stream), c->cfg.max_seq_len);
}

int gqa_decode_append(gqa_ctx* c, const uint16_t* q, const uint16_t* k_rows, const uint16_t* v_rows,
                      const int32_t* positions, const int32_t* ctx_lens, uint16_t* o, float* lse) {
    if (!c || !q || !k_rows || !v_rows || !positions || !ctx_lens || !o) return GQA_ERR_NULL;
    int max_len = 0;
    for (int b = 0; b < c->cfg.batch; ++b) {
        if (ctx_lens[b] < 0 || ctx_lens[b] > c->cfg.max_seq_len) return GQA_ERR_RANGE;
        if (positions[b] < -1 || positions[b] >= c->cfg.max_seq_len) return GQA_ERR_RANGE;
        if (!rows_backed(c, b, 0, ctx_lens[b]) || (positions[b] >= 0 && !rows_backed(c, b, positions[b], 1)))
            return GQA_ERR_RANGE;
        if (ctx_lens[b] > max_len) max_len = ctx_lens[b];
    }
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipSetDevice(c->cfg.device));
    if (c->paged)
        for (int b = 0; b < c->cfg.batch; ++b)
            if (ctx_lens[b] > 0 || positions[b] >= 0) c->pages.touch(b);
    const size_t qwords = (size_t)c->cfg.batch * c->cfg.n_q_heads * c->cfg.head_dim;
    const size_t row_words = (size_t)c->cfg.batch * c->cfg.n_kv_heads * c->cfg.head_dim;
    const size_t i32 = (size_t)c->cfg.batch * sizeof(int32_t);
    HIP_TRY(hipEventRecord(c->ev_begin, c->stream));
    HIP_TRY(hipMemcpyAsync(c->q_dev, q, qwords * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->rows_dev, k_rows, row_words * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->rows_dev + row_words, v_rows, row_words * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->pos_dev, positions, i32, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->lens_dev, ctx_lens, i32, hipMemcpyHostToDevice, c->stream));
    rc = run_decode(c, c->q_dev, c->lens_dev, c->rows_dev, c->rows_dev + row_words, c->pos_dev, c->o_dev,
                    lse ? c->lse_dev : nullptr, c->stream, max_len);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipMemcpyAsync(o, c->o_dev, qwords * 2, hipMemcpyDeviceToHost, c->stream));
    if (lse)
        HIP_TRY(hipMemcpyAsync(lse, c->lse_dev, (size_t)c->cfg.batch * c->cfg.n_q_heads * sizeof(float),
                               hipMemcpyDeviceToHost, c->stream));
    return finish_sync(c);
}

int gqa_decode_append_device(gqa_ctx* c, const void* q, const void* k_rows, const void* v_rows,
                             const int32_t* positions, const int32_t* ctx_lens, void* o, float* lse, void* stream) {
    if (!c || !q || !k_rows || !v_rows || !positions || !ctx_lens || !o) return GQA_ERR_NULL;
    if (!aligned16(q) || !aligned16(k_rows) || !aligned16(v_rows)) return GQA_ERR_RANGE;
    return run_decode(c, q, ctx_lens, k_rows, v_rows, positions, o, lse, pick_stream(c, stream),
                      c->cfg.max_seq_len);
}

int gqa_decode_append_noalloc(const gqa_config* cfg, void* k_cache, void* v_cache, int32_t l_cap, const void* q,
                              const void* k_rows, const void* v_rows, const int32_t* positions,
                              const int32_t* ctx_lens, void* o, float* lse, void* stream) {
    if (!cfg || !k_cache || !v_cache || !q || !ctx_lens || !o) return GQA_ERR_NULL;
    if ((k_rows == nullptr) != (v_rows == nullptr) || (k_rows != nullptr && positions == nullptr)) return GQA_ERR_NULL;
    const gqa_config& k = *cfg;
    if (k.batch < 1 || k.n_q_heads < 1 || k.n_kv_heads < 1 || k.n_q_heads % k.n_kv_heads != 0 || k.max_seq_len < 1 ||
        k.max_seq_len > kMaxRows || !(k.scale >= 0.f) || !isfinite(k.scale))
        return GQA_ERR_BAD_CFG;
    const int group = k.n_q_heads / k.n_kv_heads;
    if (!decode_supported(k.head_dim, group)) return GQA_ERR_UNSUPPORTED;
    // Rounds of keys never straddle a (sequence, kv head) region: l_cap is a multiple of 64.
    if (l_cap < k.max_seq_len || l_cap % 64 != 0 || l_cap > kMaxRows + 64) return GQA_ERR_RANGE;
    if (!aligned16(q) || !aligned16(k_rows) || !aligned16(v_rows) || !aligned16(k_cache) || !aligned16(v_cache))
        return GQA_ERR_RANGE;
    int n_dev = 0;
    if (hipGetDeviceCount(&n_dev) != hipSuccess || k.device < 0 || k.device >= n_dev || k.device >= kNoAllocDevices)
        return GQA_ERR_NO_DEVICE;
    HIP_TRY(hipSetDevice(k.device));
    NoAllocDevice* dev = nullptr;
    int rc = noalloc_setup(k.device, (hipStream_t)stream, &dev);
    if (rc != GQA_OK) return rc;
    // The plan gqa_decode_append_device makes for the same configuration (keys per split from the
    // CU count and max_seq_len), so both entry points give the same words.
    const DecodeShape shape =
        plan_decode_shape(k.batch, k.n_kv_heads, group, k.head_dim, dev->n_cu, k.max_seq_len, 0, GQA_DECODE_MERGE_AUTO);
    const int chunk = shape.chunk;
    const int max_splits = shape.max_splits;
    const size_t rows = (size_t)k.batch * k.n_kv_heads * max_splits * group;  // partial rows of the plan
    const size_t o_bytes = max_splits > 1 ? (rows * k.head_dim * sizeof(float) + 255) / 256 * 256 : 0;
    const size_t ml_bytes = max_splits > 1 ? rows * 2 * sizeof(float) : 0;
    if (o_bytes + ml_bytes > kNoAllocPartialBytes) return GQA_ERR_SCRATCH;
    DecodeArgs a{};
    a.q = (const uint16_t*)q;
    a.kc = (uint16_t*)k_cache;
    a.vc = (uint16_t*)v_cache;
    a.lens = ctx_lens;
    a.k_new = (const uint16_t*)k_rows;
    a.v_new = (const uint16_t*)v_rows;
    a.positions = positions;
    a.batch = k.batch;
    a.n_kv_heads = k.n_kv_heads;
    a.l_cap = l_cap;
    a.l_max = k.max_seq_len;
    a.chunk = chunk;
    a.max_splits = max_splits;
    const float scale = k.scale > 0.f ? k.scale : (float)(1.0 / sqrt((double)k.head_dim));
    a.scale_log2 = scale * 1.4426950408889634f;
    a.part_o = reinterpret_cast<float*>(dev->scratch);
    a.part_ml = reinterpret_cast<float*>(dev->scratch + o_bytes);
    a.out = (uint16_t*)o;
    a.lse = lse;
    a.zero_row = dev->zero;
    a.longest_first = k.batch > 1;
    a.cached = decode_cached_loads((int64_t)k.batch * k.n_kv_heads, k.max_seq_len, k.head_dim) ? 1 : 0;
    a.waves = shape.waves;
    // The same merge as the context entry point's default (GQA_DECODE_MERGE_AUTO), when the counters
    // cover the units.
    const int units = k.batch * k.n_kv_heads;
    a.arrivals = units <= kNoAllocCounters && fuse_merge(GQA_DECODE_MERGE_AUTO, units, max_splits, dev->n_cu)
                     ? dev->arrivals
                     : nullptr;
    Launch l;
    l.stream = (hipStream_t)stream;
    HIP_TRY(launch_decode(k.head_dim, group, a, l));
    if (max_splits > 1 && a.arrivals == nullptr) HIP_TRY(launch_combine(k.head_dim, group, a, l));
    return GQA_OK;
}

int gqa_prefill(gqa_ctx* c, int32_t b, const uint16_t* q, int32_t q_len, int32_t q_pos_base, int32_t kv_len,
                int32_t kv_pos_base, int32_t causal, uint16_t* o, float* lse) {
    if (!c || !q || !o) return GQA_ERR_NULL;
    int rc = check_prefill_args(c, b, q_len, q_pos_base, kv_len, kv_pos_base);
    if (rc != GQA_OK) return rc;
    if (!rows_backed(c, b, 0, kv_len)) return GQA_ERR_RANGE;
    rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipSetDevice(c->cfg.device));
    const size_t qwords = (size_t)c->cfg.n_q_heads * q_len * c->cfg.head_dim;
    HIP_TRY(hipEventRecord(c->ev_begin, c->stream));
    HIP_TRY(hipMemcpyAsync(c->q_dev, q, qwords * 2, hipMemcpyHostToDevice, c->stream));
    rc = run_prefill(c, b, c->q_dev, q_len, q_pos_base, kv_len, kv_pos_base, causal, c->o_dev,
                     lse ? c->lse_dev : nullptr, c->stream);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipMemcpyAsync(o, c->o_dev, qwords * 2, hipMemcpyDeviceToHost, c->stream));
    if (lse)
        HIP_TRY(hipMemcpyAsync(lse, c->lse_dev, (size_t)c->cfg.n_q_heads * q_len * sizeof(float),
                               hipMemcpyDeviceToHost, c->stream));
    return finish_sync(c);
}

int gqa_prefill_append(gqa_ctx* c, int32_t b, const uint16_t* q, const uint16_t* k_rows, const uint16_t* v_rows,
                       int32_t n_new, int32_t q_len, int32_t q_pos_base, int32_t kv_len, int32_t kv_pos_base,
                       int32_t causal, uint16_t* o, float* lse) {
    if (!c || !q || !k_rows || !v_rows || !o) return GQA_ERR_NULL;
    int rc = check_prefill_args(c, b, q_len, q_pos_base, kv_len, kv_pos_base);
    if (rc != GQA_OK) return rc;
    if (!rows_backed(c, b, 0, kv_len)) return GQA_ERR_RANGE;
    if (n_new < 1 || n_new > kv_len || n_new > c->cfg.max_q_len) return GQA_ERR_RANGE;
    rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipSetDevice(c->cfg.device));
    const size_t qwords = (size_t)c->cfg.n_q_heads * q_len * c->cfg.head_dim;
    const size_t rwords = (size_t)c->cfg.n_kv_heads * n_new * c->cfg.head_dim;
    HIP_TRY(hipEventRecord(c->ev_begin, c->stream));
    HIP_TRY(hipMemcpyAsync(c->q_dev, q, qwords * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->new_dev, k_rows, rwords * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->new_dev + rwords, v_rows, rwords * 2, hipMemcpyHostToDevice, c->stream));
    rc = run_prefill(c, b, c->q_dev, q_len, q_pos_base, kv_len, kv_pos_base, causal, c->o_dev,
                     lse ? c->lse_dev : nullptr, c->stream, c->new_dev, c->new_dev + rwords, n_new);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipMemcpyAsync(o, c->o_dev, qwords * 2, hipMemcpyDeviceToHost, c->stream));
    if (lse)
        HIP_TRY(hipMemcpyAsync(lse, c->lse_dev, (size_t)c->cfg.n_q_heads * q_len * sizeof(float),
                               hipMemcpyDeviceToHost, c->stream));
    return finish_sync(c);
}

int gqa_prefill_append_device(gqa_ctx* c, int32_t b, const void* q, const void* k_rows, const void* v_rows,
                              int32_t n_new, int32_t q_len, int32_t q_pos_base, int32_t kv_len, int32_t kv_pos_base,
                              int32_t causal, void* o, float* lse, void* stream) {
    if (!c || !q || !k_rows || !v_rows || !o) return GQA_ERR_NULL;
    if (!aligned16(q) || !aligned16(k_rows) || !aligned16(v_rows) || !aligned16(o)) return GQA_ERR_RANGE;
    int rc = check_prefill_args(c, b, q_len, q_pos_base, kv_len, kv_pos_base);
    if (rc != GQA_OK) return rc;
    if (!rows_backed(c, b, 0, kv_len)) return GQA_ERR_RANGE;
    if (n_new < 1 || n_new > kv_len) return GQA_ERR_RANGE;
    return run_prefill(c, b, q, q_len, q_pos_base, kv_len, kv_pos_base, causal, o, lse, pick_stream(c, stream),
                       k_rows, v_rows, n_new);
}

int gqa_prefill_device(gqa_ctx* c, int32_t b, const void* q, int32_t q_len, int32_t q_pos_base, int32_t kv_len,
                       int32_t kv_pos_base, int32_t causal, void* o, float* lse, void* stream) {
    if (!c || !q || !o) return GQA_ERR_NULL;
    if (!aligned16(q) || !aligned16(o)) return GQA_ERR_RANGE;
    int rc = check_prefill_args(c, b, q_len, q_pos_base, kv_len, kv_pos_base);
    if (rc != GQA_OK) return rc;
    if (!rows_backed(c, b, 0, kv_len)) return GQA_ERR_RANGE;
    return run_prefill(c, b, q, q_len, q_pos_base, kv_len, kv_pos_base, causal, o, lse, pick_stream(c, stream));
}

// ---- transaction protocol ----------------------------------------------------------

int gqa_submit(gqa_ctx* c, int32_t b, const uint16_t* q, int32_t q_len, int32_t q_pos_base, int32_t kv_len,
               int32_t kv_pos_base, int32_t causal) {
    if (!c || !q) return GQA_ERR_NULL;
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    rc = check_prefill_args(c, b, q_len, q_pos_base, kv_len, kv_pos_base);
    if (rc != GQA_OK) return rc;
    if (!rows_backed(c, b, 0, kv_len)) return GQA_ERR_RANGE;
    if (!prefill_supported(c->cfg.head_dim, c->group)) return GQA_ERR_UNSUPPORTED;
    HIP_TRY(hipSetDevice(c->cfg.device));
    c->txn = Txn();
    c->txn.layer = c->layer;
    c->txn.b = b;
    c->txn.q_len = q_len;
    c->txn.q_pos_base = q_pos_base;
    c->txn.kv_len = kv_len;
    c->txn.kv_pos_base = kv_pos_base;
    c->txn.causal = causal ? 1 : 0;
    const size_t qwords = (size_t)c->cfg.n_q_heads * q_len * c->cfg.head_dim;
    HIP_TRY(hipEventRecord(c->ev_t[0], c->stream));
    HIP_TRY(hipMemcpyAsync(c->q_dev, q, qwords * 2, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->txn.valid = 1;
    return GQA_OK;
}

int gqa_layer_qkv_device(gqa_ctx* c, int32_t b, const void* x, int32_t n_tokens, int32_t hidden, const void* wq,
                         const void* wk, const void* wv, const void* rms_weight, float rms_eps, int32_t q_pos_base,
                         int32_t kv_pos_base, int32_t kv_row0, int32_t rope, void* q_out, void* stream) {
    if (!c || !x || !wq || !wk || !wv || !q_out) return GQA_ERR_NULL;
    if (reinterpret_cast<uintptr_t>(q_out) & 15) return GQA_ERR_RANGE;  // Q is written in 16-byte chunks
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    rc = check_layer_args(c, b, n_tokens, hidden, q_pos_base, kv_pos_base, kv_row0);
    if (rc != GQA_OK) return rc;
    if (!rows_backed(c, b, kv_row0, n_tokens)) return GQA_ERR_RANGE;
    if (!(rms_eps >= 0.f) || !isfinite(rms_eps)) return GQA_ERR_RANGE;
    HIP_TRY(hipSetDevice(c->cfg.device));
    return run_layer_qkv(c, b, x, n_tokens, hidden, wq, wk, wv, rms_weight, rms_eps, q_pos_base, kv_pos_base, kv_row0,
                         rope, q_out, pick_stream(c, stream), false);
}

int gqa_submit_layer(gqa_ctx* c, int32_t b, const uint16_t* x, int32_t n_tokens, int32_t hidden, const uint16_t* wq,
                     const uint16_t* wk, const uint16_t* wv, const uint16_t* rms_weight, float rms_eps,
                     int32_t q_pos_base, int32_t kv_pos_base, int32_t causal, int32_t rope) {
    if (!c || !x || !wq || !wk || !wv) return GQA_ERR_NULL;
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    rc = check_layer_args(c, b, n_tokens, hidden, q_pos_base, kv_pos_base, 0);
    if (rc != GQA_OK) return rc;
    rc = check_prefill_args(c, b, n_tokens, q_pos_base, n_tokens, kv_pos_base);
    if (rc != GQA_OK) return rc;
    if (!rows_backed(c, b, 0, n_tokens)) return GQA_ERR_RANGE;
    if (!(rms_eps >= 0.f) || !isfinite(rms_eps)) return GQA_ERR_RANGE;
    if (!prefill_supported(c->cfg.head_dim, c->group)) return GQA_ERR_UNSUPPORTED;
    HIP_TRY(hipSetDevice(c->cfg.device));
    const size_t D = c->cfg.head_dim, nq = (size_t)c->cfg.n_q_heads * D, nkv = (size_t)c->cfg.n_kv_heads * D;
    auto pad = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    const size_t xb = (size_t)n_tokens * hidden * 2, wqb = nq * hidden * 2, wkb = nkv * hidden * 2,
                 gb = rms_weight ? (size_t)hidden * 2 : 0;
    rc = ensure_buffer(&c->layer_in, &c->layer_in_bytes, pad(xb) + pad(wqb + 2 * wkb) + pad(gb));
    if (rc != GQA_OK) return rc;
    uint8_t* dx = c->layer_in;
    uint8_t* dwq = dx + pad(xb);  // Wq, Wk, Wv back to back: one fused projection GEMM
    uint8_t* dwk = dwq + wqb;
    uint8_t* dwv = dwk + wkb;
    uint8_t* dg = dwq + pad(wqb + 2 * wkb);
    c->txn = Txn();
    c->txn.layer = c->layer;
    c->txn.b = b;
    c->txn.q_len = n_tokens;
    c->txn.q_pos_base = q_pos_base;
    c->txn.kv_len = n_tokens;
    c->txn.kv_pos_base = kv_pos_base;
    c->txn.causal = causal ? 1 : 0;
    HIP_TRY(hipEventRecord(c->ev_t[0], c->stream));
    HIP_TRY(hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(dwq, wq, wqb, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(dwk, wk, wkb, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(dwv, wv, wkb, hipMemcpyHostToDevice, c->stream));
    if (rms_weight) HIP_TRY(hipMemcpyAsync(dg, rms_weight, gb, hipMemcpyHostToDevice, c->stream));
    rc = run_layer_qkv(c, b, dx, n_tokens, hidden, dwq, dwk, dwv, rms_weight ? dg : nullptr, rms_eps, q_pos_base,
                       kv_pos_base, 0, rope, c->q_dev, c->stream, true);
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    rc = layer_times(c);
    if (rc != GQA_OK) return rc;
    c->txn.valid = 1;
    return GQA_OK;
}

int gqa_layer_times(gqa_ctx* c, float* out_us, int32_t n) {
    if (!c || !out_us) return GQA_ERR_NULL;
    if (n < 0 || n > 3) return GQA_ERR_RANGE;
    if (!c->layer_timed) return GQA_ERR_NO_TRANSACTION;
    int rc = layer_times(c);
    if (rc != GQA_OK) return rc;
    for (int i = 0; i < n; ++i) out_us[i] = c->layer_us[i];
    return GQA_OK;
}

// ---- HIP graphs ------------------------------------------------------------------------

int gqa_graph_capture_decode_append(gqa_ctx* c, const void* q, const void* k_rows, const void* v_rows,
                                    const int32_t* positions, const int32_t* ctx_lens, void* o, float* lse,
                                    gqa_graph** out) {
    if (!c || !q || !ctx_lens || !o || !out) return GQA_ERR_NULL;
    if ((k_rows == nullptr) != (v_rows == nullptr) || (k_rows != nullptr && positions == nullptr))
        return GQA_ERR_NULL;
    *out = nullptr;
    if (!aligned16(q) || !aligned16(k_rows) || !aligned16(v_rows)) return GQA_ERR_RANGE;
    int rc = txn_idle(c);
    if (rc != GQA_OK) return rc;
    gqa_graph* g = new gqa_graph();
    g->ctx = c;
    // The plan of gqa_decode_append_device for device-resident lengths (sized for max_seq_len).
    rc = plan_decode(c, q, ctx_lens, k_rows, v_rows, positions, o, lse, c->cfg.max_seq_len, &g->args, &g->combine);
    if (rc != GQA_OK) {
        delete g;
        return rc;
    }
    *out = g;
    return GQA_OK;
}

int gqa_graph_launch(gqa_graph* g, void* stream) {
    if (!g || !g->ctx) return GQA_ERR_NULL;
    gqa_ctx* c = g->ctx;
    HIP_TRY(hipSetDevice(c->cfg.device));
    Launch l;
    l.stream = pick_stream(c, stream);
    HIP_TRY(launch_decode(c->cfg.head_dim, c->group, g->args, l));
    if (g->combine) HIP_TRY(launch_combine(c->cfg.head_dim, c->group, g->args, l));
    return GQA_OK;
}

int gqa_graph_destroy(gqa_graph* g) {
    if (!g) return GQA_ERR_NULL;
    delete g;
    return GQA_OK;
}

int gqa_start(gqa_ctx* c) {
    if (!c) return GQA_ERR_NULL;
    if (c->txn.running && txn_idle(c) != GQA_OK) return GQA_ERR_BUSY_START;
    if (!c->txn.valid) return GQA_ERR_NO_TRANSACTION;
    HIP_TRY(hipSetDevice(c->cfg.device));
    const Txn& t = c->txn;
    HIP_TRY(hipEventRecord(c->ev_t[1], c->stream));
    // The transaction reads the layer it was submitted on, whichever layer is active now.
    uint16_t* const k_active = c->k_cache;
    uint16_t* const v_active = c->v_cache;
    c->k_cache = c->k_pool + kv_words(c) * (size_t)t.layer;
    c->v_cache = c->v_pool + kv_words(c) * (size_t)t.layer;
    int rc = run_prefill(c, t.b, c->q_dev, t.q_len, t.q_pos_base, t.kv_len, t.kv_pos_base, t.causal, c->o_dev,
                         nullptr, c->stream);
    c->k_cache = k_active;
    c->v_cache = v_active;
    if (rc != GQA_OK) return rc;
    HIP_TRY(hipEventRecord(c->ev_t[2], c->stream));
    const size_t owords = (size_t)c->cfg.n_q_heads * t.q_len * c->cfg.head_dim;
    HIP_TRY(hipMemcpyAsync(c->o_pinned, c->o_dev, owords * 2, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipEventRecord(c->ev_t[3], c->stream));
    c->txn.running = 1;
    return GQA_OK;
}

int gqa_status(gqa_ctx* c, uint32_t* out_status) {
    if (!c || !out_status) return GQA_ERR_NULL;
    if (!c->txn.running) {
        *out_status = GQA_STATUS_START_READY;
        return GQA_OK;
    }
    hipError_t e = hipEventQuery(c->ev_t[3]);
    if (e == hipErrorNotReady) {
        *out_status = GQA_STATUS_BUSY;
        return GQA_OK;
    }
    if (e != hipSuccess) {
        last_hip_error(e, "hipEventQuery");
        *out_status = GQA_STATUS_ERROR;
        return GQA_ERR_HIP;
    }
    *out_status = GQA_STATUS_DONE | GQA_STATUS_START_READY;
    return GQA_OK;
}

int gqa_wait(gqa_ctx* c, int32_t timeout_ms) {
    if (!c) return GQA_ERR_NULL;
    if (!c->txn.running) return GQA_ERR_NO_TRANSACTION;  // nothing started (submitted or not)
    struct timespec t0;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (;;) {
        hipError_t e = hipEventQuery(c->ev_t[3]);
        if (e == hipSuccess) break;
        if (e != hipErrorNotReady) {
            last_hip_error(e, "hipEventQuery");
            return GQA_ERR_HIP;
        }
        if (timeout_ms >= 0) {
            struct timespec t1;
            clock_gettime(CLOCK_MONOTONIC, &t1);
            const double ms = (t1.tv_sec - t0.tv_sec) * 1e3 + (t1.tv_nsec - t0.tv_nsec) * 1e-6;
            if (ms > timeout_ms) return GQA_ERR_TIMEOUT;
        }
        struct timespec nap = {0, 20000};
        nanosleep(&nap, nullptr);
    }
    float k_ms = 0.f, tot_ms = 0.f, copy_ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&k_ms, c->ev_t[1], c->ev_t[2]));
    HIP_TRY(hipEventElapsedTime(&tot_ms, c->ev_t[0], c->ev_t[3]));
    HIP_TRY(hipEventElapsedTime(&copy_ms, c->ev_t[2], c->ev_t[3]));
    c->txn.kernel_us = k_ms * 1000.f;
    c->txn.total_us = tot_ms * 1000.f;
    c->txn.copy_us = copy_ms * 1000.f;
    c->last_us = c->txn.total_us;
    return GQA_OK;
}

int gqa_read_output(gqa_ctx* c, uint16_t* o, int64_t n_words) {
    if (!c || !o) return GQA_ERR_NULL;
    if (!c->txn.running) return GQA_ERR_NO_TRANSACTION;
    const int64_t expect = (int64_t)c->cfg.n_q_heads * c->txn.q_len * c->cfg.head_dim;
    if (n_words != expect) return GQA_ERR_RESULT_LEN;
    int rc = gqa_wait(c, -1);
    if (rc != GQA_OK) return rc;
    memcpy(o, c->o_pinned, (size_t)expect * 2);
    return GQA_OK;
}

int gqa_read_perf(gqa_ctx* c, uint64_t* total_ticks, uint64_t* kernel_ticks, uint64_t* copy_ticks,
                  double* clock_mhz) {
    if (!c) return GQA_ERR_NULL;
    const double mhz = c->clock_mhz;
    if (total_ticks) *total_ticks = (uint64_t)llround(c->txn.total_us * mhz);
    if (kernel_ticks) *kernel_ticks = (uint64_t)llround(c->txn.kernel_us * mhz);
    if (copy_ticks) *copy_ticks = (uint64_t)llround(c->txn.copy_us * mhz);
    if (clock_mhz) *clock_mhz = mhz;
    return GQA_OK;
}

// ---- measurement ----------------------------------------------------------------------

int gqa_stream_read_device(const void* src, int64_t n_bytes, int32_t n_wgs, int32_t unroll, uint32_t* sink,
                           void* stream) {
    if (!src || !sink) return GQA_ERR_NULL;
    if (n_bytes < 16 || n_bytes % 16 != 0 || n_wgs < 1 || !aligned16(src)) return GQA_ERR_RANGE;
    if (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8) return GQA_ERR_RANGE;
    Launch l;
    l.stream = (hipStream_t)stream;
    HIP_TRY(launch_stream_read(src, n_bytes, n_wgs, unroll, sink, l));
    return GQA_OK;
}

// ---- timing -------------------------------------------------------------------------

int gqa_last_elapsed_us(gqa_ctx* c, float* out_us) {
    if (!c || !out_us) return GQA_ERR_NULL;
    *out_us = c->last_us;
    return GQA_OK;
}

int gqa_kernel_times(gqa_ctx* c, float* out_us, int32_t n) {
    if (!c || !out_us) return GQA_ERR_NULL;
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (int i = 0; i < n; ++i) out_us[i] = 0.f;
    for (int i = 0; i < n && i < GQA_TIMER_COUNT; ++i) {
        if (!c->profile || c->ev_count[i] == 0) continue;
        double total = 0.0;
        for (int k = 0; k < c->ev_count[i]; ++k) {
            HIP_TRY(hipEventSynchronize(c->ev_pool[i][2 * k + 1]));
            float ms = 0.f;
            HIP_TRY(hipEventElapsedTime(&ms, c->ev_pool[i][2 * k], c->ev_pool[i][2 * k + 1]));
            total += ms;
        }
        out_us[i] = (float)(total * 1000.0 / c->ev_count[i]);
    }
    return GQA_OK;
}

int gqa_kernel_durations(gqa_ctx* c, int32_t slot, float* out_us, int32_t n, int32_t* n_out) {
    if (!c || (n > 0 && !out_us)) return GQA_ERR_NULL;
    if (slot < 0 || slot >= GQA_TIMER_COUNT || n < 0) return GQA_ERR_RANGE;
    const int recorded = c->profile ? c->ev_count[slot] : 0;
    if (n_out) *n_out = recorded;
    for (int k = 0; k < recorded && k < n; ++k) {
        HIP_TRY(hipEventSynchronize(c->ev_pool[slot][2 * k + 1]));
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, c->ev_pool[slot][2 * k], c->ev_pool[slot][2 * k + 1]));
        out_us[k] = ms * 1000.f;
    }
    return GQA_OK;
}

int gqa_kernel_launch_counts(gqa_ctx* c, int32_t* out_counts, int32_t n) {
    if (!c || !out_counts) return GQA_ERR_NULL;
    for (int i = 0; i < n; ++i) out_counts[i] = (i < GQA_TIMER_COUNT && c->profile) ? c->ev_count[i] : 0;
    return GQA_OK;
}

int gqa_last_prefill_plan(gqa_ctx* c, int32_t* kernel, int32_t* n_segs) {
    if (!c || !kernel || !n_segs) return GQA_ERR_NULL;
    *kernel = c->last_prefill_kernel;
    *n_segs = c->last_prefill_segs;
    return GQA_OK;
}

int gqa_synchronize(gqa_ctx* c) {
    if (!c) return GQA_ERR_NULL;
    HIP_TRY(hipStreamSynchronize(c->stream));
    return GQA_OK;
}

}  // extern "C"
