/*
 * gqa.h -- C ABI of libgqa.so, the MI355X (gfx950) GQA streaming-attention engine.
 *
 * The library replaces the PS->PL hardware boundary of the LARA KV260 accelerator
 * (CSR block + AXI-Stream K/V/Q sink + O source) with device-resident K/V caches in
 * HBM and hand-written HIP kernels.  Every entry point below names the reference
 * interface it stands in for (paths are relative to the reference repository).
 *
 * Conventions
 *   - bf16 tensors cross the boundary as raw IEEE bf16 words (uint16_t), exactly the
 *     words sw/attn_driver.py:88-98 (fp32_to_bf16_u16) produces.
 *   - Host buffers are caller-owned; the library never frees or retains them.
 *   - Every function returns a status code: 0 = OK, otherwise one of GQA_ERR_*.
 *     Codes 0x01..0x12 keep the values of error_code_t (hw/rtl/pkg/attn_pkg.sv:279-286).
 *   - Calls on one context are serialised by the caller (one transaction at a time,
 *     like the reference's start_ready handshake).  Separate contexts are independent.
 *   - K/V cache layout in HBM: [B][H_kv][L_cap][D] bf16, row stride D*2 bytes, where
 *     L_cap = max_seq_len rounded up to a multiple of 64.  Element (b, h, t, d) lives at
 *     ((b*H_kv + h)*L_cap + t)*D + d -- per (b, h) this is the token*HEAD_DIM + dim
 *     addressing of hw/rtl/mem/kv_cache_ram.sv:77-83.
 */
#ifndef LARA_GQA_H
#define LARA_GQA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------- */
#define GQA_OK                 0x00
#define GQA_ERR_BAD_CFG        0x01 /* ERR_BAD_CFG    attn_pkg.sv:281 */
#define GQA_ERR_BUSY_START     0x02 /* ERR_BUSY_START attn_pkg.sv:282 */
#define GQA_ERR_STREAM_LEN     0x10 /* ERR_STREAM_LEN attn_pkg.sv:283: payload size mismatch */
#define GQA_ERR_STREAM_DEST    0x11 /* ERR_STREAM_DEST attn_pkg.sv:284: bad destination/index */
#define GQA_ERR_RESULT_LEN     0x12 /* ERR_RESULT_LEN attn_pkg.sv:285: output size mismatch */
#define GQA_ERR_HIP            0x20 /* a HIP runtime call failed */
#define GQA_ERR_OOM            0x21 /* device or pinned allocation failed */
#define GQA_ERR_NO_DEVICE      0x22 /* no usable gfx950 device */
#define GQA_ERR_NULL           0x23 /* required pointer argument is NULL */
#define GQA_ERR_RANGE          0x24 /* length / position outside the configured capacity */
#define GQA_ERR_TIMEOUT        0x25 /* gqa_wait deadline expired */
#define GQA_ERR_NO_TRANSACTION 0x26 /* start/wait/read with nothing submitted */
#define GQA_ERR_UNSUPPORTED    0x27 /* shape with no compiled kernel (head_dim, group) */
#define GQA_ERR_SCRATCH        0x28 /* plan exceeds GQA_NOALLOC_SCRATCH_BYTES (gqa_decode_append_noalloc) */

/* STATUS word bits returned by gqa_status (CSR_STATUS, attn_driver.py:51-57). */
#define GQA_STATUS_START_READY (1u << 0)
#define GQA_STATUS_BUSY        (1u << 1)
#define GQA_STATUS_DONE        (1u << 2)
#define GQA_STATUS_ERROR       (1u << 3)

/* Per-kernel timer slots reported by gqa_kernel_times. */
#define GQA_TIMER_APPEND  0
#define GQA_TIMER_DECODE  1
#define GQA_TIMER_COMBINE 2 /* log-sum-exp merge launch of split-KV decode or segmented prefill */
#define GQA_TIMER_PREFILL 3
#define GQA_TIMER_NORM    4 /* layer stage: RMSNorm (gqa_layer_qkv_device) */
#define GQA_TIMER_PROJECTION 5 /* layer stage: the QKV projection's hipBLASLt kernels, between two recorded events */
#define GQA_TIMER_ROPE    6 /* layer stage: RoPE + scatter */
#define GQA_TIMER_COUNT   7

/* Tunables for gqa_set_option. */
#define GQA_OPT_DECODE_CHUNK 1 /* keys per split-KV work-group (a multiple of 64 giving at most max(l_cap / 256,
                                  the automatic plan's) splits; a last split of <= chunk/4 keys joins the one
                                  before it; 0 = auto: about 8 waves per CU, whole 16-key rounds per wave).
                                  The automatic plan does not split a (sequence, kv head) whose K/V take
                                  at most 128 KiB.  Work-groups have 8 waves, or 4 when the 8-wave plan
                                  has at most 8 work-groups (the automatic chunk is then planned for 4) */
#define GQA_OPT_PROFILE      2 /* 1 = time every kernel launch with a HIP event pair bound to the launch
                                  (hipExtLaunchKernel; restarts the record).  Binding adds no GPU work
                                  between launches, but each timed launch costs the host several us,
                                  so launches run back to back only if queued ahead of the GPU */
#define GQA_OPT_PREFILL_WGS  3 /* prefill work-groups the KV segmentation aims for (0 = auto: one per CU, 1 = none) */
#define GQA_OPT_NUMERICS     4 /* GQA_NUMERICS_*: arithmetic of prefill / transactions (decode: EXACT only) */
#define GQA_OPT_DECODE_MERGE 5 /* GQA_DECODE_MERGE_*: how split-KV decode merges a sequence's splits */
#define GQA_OPT_PREFILL_KERNEL 6 /* GQA_PREFILL_KERNEL_*: decomposition of prefill / transaction launches */
#define GQA_OPT_LAYER        7 /* layered paged context: the cache layer every entry point reads and writes
                                  (0 .. n_layers-1; gqa_create_paged_layers) */

/* Prefill decomposition (GQA_OPT_PREFILL_KERNEL).  SHARED: a work-group per kv head and 8 (32-row
 * block, query head) tasks shares each K/V tile over its GQA group; launches smaller than the GPU are
 * cut into KV segments merged by a second launch (GQA_OPT_PREFILL_WGS).  ROWS: a work-group per
 * (query head, 32-row block) whose waves split the keys and merge in LDS (one launch, no segments).
 * PAIRED: SHARED whose work-groups each own a long and a short causal row block (last and first),
 * the short one's waves moving to the long one's keys once theirs end, so the work-groups of a causal
 * launch carry equal work (causal launches of group 4 with more than one row block, always planned in
 * one KV segment; others as SHARED).
 * AUTO (default, no segment target set): PAIRED (one segment) for a causal prompt whose rows see no
 * keys before its own and whose SHARED grid holds half to one work-group per CU (a single dispatch
 * round, which longest-first dispatch cannot balance); else ROWS when the SHARED grid without
 * segments has fewer work-groups than the GPU has CUs; else SHARED -- paired when that grid is exactly
 * one work-group per CU (for instance a causal 2048-row chunk after earlier keys at 32q/8kv on 256
 * CUs), unpaired when larger.  gqa_last_prefill_plan reports the decomposition a launch took. */
#define GQA_PREFILL_KERNEL_AUTO   0
#define GQA_PREFILL_KERNEL_SHARED 1
#define GQA_PREFILL_KERNEL_ROWS   2
#define GQA_PREFILL_KERNEL_PAIRED 3

/* Split merge of the decode (GQA_OPT_DECODE_MERGE).  FUSED: the last split of a (sequence, kv head) to
 * finish merges the others' partials inside the decode launch (agent-scope atomics and a per-unit
 * arrival counter; one launch per step).  LAUNCH: a second, log-sum-exp merge launch.  AUTO (default):
 * FUSED while the split grid (sequences x kv heads x splits) is at most half the GPU's CU count and a
 * sequence has at most 16 splits -- every split ends with an L2 write-back of its XCD and an increment
 * of its sequence's counter, which saves the launch for short steps but slows the streaming of larger
 * grids more than a launch costs -- else LAUNCH.  An automatic plan of the shortest splits (one round
 * of every wave) that would need the merge launch takes splits twice as long where that lets AUTO fuse.
 * Both fold the splits in the same order (the same output words). */
#define GQA_DECODE_MERGE_AUTO   0
#define GQA_DECODE_MERGE_LAUNCH 1
#define GQA_DECODE_MERGE_FUSED  2

/* Numerics of the attention kernels (GQA_OPT_NUMERICS).
 * EXACT: fp32 scores, softmax, sums and accumulation, exact divide; the P.V product takes each
 *        softmax weight rounded to bf16 (RNE; the board truncates it, attn_top.sv:653-658) while
 *        l sums the fp32 weights.  Each output element is within 2 bf16 ulp of its row's largest
 *        |output| of exact attention plus 2^-8 of exact attention over |V| at that element
 *        (sum_k p_k |v_k[d]| / l); the second term matters only where V rows cancel -- otherwise
 *        it lies within the first.
 * KV260: the deployed KV260 datapath bit for bit -- sequential fp32 sums of exact bf16 products,
 *        the 1024-entry interpolated exp table (softmax_engine.sv:570-706), P truncated to bf16
 *        for PV (attn_top.sv:653-658), reciprocal-table normalisation (output_buffer.sv:192-286),
 *        16-key sub-blocks in the board's tile order (attn_core.sv:107-154); for comparing with
 *        board results word for word.  Transactions with q_len == kv_len follow the board's
 *        contract exactly; other shapes use the same walk over their own lengths. */
#define GQA_NUMERICS_EXACT 0
#define GQA_NUMERICS_KV260 1

typedef struct gqa_config {
    int32_t batch;       /* B: sequences resident in the cache                         */
    int32_t n_q_heads;   /* H_q  (N_Q_HEADS, attn_driver.py:65)                         */
    int32_t n_kv_heads;  /* H_kv (N_KV_HEADS, attn_driver.py:66); H_q % H_kv == 0        */
    int32_t head_dim;    /* D    (HEAD_DIM, attn_driver.py:63): 64 or 128               */
    int32_t max_seq_len; /* cache rows per (b, kv head), 1 .. 2^30 (MAX_SEQ_LEN generalised) */
    int32_t max_q_len;   /* largest prefill chunk / transaction length, 1 .. 2^30       */
    float   scale;       /* softmax scale; 0 selects fp32(1/sqrt(D)) (attn_pkg.sv:241)   */
    int32_t device;      /* HIP device ordinal                                          */
} gqa_config;

typedef struct gqa_ctx gqa_ctx;

/* ---- lifetime ---------------------------------------------------------------
 * gqa_create replaces AttentionAccelerator.__init__'s overlay/buffer set-up
 * (sw/attn_driver.py:251-288): it allocates the HBM K/V cache, staging and split-KV
 * workspace and a HIP stream.  gqa_destroy replaces close() (attn_driver.py:324-331). */
int gqa_create(const gqa_config* cfg, gqa_ctx** out_ctx);
int gqa_destroy(gqa_ctx* ctx);
int gqa_get_config(const gqa_ctx* ctx, gqa_config* out_cfg);
int gqa_set_option(gqa_ctx* ctx, int32_t option, int64_t value);
const char* gqa_status_string(int32_t code);
int gqa_device_count(int32_t* out_count);

/* ---- paged K/V cache --------------------------------------------------------
 * No reference counterpart: the KV260 reloads its cache on every transaction
 * (kv_cache_ram.sv:77-91, attn_driver.py:418-422), so it has no cache manager.  A paged
 * context keeps K and V in pools of n_pages pages of page_size rows (a power of two >= 64;
 * layout [n_pages][H_kv][page_size][D]) and one block table per sequence (page of each
 * page_size-row run of token rows, -1 = unmapped).  Every entry point works as on a
 * contiguous context, reading and writing through the tables; host-pointer forms return
 * GQA_ERR_RANGE when a row they touch is unmapped, device forms read unmapped rows as
 * zeros and skip writes to them.  KV260 numerics are not available on a paged context.
 * gqa_paged_reserve maps pages so rows [0, n_rows) of sequence b are backed (GQA_ERR_OOM,
 * changing nothing, when the pool is short); gqa_paged_release returns a sequence's pages;
 * gqa_paged_evict_lru releases whole sequences, least recently used first (reserve, load,
 * prefill and host-pointer decode calls count as uses) and skipping the n_pinned sequence
 * indices in pinned, until n_free_pages pages are free, writing up to max_evicted evicted
 * sequence indices (GQA_ERR_OOM, releasing nothing, if that cannot be reached).  Reserve,
 * release and evict synchronise the context stream; launches on other streams that read a
 * sequence must finish before its pages are released.  gqa_cache_pointers returns the
 * pools and page_size as l_cap. */
int gqa_create_paged(const gqa_config* cfg, int32_t page_size, int32_t n_pages, gqa_ctx** out_ctx);
int gqa_paged_reserve(gqa_ctx* ctx, int32_t b, int32_t n_rows);
int gqa_paged_release(gqa_ctx* ctx, int32_t b);
int gqa_paged_evict_lru(gqa_ctx* ctx, int32_t n_free_pages, const int32_t* pinned, int32_t n_pinned,
                        int32_t* evicted, int32_t max_evicted, int32_t* n_evicted);
int gqa_paged_info(gqa_ctx* ctx, int32_t* page_size, int32_t* n_pages, int32_t* n_free,
                   int32_t* max_pages);
int gqa_paged_table(gqa_ctx* ctx, int32_t b, int32_t* out, int32_t n);

/* ---- multi-layer paged K/V cache ---------------------------------------------
 * No reference counterpart: the board runs one layer per transaction and reloads its cache each
 * time (attn_driver.py:552-586).  gqa_create_paged_layers is gqa_create_paged for a model of
 * n_layers attention layers (1 .. GQA_MAX_LAYERS) sharing one block table per sequence and one
 * page allocator: a page index names the same token rows in every layer, so reserve, release and
 * evict map and unmap a run of tokens for all layers at once.  Each layer has its own pools
 * (layout [n_layers][n_pages][H_kv][page_size][D], K and V apart).  GQA_OPT_LAYER selects the
 * layer that decode, prefill, append, load, read, the layer stage and gqa_cache_pointers address
 * (default 0); switching is a host-side pointer change, ordered with the launches already queued
 * (each launch keeps the pools it was given).  A transaction reads the layer that was active when
 * it was submitted; a captured graph, the layer active at capture.  gqa_paged_layers returns
 * n_layers and the active layer (GQA_ERR_UNSUPPORTED on a contiguous context; gqa_create_paged
 * contexts have one layer). */
#define GQA_MAX_LAYERS 1024
int gqa_create_paged_layers(const gqa_config* cfg, int32_t page_size, int32_t n_pages, int32_t n_layers,
                            gqa_ctx** out_ctx);
int gqa_paged_layers(gqa_ctx* ctx, int32_t* n_layers, int32_t* layer);

/* ---- K/V cache --------------------------------------------------------------
 * gqa_load_kv replaces the KV branch of _service_request + _transfer(DEST_K_CACHE /
 * DEST_V_CACHE) (attn_driver.py:378-422) and the cache write of kv_cache_ram.sv:77-83:
 * k, v are host [H_kv][n][D] bf16 words written to rows start_pos..start_pos+n-1 of
 * sequence b.  Bit-exact. */
int gqa_load_kv(gqa_ctx* ctx, int32_t b, int32_t start_pos, int32_t n,
                const uint16_t* k, const uint16_t* v);
/* gqa_append_kv: one new row per sequence (no reference counterpart: the KV260 reloads
 * the whole cache per transaction, attn_driver.py:418-422).  k_rows, v_rows are host
 * [B][H_kv][D]; positions[b] is the row index, or -1 to leave sequence b untouched. */
int gqa_append_kv(gqa_ctx* ctx, const uint16_t* k_rows, const uint16_t* v_rows,
                  const int32_t* positions);
/* gqa_read_kv: copy rows back to the host ([H_kv][n][D] each) for bit-exact checks. */
int gqa_read_kv(gqa_ctx* ctx, int32_t b, int32_t start_pos, int32_t n,
                uint16_t* k, uint16_t* v);

/* ---- attention, synchronous host-pointer forms --------------------------------
 * gqa_decode replaces run_attention (attn_driver.py:469-550) for one new query row per
 * sequence: q is host [B][H_q][D]; ctx_lens[b] keys (rows 0..len-1) are attended,
 * q_head h reads kv head h / (H_q/H_kv) (board_performance.py:182-191).  o is host
 * [B][H_q][D] bf16 words (RNE), lse (optional) is host [B][H_q] natural-log
 * log-sum-exp of the scaled scores.  A sequence with ctx_lens[b] == 0 outputs zeros
 * (output_buffer.sv:276-277 semantics) and lse = -inf. */
int gqa_decode(gqa_ctx* ctx, const uint16_t* q, const int32_t* ctx_lens,
               uint16_t* o, float* lse);
/* gqa_decode_append: one decode step as a single kernel launch -- append one K/V row per
 * sequence (k_rows, v_rows host [B][H_kv][D] at positions[b], -1 = none; the same write
 * gqa_append_kv makes, bit-exact) and attend rows 0..ctx_lens[b]-1, which may include the
 * row just appended.  Replaces the KV-load + run_attention pair of attn_driver.py:418-550
 * for one new token per sequence; outputs as gqa_decode. */
int gqa_decode_append(gqa_ctx* ctx, const uint16_t* q, const uint16_t* k_rows, const uint16_t* v_rows,
                      const int32_t* positions, const int32_t* ctx_lens, uint16_t* o, float* lse);
/* gqa_prefill replaces run_attention for a block of q_len query rows of sequence b
 * against cache rows 0..kv_len-1: q and o are host head-major [H_q][q_len][D]
 * (attn_driver.py:487-488, 464).  Query i sits at absolute position q_pos_base + i,
 * key j at kv_pos_base + j; with causal != 0 key j is valid iff its position <= the
 * query's (softmax_engine.sv:865-871).  Rows with no valid key output zeros. */
int gqa_prefill(gqa_ctx* ctx, int32_t b, const uint16_t* q, int32_t q_len,
                int32_t q_pos_base, int32_t kv_len, int32_t kv_pos_base, int32_t causal,
                uint16_t* o, float* lse);

/* gqa_prefill_append: one chunk of a chunked prefill as a single launch -- place the chunk's
 * own K/V rows (k_rows, v_rows host [H_kv][n_new][D]) at cache rows kv_len-n_new .. kv_len-1 of
 * sequence b (bit-exact, as gqa_load_kv) and attend as gqa_prefill.  Replaces the per-transaction
 * K/V DMA + run_attention pair (attn_driver.py:418-550) when the cache grows chunk by chunk. */
int gqa_prefill_append(gqa_ctx* ctx, int32_t b, const uint16_t* q, const uint16_t* k_rows,
                       const uint16_t* v_rows, int32_t n_new, int32_t q_len, int32_t q_pos_base,
                       int32_t kv_len, int32_t kv_pos_base, int32_t causal, uint16_t* o, float* lse);

/* ---- transaction protocol (configure / start / status / wait_done / readback) -----
 * gqa_submit replaces configure() + the Q DMA (attn_driver.py:364-376, 423-432): it
 * validates the transaction and stages q (host head-major [H_q][q_len][D]) in HBM.
 * gqa_start replaces start() (attn_driver.py:434-437): it launches the kernels
 * asynchronously; GQA_ERR_BUSY_START if a transaction is still running.
 * gqa_status replaces status() (attn_driver.py:439-440) with the STATUS bits above.
 * gqa_wait replaces wait_done (attn_driver.py:442-456): timeout_ms < 0 waits forever.
 * gqa_read_output replaces readback_o (attn_driver.py:458-464); n_words must equal
 * H_q*q_len*D (else GQA_ERR_RESULT_LEN, like CSR_RESULT_LEN).
 * gqa_read_perf replaces read_perf (attn_driver.py:466-467): device-clock ticks of the
 * last transaction (total, kernel-only, copy-only) at clock_mhz. */
int gqa_submit(gqa_ctx* ctx, int32_t b, const uint16_t* q, int32_t q_len,
               int32_t q_pos_base, int32_t kv_len, int32_t kv_pos_base, int32_t causal);
int gqa_start(gqa_ctx* ctx);
int gqa_status(gqa_ctx* ctx, uint32_t* out_status);
int gqa_wait(gqa_ctx* ctx, int32_t timeout_ms);
int gqa_read_output(gqa_ctx* ctx, uint16_t* o, int64_t n_words);
int gqa_read_perf(gqa_ctx* ctx, uint64_t* total_ticks, uint64_t* kernel_ticks,
                  uint64_t* copy_ticks, double* clock_mhz);

/* ---- device-pointer forms (inputs already in HBM; stream may be NULL = ctx stream) --
 * Same semantics as the host forms; all pointers are device pointers.  They enqueue
 * and return without synchronising.  The context stream is a blocking HIP stream: work
 * on it is ordered both ways with the legacy default stream (handle 0, PyTorch's default
 * stream), so passing NULL from code that uses the default stream needs no extra sync.
 * A non-default caller stream gets no such ordering: pass that stream itself.
 * q, k_rows, v_rows and the prefill output o must be 16-byte aligned (the kernels move them
 * in 16-byte vectors; any hipMalloc or PyTorch allocation is), else GQA_ERR_RANGE. */
int gqa_append_kv_device(gqa_ctx* ctx, const void* k_rows, const void* v_rows,
                         const int32_t* positions, void* stream);
int gqa_decode_device(gqa_ctx* ctx, const void* q, const int32_t* ctx_lens,
                      void* o, float* lse, void* stream);
int gqa_decode_append_device(gqa_ctx* ctx, const void* q, const void* k_rows, const void* v_rows,
                             const int32_t* positions, const int32_t* ctx_lens, void* o, float* lse,
                             void* stream);
int gqa_prefill_device(gqa_ctx* ctx, int32_t b, const void* q, int32_t q_len,
                       int32_t q_pos_base, int32_t kv_len, int32_t kv_pos_base,
                       int32_t causal, void* o, float* lse, void* stream);
int gqa_prefill_append_device(gqa_ctx* ctx, int32_t b, const void* q, const void* k_rows,
                              const void* v_rows, int32_t n_new, int32_t q_len, int32_t q_pos_base,
                              int32_t kv_len, int32_t kv_pos_base, int32_t causal, void* o, float* lse,
                              void* stream);
/* gqa_load_kv_device: gqa_load_kv from device memory (k, v are [H_kv][n][D] in HBM). */
int gqa_load_kv_device(gqa_ctx* ctx, int32_t b, int32_t start_pos, int32_t n,
                       const void* k, const void* v, void* stream);
/* Device addresses of the K and V caches ([B][H_kv][L_cap][D] bf16) and L_cap. */
int gqa_cache_pointers(gqa_ctx* ctx, void** k_cache, void** v_cache, int32_t* l_cap);

/* ---- decode without allocation ------------------------------------------------------
 * No counterpart in the reference (the board has no allocator to avoid).  For callers that
 * cannot allocate device memory -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc: gqa_decode_append_device without a context.  The caller owns every
 * buffer: k_cache and v_cache are [B][H_kv][l_cap][D] bf16 in device memory (l_cap a multiple of
 * 64, >= cfg->max_seq_len; the layout of gqa_create's cache), q, k_rows, v_rows, positions,
 * ctx_lens, o and lse as for gqa_decode_append_device (k_rows = v_rows = positions = NULL:
 * attend only).  cfg supplies B, H_q, H_kv, D, max_seq_len, scale and device (max_q_len is
 * ignored).  The call allocates nothing: the split-KV partials of sequences longer than one split
 * live in a static device array of GQA_NOALLOC_SCRATCH_BYTES per device, held until the process
 * ends (its last 256 bytes are a zero K/V row); a plan that needs more returns GQA_ERR_SCRATCH
 * (the automatic plan needs at most about 9 MiB).  Every call on a device shares that array,
 * which keeps the last call's partials (each call writes every partial it reads): calls that
 * overlap on one device (other streams, other threads) race and must be serialised by the caller.
 * The first call on a device sets the array up (address lookup, zero row; it synchronises the
 * device) and returns GQA_ERR_UNSUPPORTED if `stream` is capturing: make one call before
 * capturing.  Same kernels and split plan as gqa_decode_append_device for the same cfg, so the
 * output words are the same. */
#define GQA_NOALLOC_SCRATCH_BYTES (16u << 20)
int gqa_decode_append_noalloc(const gqa_config* cfg, void* k_cache, void* v_cache, int32_t l_cap, const void* q,
                              const void* k_rows, const void* v_rows, const int32_t* positions,
                              const int32_t* ctx_lens, void* o, float* lse, void* stream);

/* ---- layer input stage (run_layer) -------------------------------------------------
 * Replace the host RMSNorm / QKV projection / RoPE / reshape_to_heads of
 * AttentionAccelerator.run_layer (attn_driver.py:552-576; the absent host_attention module;
 * hw/rtl/ext/rms_norm/rms_norm.sv:7-8, hw/rtl/ext/qkv_projection/qkv_projection.sv:7-8,
 * hw/rtl/core/rope_engine.sv:4-10).  x is [n_tokens][hidden] bf16; wq is
 * [H_q*D][hidden], wk and wv [H_kv*D][hidden] bf16 (out x in, Q = x Wq^T); rms_weight
 * (gamma, [hidden] bf16) may be NULL for no normalisation, else
 * y = x / sqrt(mean(x^2) + rms_eps) * gamma.  With rope != 0 the pair (2p, 2p+1) of each Q
 * head of token t is rotated by (q_pos_base + t) * theta_p and of each K head by
 * (kv_pos_base + t) * theta_p, theta_p = 10000^(-2p/D) in fp32 (hw/data/rope_theta.hex).
 * Positions must stay below 2^24.
 * gqa_submit_layer is gqa_submit for a layer: it uploads x and the weights, writes Q into
 * the transaction's staging and K/V into rows [0, n_tokens) of sequence b, and leaves a
 * transaction (q_len = kv_len = n_tokens) for gqa_start / gqa_wait / gqa_read_output.
 * gqa_layer_qkv_device does the same from device memory without a transaction: Q goes to
 * q_out ([H_q][n_tokens][D], 16-byte aligned, else GQA_ERR_RANGE), K/V to rows
 * [kv_row0, kv_row0 + n_tokens) of sequence b; it
 * allocates its workspace on first use.  The projection of a (token count, hidden) shape keeps
 * hipBLASLt's up to 8 best-ranked algorithms; the first call of the shape outside a stream capture
 * times them on the caller's operands (each run four times, the stream synchronised once per
 * algorithm: a few ms, once) and later calls use the fastest, while calls under a capture use the
 * best-ranked until such a call has run.  The context keeps the last 8 shapes.
 * gqa_layer_times returns the device time in us of
 * the RMSNorm, projection and RoPE stages (n <= 3; synchronises) of the last gqa_submit_layer
 * call (GQA_ERR_NO_TRANSACTION when there is none); gqa_layer_qkv_device calls made while
 * GQA_OPT_PROFILE is on record their stages in the GQA_TIMER_NORM / _PROJECTION / _ROPE slots of
 * gqa_kernel_times instead. */
int gqa_submit_layer(gqa_ctx* ctx, int32_t b, const uint16_t* x, int32_t n_tokens, int32_t hidden,
                     const uint16_t* wq, const uint16_t* wk, const uint16_t* wv,
                     const uint16_t* rms_weight, float rms_eps, int32_t q_pos_base,
                     int32_t kv_pos_base, int32_t causal, int32_t rope);
int gqa_layer_qkv_device(gqa_ctx* ctx, int32_t b, const void* x, int32_t n_tokens, int32_t hidden,
                         const void* wq, const void* wk, const void* wv, const void* rms_weight,
                         float rms_eps, int32_t q_pos_base, int32_t kv_pos_base, int32_t kv_row0,
                         int32_t rope, void* q_out, void* stream);
int gqa_layer_times(gqa_ctx* ctx, float* out_us, int32_t n);

/* ---- prepared decode steps ---------------------------------------------------------
 * No reference counterpart (the board's transaction is driven by CSR writes).  For serving loops
 * that replay one step shape over fixed device buffers.  gqa_graph_capture_decode_append plans one
 * gqa_decode_append_device step (k_rows = v_rows = positions = NULL: gqa_decode_device) over these
 * device pointers -- split plan sized for max_seq_len, kernel arguments bound -- and launches
 * nothing; gqa_graph_launch launches that step on `stream` (NULL = the context stream), reading q,
 * rows, positions and ctx_lens and writing o, lse and the cache at the bound addresses, so the
 * caller updates those buffers in place between launches.  A launch is the eager step's kernels
 * without the planning: no slower than gqa_decode_append_device.  (A HIP graph of the same step,
 * replayed back to back on this ROCm, cost 4.6 us more GPU time per replay and about 15 us of host
 * time per launch: B1 x 4097 keys 12.9 us against 8.3 eager.)  Callers that need a real HIP graph
 * capture gqa_decode_append_device or gqa_decode_append_noalloc in their own stream capture:
 * those calls enqueue only kernel launches (no allocation, synchronisation or memset).  A prepared
 * step must be destroyed before its context; profiling timers do not record its launches. */
typedef struct gqa_graph gqa_graph;
int gqa_graph_capture_decode_append(gqa_ctx* ctx, const void* q, const void* k_rows, const void* v_rows,
                                    const int32_t* positions, const int32_t* ctx_lens, void* o,
                                    float* lse, gqa_graph** out_graph);
int gqa_graph_launch(gqa_graph* graph, void* stream);
int gqa_graph_destroy(gqa_graph* graph);

/* ---- measurement -----------------------------------------------------------------
 * gqa_stream_read_device: no reference counterpart (the board harness reports against its own
 * measured PL clock, sw/board_performance.py:237-273).  Reads n_bytes (a multiple of 16) of device
 * memory at src the way the decode kernel streams its cache -- 16-byte nontemporal loads, 1 KiB
 * per wave instruction, `unroll` (1, 2, 4 or 8) loads in flight per thread, n_wgs work-groups of
 * 512 threads over contiguous shares -- and writes (almost) nothing (sink: n_wgs words): the
 * measured HBM read ceiling beside the 8 TB/s specification.  Enqueues on `stream` (NULL = the
 * legacy default stream) and returns. */
int gqa_stream_read_device(const void* src, int64_t n_bytes, int32_t n_wgs, int32_t unroll, uint32_t* sink,
                           void* stream);

/* ---- timing ---------------------------------------------------------------------
 * gqa_last_elapsed_us: elapsed time of the last synchronous call (HIP events on the ctx
 * stream).  With GQA_OPT_PROFILE on, every kernel launch is bracketed by HIP events on
 * the stream it runs on (up to 512 launches per kernel; setting the option again
 * restarts the record); gqa_kernel_times returns each kernel's AVERAGE duration in
 * microseconds, indexed by GQA_TIMER_* (0 when it did not run), and
 * gqa_kernel_launch_counts the number of launches averaged.  These replace the PL cycle
 * counters CSR_PERF_* (attn_pkg.sv:274-277) as the source of RunProfile timings. */
int gqa_last_elapsed_us(gqa_ctx* ctx, float* out_us);
int gqa_kernel_times(gqa_ctx* ctx, float* out_us, int32_t n);
int gqa_kernel_launch_counts(gqa_ctx* ctx, int32_t* out_counts, int32_t n);
/* gqa_kernel_durations: the duration (us) of each launch recorded in timer slot `slot` since
 * profiling was (re)started, in launch order, up to n of them (synchronises on them);
 * *n_out = the number recorded. */
int gqa_kernel_durations(gqa_ctx* ctx, int32_t slot, float* out_us, int32_t n, int32_t* n_out);
int gqa_synchronize(gqa_ctx* ctx);
/* gqa_last_prefill_plan: the decomposition (GQA_PREFILL_KERNEL_ROWS, _SHARED or _PAIRED) and the KV
 * segment count of the context's last prefill launch (gqa_prefill*, a transaction, run_layer's
 * attention); 0, 0 before any and after a KV260-numerics launch.  A diagnostic beside read_perf
 * (attn_driver.py:466-467): the board's tiling is fixed (attn_core.sv:107-154), the engine's is
 * chosen per launch, and tests use this to check which decomposition a launch took. */
int gqa_last_prefill_plan(gqa_ctx* ctx, int32_t* kernel, int32_t* n_segs);

#ifdef __cplusplus
}
#endif
#endif /* LARA_GQA_H */
