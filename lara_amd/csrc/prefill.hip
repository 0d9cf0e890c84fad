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
// Work decomposition.  A wave owns 32 query rows of one query head; the eight waves of a
// work-group own eight (row block, head) tasks of one KV head, heads fastest, so a GQA group
// of 4 shares every K/V tile across its heads and two row blocks.  Keys are processed in
// blocks of 64:
//   S^T [64 keys x 32 rows] = K [64 x D] . Q^T [D x 32]   two v_mfma_f32_32x32x16_bf16 chains;
//                                                          K from LDS (A), Q^T from VGPRs (B)
//   O^T [D x 32 rows]      += V^T [D x 64] . P^T [64 x 32] D/32 chains of four MFMAs;
//                                                          V^T from LDS through transposing
//                                                          reads (A), P^T from VGPRs (B)
// Computing the transposed products keeps every lane on one query row (column l % 32 of the
// MFMA result; lanes l and l + 32 hold two halves of the row's keys), so the softmax state of
// a row and its O accumulator live in the same lane pair: between the two products the only
// cross-lane step is the pair's row max (v_permlane32_swap).
//
// Staging.  K and V tiles stream from HBM straight into a three-stage LDS ring with
// direct-to-LDS loads (no register staging): while block j is computed, blocks j+1 and j+2
// are in flight.  Each lane loads the global 16-byte chunk that the swizzled LDS layout wants
// in its slot -- the cache row (from a wave-uniform base and a fixed per-lane offset), the row
// this launch appends, or a zero row past kv_len (P is 0 there, and V must be finite).
//
// MFMA 32x32x16 operand layout used below: lane l supplies row (A) / column (B) l % 32 and
// the eight k-values 8*(l/32)..8*(l/32)+7 of the step; result register i of lane l holds
// row 8*(i/4) + 4*(l/32) + (i%4), column l % 32.  The products only require A and B to
// agree on which k-values a lane holds, so the PV step feeds the P values in the order
// the S^T result leaves them, and V^T is stored in LDS with the matching key order.
#include "gqa_internal.h"

#include <type_traits>

#include <math.h>

namespace lara {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kBN = 64;     // keys per block
constexpr int kRows = kPrefillRows;  // query rows per wave
constexpr int kWaves = 8;   // waves per work-group: (row block, head) tasks, heads fastest
constexpr int kStages = 3;  // LDS ring depth: two blocks in flight behind the one computed
constexpr float kLn2 = 0.693147180559945309f;

__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// The value lane l ^ 32 holds (the other half-wave of the row), without an LDS round trip:
// v_permlane32_swap leaves lanes 0-31 of its second result and lanes 32-63 of its first
// holding the opposite half's values.  `half` is the lane's half-wave (lane / 32).
__device__ __forceinline__ float half_swap(float x, int half) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(half ? sw[0] : sw[1]);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};  // v_cvt_pk_bf16_f32, round to nearest even
    return __builtin_bit_cast(uint32_t, v);
}

// 16-byte chunk swizzles (bank-conflict-free MFMA operand reads).
template <int NCH>
__device__ __forceinline__ int k_swz(int row) {
    return NCH == 16 ? (row & 15) : ((row >> 1) & 7);
}

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// s_waitcnt vmcnt(N), leaving the LDS and export counters alone (gfx9 field layout).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Direct-to-LDS load of 16 bytes per lane (global_load_lds_dwordx4): lane L's bytes land at
// LDS byte address lds_addr + 16*L.  Issued from inline assembly so that the compiler's
// wait-count pass, which cannot tell which LDS bytes such a load writes, does not wait for
// every load in flight before each LDS read; the kernel waits for them itself (wait_vmcnt)
// before the barrier that publishes a stage.  lds_addr must be wave-uniform.
// (M0 is declared clobbered; the compiler does not keep values in it in this file's kernels,
// so its "reserved register" warning is silenced.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(lds_addr)
                 : "memory", "m0");
}
// The same load with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset.
__device__ __forceinline__ void dma16_sbase(uint64_t sbase, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 offset:0" : : "v"(voff), "s"(sbase),
                 "s"(lds_addr) : "memory", "m0");
}
#pragma clang diagnostic pop

// A wave-uniform pointer as an SGPR pair.
__device__ __forceinline__ uint64_t uniform_address(const void* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// 16-byte LDS read issued from inline assembly, so it stays where it is written: the
// compiler's scheduler, short of registers, would otherwise move every read next to its use
// and make each MFMA wait for its own read.  The result is valid only after lgkm_wait.  Reads
// addr + OFF (OFF in the instruction's 16-bit offset field).
template <int OFF = 0>
__device__ __forceinline__ u32x4 lds_read128(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
    return v;
}

// 16-byte global load into VGPRs from inline assembly: the compiler adds no s_waitcnt for it, so
// it can stay in flight behind later direct-to-LDS loads.  The result is valid only after vm_wait.
__device__ __forceinline__ u32x4 load16_untracked(const void* p) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}

// s_waitcnt vmcnt(N) (lgkm and export counters untouched) that the compiler sees as producing a
// and b (results of load16_untracked), so no use of them can move above it.
template <int N, typename T>
__device__ __forceinline__ void vm_wait(T& a, T& b) {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt %2" : "+v"(a), "+v"(b) : "i"((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8))
                 : "memory");
}

// s_waitcnt lgkmcnt(N) (vm and export counters untouched) that the compiler sees as
// producing a and b, so no use of them can move above it.  Only this kernel's own LDS reads
// are outstanding when it is used (the stage DMA counts on vmcnt).
template <int N, typename T>
__device__ __forceinline__ void lgkm_wait(T& a, T& b) {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt %2" : "+v"(a), "+v"(b) : "i"(0xF | (0x3 << 14) | (0x7 << 4) | (N << 8)));
}

// s_waitcnt lgkmcnt(N) that the compiler sees as producing a (one fragment; see lgkm_wait).
template <int N, typename T>
__device__ __forceinline__ void lgkm_wait1(T& a) {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt %1" : "+v"(a) : "i"(0xF | (0x3 << 14) | (0x7 << 4) | (N << 8)));
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1 (compile-time indices).
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// Transposing 8-byte LDS read (ds_read_b64_tr_b16) from inline assembly, at addr + OFF.
template <int OFF>
__device__ __forceinline__ u32x2 lds_read_tr64(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
    u32x2 v;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
    return v;
}

// Work-group barrier for the stage ring: LDS traffic is ordered by the explicit waits, so no
// memory fence (which would wait for every load in flight) is attached.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" : : : "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>((lds_void_ptr)p);
}

// V tile: rows of keys, 16-byte chunks XOR-swizzled so that the four keys a transposing read
// covers put their 64-byte runs (the 32 dims of one PV tile) in four different quarters of the
// 64 banks: rows are 2*D bytes apart, so D = 128 rows all start in bank 0 and the swizzle uses
// the key's two low bits; D = 64 rows alternate bank halves and the swizzle uses bit 1.
template <int D>
__device__ __forceinline__ int v_swz(int key) {
    return D == 128 ? 4 * (key & 3) : 4 * ((key >> 1) & 1);
}

// A wave's output block ([32 rows][D] bf16) goes to global memory through LDS: the lanes put their
// O^T fragments (row `col`, dims mt*32 + 8*r4 + 4*half .. +3) into a stash of 16-byte chunks, chunk
// c of row r at r*NCH + (c ^ (r % NCH)) (no bank conflicts either way), then store whole rows, 16
// bytes per lane: one store instruction covers four 256-byte rows instead of 16 bytes of 32 rows.
// Plain stores: nontemporal ones shortened these launches further but sent the rows past the
// memory-side cache, so whatever reads the output next paid about as much again.
template <int D>
__device__ __forceinline__ void stash_put(uint2* stash, int col, int half, int mt, int r4, uint2 w) {
    constexpr int NCH = D / 8;
    const int chunk = 4 * mt + r4;  // dims 8*chunk .. +7; this lane's four: + 4*half
    stash[2 * (col * NCH + (chunk ^ (col & (NCH - 1)))) + half] = w;
}

// Stores rows row0 .. row0 + 31 (those below q_len) of the stash to out (row r at out + r*D).  The
// stash was written by this wave; the wait orders its LDS writes before the reads.
template <int D>
__device__ __forceinline__ void stash_store_rows(const uint2* stash, uint16_t* out, int row0, int q_len, int lane) {
    constexpr int NCH = D / 8;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const uint4* s4 = reinterpret_cast<const uint4*>(stash);
#pragma unroll
    for (int it = 0; it < D / 16; ++it) {
        const int qc = it * 64 + lane;  // chunk qc of the block: row r, chunk c
        const int r = qc / NCH, c = qc % NCH;
        if (row0 + r < q_len)
            *reinterpret_cast<uint4*>(out + (size_t)(row0 + r) * D + 8 * c) = s4[r * NCH + (c ^ (r & (NCH - 1)))];
    }
}

// V^T operand of one PV step (eight bf16: dims mt*32 + lane%32, keys kb + 4*half + 0..3 and
// kb + 8 + 4*half + 0..3): ds_read_b64_tr_b16 hands lane i of each 16-lane group element (i % 4)
// of the 8-byte piece that lane 4j + i/4 of the group addresses, for j = 0..3, so every lane
// addresses key (lane%16)/4 of the four, dims d_g + 4*(lane%4) .. +3, and receives one dim of
// four keys.

template <int D, int G, bool PAGED, bool PAIR>
__global__ __launch_bounds__(kWaves * 64) void prefill_kernel(PrefillArgs a) {
    constexpr int NCH = D / 8;                   // 16-byte chunks per K/V row
    constexpr int KSTEPS = D / 16;               // QK k-steps
    constexpr int MT = D / 32;                   // PV result tiles (32 dims each)
    constexpr int TILE = kBN * NCH;              // 16-byte chunks per K (or V) tile
    // Waves 4-7 alone issue the ring's K/V loads.  The issue of a block's 32 KiB stalls its waves
    // for about 500 cycles (the load path's address rate), in which waves 0-3, on the same SIMDs,
    // compute their scores; waves 4-7 then start theirs after, so the two waves of a SIMD are out
    // of phase (MFMA beside softmax) instead of in lockstep.
    constexpr int kLoaders = 4;                  // waves 4 .. 4 + kLoaders - 1
    constexpr int DMA = TILE / (kLoaders * 64);  // direct-to-LDS loads per loading thread per tile
    constexpr int LPB = 2 * DMA;                 // per block (K and V)
    static_assert(DMA >= 1 && DMA * kLoaders * 64 == TILE, "tile shape");
    static_assert(kWaves == 8, "waves 4-7 load the ring");

    constexpr int NST = PAIR ? 4 : kStages;  // ring stages (PAIR: two blocks computed, two in flight)
    __shared__ __attribute__((aligned(16))) u32x4 lds_k[NST][TILE];
    __shared__ __attribute__((aligned(16))) u32x4 lds_v[NST][TILE];
    // PAIR: row block L's Q^T operand handed from wave g to wave g + 4, then that wave's bf16 output
    // rows of row block S ([32 rows][D], 16-byte chunks XOR-swizzled by the row).
    __shared__ __attribute__((aligned(16))) u32x4 lds_q[PAIR ? 4 : 1][PAIR ? KSTEPS : 1][64];
    static_assert(!PAIR || (G == 4 && kWaves == 8), "paired row blocks: two row blocks of four heads");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Work-group -> (kv head, task group): consecutive work-groups take consecutive kv heads, so
    // with the dispatcher's round robin over the 8 XCDs every XCD serves one kv head (or a fixed
    // subset of them) and its L2 holds only that head's K/V tiles.
    const int lin = blockIdx.y * gridDim.x + blockIdx.x;  // position within the segment's grid
    const int h = lin % a.n_kv_heads;                    // kv head
    const int wx = lin / a.n_kv_heads;                   // task group of the head
    const int n_rb = (a.q_len + kRows - 1) / kRows;
    const int n_tasks = n_rb * G;
    // Causal row blocks grow in work with their index: the largest go to the work-groups the
    // dispatcher starts first (longest first), so a grid larger than the GPU balances.
    // PAIR (a causal grid of one dispatch round): work-group p owns row blocks L = n_rb - 1 - p and
    // S = p, heads 0-3 each.  Waves 0-3 work on L from the first key; waves 4-7 work on S while a block
    // holds keys of S, then on L: from there on two blocks are in LDS at a time, the even one for
    // waves 0-3 and the odd one for waves 4-7, whose partials of L merge in LDS at the end.  A
    // work-group then carries about (keys(L) + keys(S)) / 2 keys per wave, instead of keys(L) for
    // the work-groups of the last row blocks.
    const int wg_x = (a.causal && !PAIR) ? (int)(gridDim.x - 1 - wx) : wx;
    const int task = PAIR ? (n_rb - 1 - wx) * G + (wave & 3) : wg_x * kWaves + wave;
    const bool active = task < n_tasks;
    const int g = task % G;
    const int rb = task / G;  // PAIR: row block L (every wave's last)
    const int hq = h * G + g;
    const bool has_s = PAIR && wx < rb;                 // PAIR: the work-group has a row block S
    const int rb_first = (has_s && wave >= 4) ? wx : rb;  // the row block the wave starts on

    // Keys a row block needs: [0, kv_limit) (causal rows stop at their diagonal).
    auto kv_limit = [&](int row_block) {
        int hi = a.kv_len;
        if (a.causal) {
            const int last_row = min(a.q_len, (row_block + 1) * kRows) - 1;
            hi = min(hi, a.q_pos_base + last_row - a.kv_pos_base + 1);
        }
        return max(hi, 0);
    };

    // Fused append: the new rows are copied into the cache by every work-group of this kv
    // head, an equal share each, so no work-group carries the whole copy.  Blocks that hold
    // these rows read them from k_new/v_new (issue below), so no work-group waits for the copy.
    const bool has_new = a.k_new != nullptr && a.n_new > 0;
    auto append_share = [&]() {
        const u32x4* ks = reinterpret_cast<const u32x4*>(a.k_new) + (size_t)h * a.n_new * NCH;
        const u32x4* vs = reinterpret_cast<const u32x4*>(a.v_new) + (size_t)h * a.n_new * NCH;
        const int words = a.n_new * NCH;
        const int n_threads = gridDim.x * gridDim.z * (kWaves * 64);
        const int first = (blockIdx.z * gridDim.x + wx) * (kWaves * 64) + tid;
        if constexpr (PAGED) {
            for (int i = first; i < words; i += n_threads) {
                const int64_t r = paged_row(a.block_table, a.page_shift, a.n_kv_heads, h, a.new_begin + i / NCH);
                if (r < 0) continue;  // unmapped page: nothing to write
                const size_t dst = (size_t)r * NCH + (i % NCH);
                reinterpret_cast<u32x4*>(a.kc)[dst] = ks[i];
                reinterpret_cast<u32x4*>(a.vc)[dst] = vs[i];
            }
        } else {
            u32x4* kd = reinterpret_cast<u32x4*>(a.kc + ((size_t)h * a.l_cap + a.new_begin) * D);
            u32x4* vd = reinterpret_cast<u32x4*>(a.vc + ((size_t)h * a.l_cap + a.new_begin) * D);
            for (int i = first; i < words; i += n_threads) {
                kd[i] = ks[i];
                vd[i] = vs[i];
            }
        }
    };
    const int last_task = min(n_tasks, (wg_x + 1) * kWaves) - 1;
    const int wg_hi = PAIR ? kv_limit(rb) : kv_limit(last_task / G);  // row blocks grow with the task index
    int wave_hi = active ? kv_limit(rb_first) : 0;
    const int seg_begin = blockIdx.z * a.seg_len;
    // With several segments, one that no row of this work-group reaches is not read by the
    // merge; a single segment always reaches the epilogue (rows without keys output 0).
    if (a.n_segs > 1 && seg_begin >= wg_hi) {
        if (has_new) append_share();
        return;
    }
    const int seg_end = min(wg_hi, seg_begin + a.seg_len);
    const int n_blocks = seg_end > seg_begin ? (seg_end - seg_begin + kBN - 1) / kBN : 0;

    const int col = lane & 31;   // query row within the wave's block (MFMA column)
    const int half = lane >> 5;  // which 8 k-values of a step this lane carries
    int cur_rb = rb_first;       // the row block the wave works on (PAIR: S, then L)
    const int row0 = cur_rb * kRows + col;
    const bool row0_ok = active && row0 < a.q_len;
    const int q_pos0 = a.q_pos_base + row0;

    f32x16 o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[mt][i] = 0.f;
    float m_run = -INFINITY;  // running max (log2 units) of this lane's row
    float l_lane = 0.f;       // this lane's half of the running sum

    const u32x4* kg = reinterpret_cast<const u32x4*>(a.kc + (PAGED ? 0 : (size_t)h * a.l_cap * D));
    const u32x4* vg = reinterpret_cast<const u32x4*>(a.vc + (PAGED ? 0 : (size_t)h * a.l_cap * D));
    const u32x4* kn = has_new ? reinterpret_cast<const u32x4*>(a.k_new) + (size_t)h * a.n_new * NCH : nullptr;
    const u32x4* vn = has_new ? reinterpret_cast<const u32x4*>(a.v_new) + (size_t)h * a.n_new * NCH : nullptr;
    const u32x4* zero = reinterpret_cast<const u32x4*>(a.zero_row);

    // Direct-to-LDS staging of block j0 into ring stage ST: wave-instruction i of loading wave w
    // (ld = w - 4) fills the 64 consecutive 16-byte slots (i*kLoaders + ld)*64 .., lane L slot +L;
    // each lane loads the chunk the swizzled layout wants in its slot.  Waves 0-3 issue nothing.
    // The slot -> (key, chunk) map is per lane and
    // fixed, so a block whose 64 rows are consecutive cache rows (every block but those past
    // kv_len, those holding rows this launch appends and unmapped pages) takes a wave-uniform
    // base in SGPRs and these fixed per-lane byte offsets (koff, voff): no per-block address
    // arithmetic.  The other blocks pick each lane's source (zero row, k_new/v_new, cache).
    const int ld = wave & 3;  // loading wave index (waves 4-7)
    int sl_key[DMA], sl_ck[DMA], sl_cv[DMA];
    uint32_t koff[DMA], voff[DMA];
#pragma unroll
    for (int i = 0; i < DMA; ++i) {
        const int slot = (i * kLoaders + ld) * 64 + lane;
        sl_key[i] = slot / NCH;
        sl_ck[i] = (slot % NCH) ^ k_swz<NCH>(sl_key[i]);
        sl_cv[i] = (slot % NCH) ^ v_swz<D>(sl_key[i]);
        koff[i] = 16u * (uint32_t)(sl_key[i] * NCH + sl_ck[i]);
        voff[i] = 16u * (uint32_t)(sl_key[i] * NCH + sl_cv[i]);
    }
    auto issue = [&](int j0, auto st_c) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_c)::value;
        if (wave < 4) return;
        const bool special = (j0 + kBN > a.kv_len) ||
                             (has_new && j0 + kBN > a.new_begin && j0 < a.new_begin + a.n_new);
        // Row j0's first word; a paged block (j0 and the page size are multiples of 64) lies in
        // one page, looked up once (-1: unmapped, read as zero rows).
        const u32x4* kb0 = kg + (PAGED ? 0 : (size_t)j0 * NCH);
        const u32x4* vb0 = vg + (PAGED ? 0 : (size_t)j0 * NCH);
        bool mapped = true;
        if constexpr (PAGED) {
            const int64_t pr = paged_row_uniform(a.block_table, a.page_shift, a.n_kv_heads, h, j0);
            mapped = pr >= 0;
            kb0 = kg + (size_t)(mapped ? pr : 0) * NCH;
            vb0 = vg + (size_t)(mapped ? pr : 0) * NCH;
        }
        if (!special && mapped) {
            const uint64_t kbase = uniform_address(kb0);
            const uint64_t vbase = uniform_address(vb0);
#pragma unroll
            for (int i = 0; i < DMA; ++i) {
                const int base = (i * kLoaders + ld) * 64;
                dma16_sbase(kbase, koff[i], lds_addr(&lds_k[ST][base]));
                dma16_sbase(vbase, voff[i], lds_addr(&lds_v[ST][base]));
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < DMA; ++i) {
            const int row_idx = j0 + sl_key[i];
            const unsigned r_new = (unsigned)(row_idx - a.new_begin);
            const u32x4* sk;
            const u32x4* sv;
            if (row_idx >= a.kv_len || !mapped) {
                sk = zero + sl_ck[i];
                sv = zero + sl_cv[i];
            } else if (has_new && r_new < (unsigned)a.n_new) {
                sk = kn + (size_t)r_new * NCH + sl_ck[i];
                sv = vn + (size_t)r_new * NCH + sl_cv[i];
            } else {
                sk = kb0 + (size_t)sl_key[i] * NCH + sl_ck[i];
                sv = vb0 + (size_t)sl_key[i] * NCH + sl_cv[i];
            }
            const int base = (i * kLoaders + ld) * 64;
            dma16(sk, lds_addr(&lds_k[ST][base]));
            dma16(sv, lds_addr(&lds_v[ST][base]));
        }
    };

    // Per-lane operand offsets.  K (A of S^T): key kt*32 + col, chunk 2*ks + half, swizzled by
    // the key's low bits, which kt does not change.  V^T (A of PV, transposing reads): the
    // lane addresses key (lane%16)/4 + 4*half of the step's key base and dims
    // mt*32 + 16*((lane/16)%2) + 4*(lane%4); the step's key base (a multiple of 4) only adds a
    // constant, and the swizzle depends on the key's low two bits alone.
    // LDS byte addresses in stage 0; the stage (the loop below runs one copy of its body per
    // stage) and the per-step parts are compile-time constants: instruction offsets.
    uint32_t kaddr[KSTEPS];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
        kaddr[ks] = lds_addr(&lds_k[0][0]) + 16u * (uint32_t)(col * NCH + ((2 * ks + half) ^ k_swz<NCH>(col)));
    uint32_t vaddr[MT];
    {
        const int key_off = (lane & 15) >> 2;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int dim = mt * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
            vaddr[mt] = lds_addr(&lds_v[0][0]) + (uint32_t)((key_off + 4 * half) * (D * 2) +
                                                            (((dim >> 3) ^ v_swz<D>(key_off)) << 4) + (((dim >> 2) & 1) << 3));
        }
    }

    // The running reference max only moves when a block's max exceeds it by more than
    // kLazyLog2 (p <= 2^kLazyLog2 meanwhile), so most blocks skip the O rescale.
    constexpr float kLazyLog2 = 8.0f;
    // Weights up to this sum per lane are taken against a stale reference max (see the block's
    // weights below): 2^16, so O = sum p v stays finite for |v| up to about 10^31 over 1024 keys.
    constexpr float kFreeSum = 65536.0f;
    const float c = a.scale_log2;

    // Q^T operand: row `row`, dims 16*ks + 8*half .. +7.  The Q loads, the first two blocks'
    // K/V loads and the append share's loads are all in flight before the first wait.
    u32x4 qb[KSTEPS];
    {
        const u32x4* qp = reinterpret_cast<const u32x4*>(a.q + ((size_t)hq * a.q_len + row0) * D);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) qb[ks] = row0_ok ? qp[2 * ks + half] : u32x4{0u, 0u, 0u, 0u};
    }
    if (n_blocks > 0) issue(seg_begin, std::integral_constant<int, 0>{});
    if (n_blocks > 1) issue(seg_begin + kBN, std::integral_constant<int, 1>{});
    if (has_new) append_share();
    // Retire everything now (Q, the append and the first blocks, issued together): with none of
    // its own loads pending, the compiler inserts no wait-for-everything inside the loop, where
    // the stage ring's loads are in flight.
    wait_vmcnt<0>();
    if constexpr (PAIR) {
        // Waves 0-3 hand row block L's Q^T operand to waves 4-7 (read once they move to L, after
        // at least one barrier).
        if (wave < 4) {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) lds_q[wave][ks][lane] = qb[ks];
        }
    }
    constexpr uint32_t kKt = 32 * NCH * 16;  // bytes between the two 32-key tiles of a block

    // The math of the 64-key block at key jb in ring stage ST (PAIR waves 4-7 past S: the stage
    // after ST, through their read addresses).
    auto compute = [&](int jb, auto st_c) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_c)::value;
        constexpr int NT = 2;  // 32-key tiles per block
        constexpr int kStageOff = ST * TILE * 16;  // bytes from stage 0 to stage ST

        // ---- S^T = K . Q^T (raw scores) ----
        f32x16 sacc[NT];
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) sacc[kt][i] = 0.f;
        // K fragments are double-buffered: step ks+1's LDS reads are in flight while step ks's
        // MFMAs run, so no MFMA waits for the read it consumes.
        // Fully unrolled, every fragment is its own value: none is copied while its read is in
        // flight.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // nothing else outstanding on lgkm
        u32x4 kf[KSTEPS][NT];
        auto read_k = [&](int ks) __attribute__((always_inline)) {
            kf[ks][0] = lds_read128<kStageOff>(kaddr[ks]);
            kf[ks][1] = lds_read128<kStageOff + kKt>(kaddr[ks]);
        };
        read_k(0);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            if (ks + 1 < KSTEPS) {
                read_k(ks + 1);
                lgkm_wait<2>(kf[ks][0], kf[ks][1]);
            } else {
                lgkm_wait<0>(kf[ks][0], kf[ks][1]);
            }
#pragma unroll
            for (int kt = 0; kt < NT; ++kt) sacc[kt] = mfma32(kf[ks][kt], qb[ks], sacc[kt]);
        }

        // ---- online softmax (log2 domain, scale folded into the exponent) ----
        const int row = PAIR ? cur_rb * kRows + col : row0;
        const bool row_ok = PAIR ? active && row < a.q_len : row0_ok;
        const int q_pos = PAIR ? a.q_pos_base + row : q_pos0;
        const int rb_now = PAIR ? cur_rb : rb;
        const bool need_mask = (jb + 32 * NT > a.kv_len) ||
                               (a.causal && a.kv_pos_base + jb + 32 * NT - 1 > a.q_pos_base + rb_now * kRows);
        if (need_mask) {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int j = jb + kt * 32 + 8 * (i >> 2) + 4 * half + (i & 3);
                    const bool ok = row_ok && j < a.kv_len && (!a.causal || a.kv_pos_base + j <= q_pos);
                    sacc[kt][i] = ok ? sacc[kt][i] : -INFINITY;
                }
        }
        // p = 2^(s*c - m_run); with no valid key yet (m_run = -inf) every s of the block is -inf
        // as well, and a finite offset keeps 2^(-inf) = 0 without a per-score select.
        float psum = 0.f;
        u32x4 pb[2 * NT];  // P^T operand of the PV k-steps (kt, a2)
        auto weights = [&]() __attribute__((always_inline)) {
            const float nm = (m_run == -INFINITY) ? 0.f : -m_run;
            psum = 0.f;
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int a2 = 0; a2 < 2; ++a2) {
                    float p[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float sv = sacc[kt][8 * a2 + j];
                        p[j] = __builtin_amdgcn_exp2f(fmaf(sv, c, nm));
                        psum += p[j];
                    }
                    pb[2 * kt + a2] = u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                            pack_bf16x2(p[6], p[7])};
                }
        };
        // Once every row of the wave has a reference max, the weights are taken against it directly
        // and the block's own max is needed only where a lane's weights sum past kFreeSum (or
        // overflow): weights up to that size keep their relative precision in the bf16 P operand and
        // in the fp32 sums, so the reference max stays until a block passes it by about 11 (log2).
        bool need_max = __ballot(m_run == -INFINITY) != 0;
        if (!need_max) {
            weights();
            need_max = __ballot(!(psum <= kFreeSum)) != 0;  // also true for inf and NaN
        }
        if (need_max) {
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[kt][i]);
            mx = pair_max32(mx);
            const float bm = mx * c;  // block max in log2 units (-inf if every key is masked)
            const bool grow = bm > m_run + kLazyLog2;
            if (__ballot(grow) != 0) {
                const float m_new = grow ? bm : m_run;
                const float corr = (m_run == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
                m_run = m_new;
                l_lane *= corr;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[mt][i] *= corr;
            }
            weights();
        }
        l_lane += psum;

        // ---- O^T += V^T . P^T ----
        // Step i = (mt, st_i): the two transposing reads of step i+1 are issued before step i's
        // MFMA, as in the S^T phase.
        constexpr int SPT = 2 * NT;  // k-steps per PV tile
        constexpr int PV = MT * SPT;
        u32x2 vf[PV][2];
        auto read_v = [&](auto step_c) {
            constexpr int i = decltype(step_c)::value;
            constexpr int st_i = i % SPT;
            constexpr int kb = 32 * (st_i >> 1) + 16 * (st_i & 1);  // step's key base (half adds 4)
            vf[i][0] = lds_read_tr64<kStageOff + kb * (D * 2)>(vaddr[i / SPT]);
            vf[i][1] = lds_read_tr64<kStageOff + (kb + 8) * (D * 2)>(vaddr[i / SPT]);
        };
        read_v(std::integral_constant<int, 0>{});
        static_for<PV>([&](auto step_c) {
            constexpr int i = decltype(step_c)::value;
            if constexpr (i + 1 < PV) {
                read_v(std::integral_constant<int, i + 1>{});
                lgkm_wait<2>(vf[i][0], vf[i][1]);
            } else {
                lgkm_wait<0>(vf[i][0], vf[i][1]);
            }
            const u32x4 vw = {vf[i][0].x, vf[i][0].y, vf[i][1].x, vf[i][1].y};
            o[i / SPT] = mfma32(vw, pb[i % SPT], o[i / SPT]);
        });
    };

    // PAIR: the move of waves 4-7 from S to L.  S's rows are final: normalised, rounded and kept
    // in LDS (written to the output after the loop, so no global store is in flight beside the ring's
    // loads); the wave takes L's Q^T from wave g and starts L with an empty partial.
    float lse_s = -INFINITY;  // PAIR: S's log-sum-exp (lanes of the first half-wave)
    auto leave_s = [&]() __attribute__((always_inline)) {
        const float l_row = l_lane + half_swap(l_lane, half);
        const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
        lse_s = l_row > 0.f ? (m_run + log2f(l_row)) * kLn2 : -INFINITY;
        const int q4 = wave & 3;
        // L's Q^T first: the stash below takes its place.
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) qb[ks] = lds_q[q4][ks][lane];
        uint2* stash = reinterpret_cast<uint2*>(&lds_q[q4][0][0]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                uint2 w;
                w.x = (uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 0] * inv) | ((uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 1] * inv) << 16);
                w.y = (uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 2] * inv) | ((uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 3] * inv) << 16);
                stash_put<D>(stash, col, half, mt, r4, w);
            }
        cur_rb = rb;
        wave_hi = kv_limit(rb);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[mt][i] = 0.f;
        m_run = -INFINITY;
        l_lane = 0.f;
    };
    // PAIR: from the first even block at or past S's keys on, blocks go in pairs: waves 4-7 read the
    // ring stage after the one waves 0-3 read.  (Waves 0-3's LDS Q hand-off precedes a barrier
    // before any wave reads it.)
    const int split_blk = has_s ? (kv_limit(wx) + kBN - 1) / kBN : 0;
    auto enter_pairs = [&]() __attribute__((always_inline)) {
        if (wave >= 4) {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) kaddr[ks] += TILE * 16;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) vaddr[mt] += TILE * 16;
            if (cur_rb != rb) leave_s();
        }
    };
    // PAIR, past S's keys: blocks j (waves 0-3) and j + 1 (waves 4-7, whose read addresses point one
    // stage on), j even and in ring stages ST and ST + 1; blocks j + 2 and j + 3 go into the two stages
    // the previous pair (or the last two single blocks) freed.
    auto block_pair = [&](int j, auto st_c) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_c)::value;
        const int j0 = seg_begin + j * kBN;
        wait_vmcnt<0>();  // blocks j and j + 1 are all that is in flight
        stage_barrier();
        if (j + 2 < n_blocks) issue(j0 + 2 * kBN, std::integral_constant<int, (ST + 2) % NST>{});
        if (j + 3 < n_blocks) issue(j0 + 3 * kBN, std::integral_constant<int, (ST + 3) % NST>{});
        const int jb = j0 + kBN * (wave >> 2);
        if (jb < wave_hi) compute(jb, st_c);
    };

    // Block blk of the segment, in ring stage ST = blk % NST.
    auto block = [&](int blk, auto st_c) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_c)::value;
        const int j0 = seg_begin + blk * kBN;
        // A loading wave's loads of block blk are done once at most the next block's remain (blocks 0
        // and 1 were retired before the loop; waves 0-3 have none in flight).
        if (blk >= 1) {
            if (blk + 1 < n_blocks) wait_vmcnt<LPB>(); else wait_vmcnt<0>();
        }
        stage_barrier();  // block blk landed in every slot; block blk-1's stage is free
        if (blk + 2 < n_blocks) issue(j0 + 2 * kBN, std::integral_constant<int, (ST + 2) % NST>{});
        if (j0 >= wave_hi) return;  // this wave's rows see no key of the block
        compute(j0, st_c);
    };
    static_assert(kStages == 3, "one copy of the block body per ring stage");
    if constexpr (PAIR) {
        // Single blocks up to the first even block past S's keys, then pairs of blocks.
        const int p0 = min(n_blocks, split_blk + (split_blk & 1));
        stage_barrier();  // the Q hand-off is visible even when no block precedes the move
        int blk = 0;
        for (; blk + NST <= p0; blk += NST) {
            block(blk, std::integral_constant<int, 0>{});
            block(blk + 1, std::integral_constant<int, 1>{});
            block(blk + 2, std::integral_constant<int, 2>{});
            block(blk + 3, std::integral_constant<int, 3>{});
        }
        if (blk < p0) block(blk++, std::integral_constant<int, 0>{});
        if (blk < p0) block(blk++, std::integral_constant<int, 1>{});
        if (blk < p0) block(blk++, std::integral_constant<int, 2>{});
        if (p0 < n_blocks) {
            enter_pairs();
            int j = p0;
            if (j % NST == 2) {
                block_pair(j, std::integral_constant<int, 2>{});
                j += 2;
            }
            for (; j < n_blocks; j += NST) {
                block_pair(j, std::integral_constant<int, 0>{});
                if (j + 2 < n_blocks) block_pair(j + 2, std::integral_constant<int, 2>{});
            }
        }
    } else {
        for (int blk = 0; blk < n_blocks; blk += kStages) {
            block(blk, std::integral_constant<int, 0>{});
            if (blk + 1 < n_blocks) block(blk + 1, std::integral_constant<int, 1>{});
            if (blk + 2 < n_blocks) block(blk + 2, std::integral_constant<int, 2>{});
        }
    }

    const int row = rb * kRows + col;  // the wave's last row block (PAIR: L)
    const bool row_ok = active && row < a.q_len;
    if constexpr (PAIR) {
        const int q4 = wave & 3;
        __syncthreads();  // every wave is done with the ring (and waves 0-3 with their Q hand-off)
        // S's keys all lay before L's last block: waves 4-7 finish S here, with an empty partial of L.
        if (wave >= 4 && cur_rb != rb) leave_s();
        // Waves 4-7 publish their partial of L (O^T fragments, running max, l) in the ring's space;
        // wave g merges it with its own: same lane, same row and dims.
        float4* part = reinterpret_cast<float4*>(q4 < 2 ? &lds_k[0][0] : &lds_v[0][0]);
        float2* part_ml = reinterpret_cast<float2*>(part + 2 * MT * 4 * 64) + (q4 & 1) * 64;
        part += (q4 & 1) * (MT * 4 * 64);
        const float l_row = l_lane + half_swap(l_lane, half);
        if (wave >= 4) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    part[(mt * 4 + r4) * 64 + lane] =
                        make_float4(o[mt][4 * r4], o[mt][4 * r4 + 1], o[mt][4 * r4 + 2], o[mt][4 * r4 + 3]);
            part_ml[lane] = make_float2(m_run, l_row);
        }
        __syncthreads();
        if (wave < 4) {
            const float2 mlb = part_ml[lane];
            const float M = fmaxf(m_run, mlb.x);
            const float wa = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - M);
            const float wb = mlb.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mlb.x - M);
            const float l_sum = fmaf(l_row, wa, mlb.y * wb);
            // Every lane stages its row (rows past q_len too: the stores skip them), since the row
            // stores below take each lane to other rows.
            const float inv = l_sum > 0.f ? 1.f / l_sum : 0.f;
            // L's rows are staged in ring stage 3 (the partials and their (m, l) fill stages 0-2).
            uint2* stash = reinterpret_cast<uint2*>(q4 < 2 ? &lds_k[NST - 1][0] : &lds_v[NST - 1][0]) +
                           (q4 & 1) * (kRows * NCH * 2);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const float4 pb4 = part[(mt * 4 + r4) * 64 + lane];
                    const float v0 = fmaf(o[mt][4 * r4 + 0], wa, pb4.x * wb) * inv;
                    const float v1 = fmaf(o[mt][4 * r4 + 1], wa, pb4.y * wb) * inv;
                    const float v2 = fmaf(o[mt][4 * r4 + 2], wa, pb4.z * wb) * inv;
                    const float v3 = fmaf(o[mt][4 * r4 + 3], wa, pb4.w * wb) * inv;
                    uint2 w;
                    w.x = (uint32_t)f32_to_bf16_rne(v0) | ((uint32_t)f32_to_bf16_rne(v1) << 16);
                    w.y = (uint32_t)f32_to_bf16_rne(v2) | ((uint32_t)f32_to_bf16_rne(v3) << 16);
                    stash_put<D>(stash, col, half, mt, r4, w);
                }
            stash_store_rows<D>(stash, a.out + (size_t)hq * a.q_len * D, rb * kRows, a.q_len, lane);
            if (row_ok && half == 0 && a.lse != nullptr)
                a.lse[(size_t)hq * a.q_len + row] = l_sum > 0.f ? (M + log2f(l_sum)) * kLn2 : -INFINITY;
        } else if (has_s) {
            // S's output rows from the stash leave_s filled.
            stash_store_rows<D>(reinterpret_cast<const uint2*>(&lds_q[q4][0][0]), a.out + (size_t)hq * a.q_len * D,
                                wx * kRows, a.q_len, lane);
            const int srow = wx * kRows + col;
            if (half == 0 && a.lse != nullptr && srow < a.q_len) a.lse[(size_t)hq * a.q_len + srow] = lse_s;
        }
        return;
    }
    if (!active) return;  // wave-uniform
    const float l_row = l_lane + half_swap(l_lane, half);
    if (a.n_segs > 1) {
        if (!row_ok) return;
        // Rows this wave never reached in the segment are not read by the merge.
        if (seg_begin >= wave_hi) return;
        // The segment's unnormalised O in fp16, divided by the power of two 2^e just above the row's
        // largest |O| (exact, any magnitude) so every dim keeps 11 significant bits relative to the
        // row (a bf16 ulp is 8), and (m, l, e) in fp32: half the bytes of an fp32 partial, written
        // here and read once by the merge.
        const size_t prow = ((size_t)blockIdx.z * a.n_q_heads + hq) * a.q_len + row;
        float amax = 0.f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(o[mt][i]));
        amax = fmaxf(amax, half_swap(amax, half));  // the row's other half-wave
        int e = 0;
        if (amax > 0.f) (void)frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
        uint16_t* po = a.part_o + prow * D;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const f16x4 w = {(_Float16)ldexpf(o[mt][4 * r4 + 0], -e), (_Float16)ldexpf(o[mt][4 * r4 + 1], -e),
                                 (_Float16)ldexpf(o[mt][4 * r4 + 2], -e), (_Float16)ldexpf(o[mt][4 * r4 + 3], -e)};
                *reinterpret_cast<uint2*>(po + mt * 32 + 8 * r4 + 4 * half) = __builtin_bit_cast(uint2, w);
            }
        if (half == 0)
            *reinterpret_cast<float4*>(a.part_ml + prow * 4) = make_float4(m_run, l_row, (float)e, 0.f);
        return;
    }
    // The rows are staged in the two ring stages no wave reads any more: block b sits in stage b % NST
    // and only the last block's stage may still be read (every wave passed the last block's barrier
    // after finishing the block before it, and no load is in flight after the last block's wait), so
    // waves 0-3 take stage n_blocks % NST and waves 4-7 the next, two waves per K or V tile.  Every
    // lane of the wave stages its row (rows past q_len too: the stores skip them).
    const int f = (n_blocks + (wave >> 2)) % NST;
    uint2* stash = reinterpret_cast<uint2*>((wave & 2) ? &lds_v[f][0] : &lds_k[f][0]) + (wave & 1) * (kRows * NCH * 2);
    const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            uint2 w;
            w.x = (uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 0] * inv) | ((uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 1] * inv) << 16);
            w.y = (uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 2] * inv) | ((uint32_t)f32_to_bf16_rne(o[mt][4 * r4 + 3] * inv) << 16);
            stash_put<D>(stash, col, half, mt, r4, w);
        }
    stash_store_rows<D>(stash, a.out + (size_t)hq * a.q_len * D, rb * kRows, a.q_len, lane);
    if (row_ok && half == 0 && a.lse != nullptr)
        a.lse[(size_t)hq * a.q_len + row] = l_row > 0.f ? (m_run + log2f(l_row)) * kLn2 : -INFINITY;
}

// ---- Row-block prefill for launches too small to fill the GPU ------------------------------
//
// One work-group per (query head, 32-row block): a 256-row chunk over 32 query heads is 256
// work-groups, one per CU, with no KV segments across work-groups and so no partials and no merge
// launch.  The NW = 8 waves (two per SIMD) take the row block's 32-key blocks in turn (wave w:
// blocks w, w+8, ...), each streaming its own K and V tile (one of each, refilled as soon as it has
// been read) with direct-to-LDS loads, so no wave waits for another inside the loop.  At the end the waves merge
// their (m, l, O) through LDS and write the bf16 rows.  Grid x is the kv head: work-groups are dealt
// to the XCDs round robin by linear index, so with 8 kv heads every work-group reading one head's
// K/V runs on the same XCD and finds them in its L2.  Fragment layouts are prefill_kernel's with one
// 32-key tile per block (S^T = K . Q^T one 32x32 tile, eight k-steps; O^T += V^T . P^T in two
// 16-key k-steps per 32-dim tile).
constexpr int kRowBN = 32;  // keys per block

// NW waves per work-group take the row block's key blocks in turn.
template <int D, bool PAGED, int NW>
__global__ __launch_bounds__(NW * 64) void prefill_rows_kernel(PrefillArgs a) {
    constexpr int kRowWaves = NW;
    constexpr int NCH = D / 8;         // 16-byte chunks per K/V row
    constexpr int KSTEPS = D / 16;     // QK k-steps
    constexpr int MT = D / 32;         // PV result tiles (32 dims each)
    constexpr int TILE = kRowBN * NCH; // 16-byte chunks per K (or V) tile
    constexpr int KA = KSTEPS > 3 ? 3 : KSTEPS - 1;  // K fragment reads in flight ahead of their MFMA
    constexpr int VA = 2;                            // V^T steps read ahead of their MFMA
    constexpr int DMA = TILE / 64;     // direct-to-LDS loads per lane per tile
    static_assert(DMA >= 1 && DMA * 64 == TILE, "tile shape");
    static_assert(D * kRows * 4 <= 2 * TILE * 16, "a wave's O^T fits its tiles");

    // Per wave: one K and one V tile, reused for the wave's O^T after the loop, and its rows' (m, l);
    // the row block's Q, loaded once for all waves.
    __shared__ __attribute__((aligned(16))) u32x4 lds[kRowWaves][2][TILE];
    __shared__ float lds_ml[kRowWaves][2][kRows];
    __shared__ __attribute__((aligned(16))) u32x4 lds_q[TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = blockIdx.x;  // kv head
    const int G = a.n_q_heads / a.n_kv_heads;
    const int n_rb = (a.q_len + kRows - 1) / kRows;
    const int g = blockIdx.y % G;
    // Causal row blocks grow in work with their index: the largest are dispatched first.
    const int rb = a.causal ? n_rb - 1 - (int)(blockIdx.y / G) : (int)(blockIdx.y / G);
    const int hq = h * G + g;

    int kv_hi = a.kv_len;  // keys the row block needs: [0, kv_hi)
    if (a.causal) kv_hi = min(kv_hi, a.q_pos_base + min(a.q_len, (rb + 1) * kRows) - 1 - a.kv_pos_base + 1);
    kv_hi = max(kv_hi, 0);
    const int n_blocks = (kv_hi + kRowBN - 1) / kRowBN;
    const int my_blocks = n_blocks > wave ? (n_blocks - wave + kRowWaves - 1) / kRowWaves : 0;

    const int col = lane & 31;   // query row within the block (MFMA column)
    const int half = lane >> 5;  // which 8 k-values of a step this lane carries
    const int row = rb * kRows + col;
    const bool row_ok = row < a.q_len;
    // Keys j < key_lim are valid for this lane's row: below kv_len and, causal, at or before the
    // row's position (kv_pos_base + j <= q_pos_base + row); none for a row past q_len.
    const int key_lim =
        row_ok ? min(a.kv_len, a.causal ? a.q_pos_base + row - a.kv_pos_base + 1 : a.kv_len) : 0;

    const u32x4* kg = reinterpret_cast<const u32x4*>(a.kc + (PAGED ? 0 : (size_t)h * a.l_cap * D));
    const u32x4* vg = reinterpret_cast<const u32x4*>(a.vc + (PAGED ? 0 : (size_t)h * a.l_cap * D));
    const bool has_new = a.k_new != nullptr && a.n_new > 0;
    const u32x4* kn = has_new ? reinterpret_cast<const u32x4*>(a.k_new) + (size_t)h * a.n_new * NCH : nullptr;
    const u32x4* vn = has_new ? reinterpret_cast<const u32x4*>(a.v_new) + (size_t)h * a.n_new * NCH : nullptr;
    const u32x4* zero = reinterpret_cast<const u32x4*>(a.zero_row);

    // Direct-to-LDS staging of the K (kv = 0) or V (kv = 1) tile of the block at key j0: load
    // instruction i fills slots i*64 + lane, and each lane loads the 16-byte chunk the swizzled layout
    // wants in its slot: byte offset koff[i] (K) / voff[i] (V) from the block's first row.  The K tile
    // of the next block is loaded as soon as S^T has read this one, and the V tile as soon as PV has,
    // so each load has the rest of a block's work to land behind.  A block whose rows all
    // come from one contiguous run -- the cache, or the rows this launch appends -- takes a
    // wave-uniform base and these fixed offsets; a block that straddles the appended rows or ends
    // past kv_len (zero row there: stale words may be NaN) picks each lane's source.
    uint32_t koff[DMA], voff[DMA];
#pragma unroll
    for (int i = 0; i < DMA; ++i) {
        const int slot = i * 64 + lane;
        const int key = slot / NCH;
        koff[i] = 16u * (uint32_t)(key * NCH + ((slot % NCH) ^ k_swz<NCH>(key)));
        voff[i] = 16u * (uint32_t)(key * NCH + ((slot % NCH) ^ v_swz<D>(key)));
    }
    const int new_end = has_new ? a.new_begin + a.n_new : 0;
    // pr: paged, the block's page row (paged_row_uniform of j0, looked up by the caller ahead of
    // time so the scalar load's latency hides behind other work; -1: unmapped, zero rows).
    auto issue = [&](int j0, int kv, int64_t pr) {
        // Row j0's K and V, or nullptr where the block's rows do not share one source.
        const u32x4* krow = nullptr;
        const u32x4* vrow = nullptr;
        if (j0 + kRowBN <= a.kv_len) {
            if (has_new && j0 >= a.new_begin && j0 + kRowBN <= new_end) {
                krow = kn + (size_t)(j0 - a.new_begin) * NCH;
                vrow = vn + (size_t)(j0 - a.new_begin) * NCH;
            } else if (!has_new || j0 + kRowBN <= a.new_begin || j0 >= new_end) {
                if constexpr (PAGED) {  // j0 and the page size are multiples of 32: one page per block
                    krow = pr < 0 ? nullptr : kg + (size_t)pr * NCH;
                    vrow = pr < 0 ? nullptr : vg + (size_t)pr * NCH;
                } else {
                    krow = kg + (size_t)j0 * NCH;
                    vrow = vg + (size_t)j0 * NCH;
                }
            }
        }
        if (krow != nullptr) {
            const uint64_t base = uniform_address(kv ? vrow : krow);
#pragma unroll
            for (int i = 0; i < DMA; ++i) dma16_sbase(base, kv ? voff[i] : koff[i], lds_addr(&lds[wave][kv][i * 64]));
            return;
        }
        const int64_t pr0 = pr;
#pragma unroll
        for (int i = 0; i < DMA; ++i) {
            const int rel = (int)(koff[i] >> 4) / NCH;  // key of this lane's slot within the block
            const int row_idx = j0 + rel;
            const uint32_t kc_off = koff[i] - 16u * (uint32_t)(rel * NCH);  // chunk offset within the row
            const uint32_t vc_off = voff[i] - 16u * (uint32_t)(rel * NCH);
            const u32x4* src;
            const unsigned r_new = (unsigned)(row_idx - a.new_begin);
            if (row_idx >= a.kv_len || (PAGED && pr0 < 0)) {
                src = zero;
            } else if (has_new && r_new < (unsigned)a.n_new) {
                src = (kv ? vn : kn) + (size_t)r_new * NCH;
            } else if constexpr (PAGED) {
                src = (kv ? vg : kg) + (size_t)(pr0 + rel) * NCH;
            } else {
                src = (kv ? vg : kg) + (size_t)row_idx * NCH;
            }
            dma16(reinterpret_cast<const uint8_t*>(src) + (kv ? vc_off : kc_off), lds_addr(&lds[wave][kv][i * 64]));
        }
    };

    // Operand addresses in this wave's tiles.
    uint32_t kaddr[KSTEPS];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
        kaddr[ks] = lds_addr(&lds[wave][0][0]) + 16u * (uint32_t)(col * NCH + ((2 * ks + half) ^ k_swz<NCH>(col)));
    uint32_t vaddr[MT];
    {
        const int key_off = (lane & 15) >> 2;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int dim = mt * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
            vaddr[mt] = lds_addr(&lds[wave][1][0]) + (uint32_t)((key_off + 4 * half) * (D * 2) +
                                                                   (((dim >> 3) ^ v_swz<D>(key_off)) << 4) +
                                                                   (((dim >> 2) & 1) << 3));
        }
    }

    f32x16 o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[mt][i] = 0.f;
    float m_run = -INFINITY;  // running max (log2 units) of this lane's row
    float l_lane = 0.f;       // this lane's half of the running sum
    constexpr float kLazyLog2 = 8.0f;  // the reference max moves only when passed by more than this
    constexpr float kFreeSum = 65536.0f;  // 2^16, as in prefill_kernel
    const float c = a.scale_log2;

    // Appended rows of kv head h go to the cache in equal shares over the kv head's work-groups;
    // blocks that hold them read k_new/v_new, so no work-group waits for the copy.  A thread's first
    // word is loaded first of all and stored after the wait below (the loop's own waits then cover
    // the store); any further words (more appended rows than threads) follow.
    const int app_words = has_new ? a.n_new * NCH : 0;
    const int app_stride = gridDim.y * (kRowWaves * 64);
    const int app_first = blockIdx.y * (kRowWaves * 64) + tid;
    auto app_dst = [&](int i) -> int64_t {  // 16-byte word index of appended word i, or -1 (unmapped)
        if constexpr (PAGED) {
            const int64_t r = paged_row(a.block_table, a.page_shift, a.n_kv_heads, h, a.new_begin + i / NCH);
            return r < 0 ? -1 : r * NCH + (i % NCH);
        } else {
            return ((int64_t)h * a.l_cap + a.new_begin) * NCH + i;
        }
    };
    // Every lane loads (past the appended words: the zero row), so the loads' results need no
    // merge with another value before the wait below that makes them valid.
    u32x4 app_k = load16_untracked(app_first < app_words ? kn + app_first : zero);
    u32x4 app_v = load16_untracked(app_first < app_words ? vn + app_first : zero);
    // Then Q^T's rows (row `row`, dims 16*ks + 8*half .. +7) and the wave's first K and V tiles.
    // Q of the row block goes to LDS once (the K tile's swizzled layout, rows past q_len from the zero
    // row), each lane one 16-byte chunk, instead of every wave loading all 32 rows.
    for (int base = wave * 64; base < TILE; base += kRowWaves * 64) {  // base is wave-uniform
        const int slot = base + lane;
        const int qrow = slot / NCH;
        const int chunk = (slot % NCH) ^ k_swz<NCH>(qrow);
        const u32x4* src = rb * kRows + qrow < a.q_len
                               ? reinterpret_cast<const u32x4*>(a.q + ((size_t)hq * a.q_len + rb * kRows + qrow) * D) + chunk
                               : zero + chunk;
        dma16(src, lds_addr(&lds_q[base]));
    }
    // Loads complete in issue order, so at most V(0)'s DMA loads in flight means the appended word,
    // Q and K(0) have landed: V(0) lands behind the first S^T (the loop waits for it before PV).
    if (my_blocks > 0) {
        const int64_t pr = PAGED ? paged_row_uniform(a.block_table, a.page_shift, a.n_kv_heads, h, wave * kRowBN) : 0;
        issue(wave * kRowBN, 0, pr);
        issue(wave * kRowBN, 1, pr);
    } else {
        wait_vmcnt<0>();
    }
    vm_wait<DMA>(app_k, app_v);
    __syncthreads();  // every wave's share of Q is in LDS
    u32x4 qb[KSTEPS];  // Q^T operand: row `row`, dims 16*ks + 8*half .. +7
    {
        const uint32_t qbase = lds_addr(&lds_q[0]);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
            qb[ks] = lds_read128(qbase + 16u * (uint32_t)(col * NCH + ((2 * ks + half) ^ k_swz<NCH>(col))));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    if (app_first < app_words) {
        const int64_t dst = app_dst(app_first);
        if (dst >= 0) {
            reinterpret_cast<u32x4*>(a.kc)[dst] = app_k;
            reinterpret_cast<u32x4*>(a.vc)[dst] = app_v;
        }
        for (int i = app_first + app_stride; i < app_words; i += app_stride) {
            const u32x4 wk = kn[i], wv = vn[i];
            const int64_t d2 = app_dst(i);
            if (d2 >= 0) {
                reinterpret_cast<u32x4*>(a.kc)[d2] = wk;
                reinterpret_cast<u32x4*>(a.vc)[d2] = wv;
            }
        }
        // The stores stay in flight: the loop's vmcnt waits also count them, which only makes the
        // first of those waits (V(0), before the first PV) wait for them as well.
    }

    // vm operations in flight enter the loop in the order K(t), V(t): K(t) (then K(t+1)) is issued
    // after S^T(t-1) (S^T(t)), V(t) after PV(t-1).
    for (int t = 0; t < my_blocks; ++t) {
        const int j0 = (wave + t * kRowWaves) * kRowBN;
        const bool more = t + 1 < my_blocks;
        // Paged: the next block's page row, needed after this block's S^T.
        const int64_t pr_next =
            PAGED && more ? paged_row_uniform(a.block_table, a.page_shift, a.n_kv_heads, h, j0 + kRowWaves * kRowBN) : 0;
        if (t >= 1) wait_vmcnt<DMA>();  // K(t) landed; V(t) may still be in flight

        // ---- S^T = K . Q^T (raw scores): one 32x32 tile, K fragments read KA steps ahead ----
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        f32x16 sacc;
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[i] = 0.f;
        u32x4 kf[KSTEPS];
        static_for<KA>([&](auto c) { kf[decltype(c)::value] = lds_read128(kaddr[decltype(c)::value]); });
        static_for<KSTEPS>([&](auto c) {
            constexpr int ks = decltype(c)::value;
            if constexpr (ks + KA < KSTEPS) {
                kf[ks + KA] = lds_read128(kaddr[ks + KA]);
                lgkm_wait1<KA>(kf[ks]);  // reads complete in order: at most the KA later ones remain
            } else {
                lgkm_wait1<KSTEPS - 1 - ks>(kf[ks]);
            }
            sacc = mfma32(kf[ks], qb[ks], sacc);
        });
        // Every read of the K tile is complete (lgkmcnt(0) above): it takes the next block's K.
        if (more) issue(j0 + kRowWaves * kRowBN, 0, pr_next);

        // ---- online softmax (log2 domain, scale folded into the exponent) ----
        const bool need_mask =
            (j0 + kRowBN > a.kv_len) || (a.causal && a.kv_pos_base + j0 + kRowBN - 1 > a.q_pos_base + rb * kRows);
        if (need_mask) {
            const int d = key_lim - (j0 + 4 * half);  // key j0 + 4*half + c is valid iff c < d
#pragma unroll
            for (int i = 0; i < 16; ++i) sacc[i] = 8 * (i >> 2) + (i & 3) < d ? sacc[i] : -INFINITY;
        }
        float psum = 0.f;
        u32x4 pb[2];  // P^T operand of the two PV k-steps (keys 0-15, 16-31 of the block)
        auto weights = [&]() __attribute__((always_inline)) {
            const float nm = (m_run == -INFINITY) ? 0.f : -m_run;
            psum = 0.f;
#pragma unroll
            for (int a2 = 0; a2 < 2; ++a2) {
                float p[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    p[j] = __builtin_amdgcn_exp2f(fmaf(sacc[8 * a2 + j], c, nm));
                    psum += p[j];
                }
                pb[a2] = u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                               pack_bf16x2(p[6], p[7])};
            }
        };
        // As in prefill_kernel: against the reference max directly once every row has one; the
        // block's own max only where a lane's weights sum past kFreeSum or overflow.
        bool need_max = __ballot(m_run == -INFINITY) != 0;
        if (!need_max) {
            weights();
            need_max = __ballot(!(psum <= kFreeSum)) != 0;  // also true for inf and NaN
        }
        if (need_max) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[i]);
            mx = pair_max32(mx);
            const float bm = mx * c;
            const bool grow = bm > m_run + kLazyLog2;
            if (__ballot(grow) != 0) {
                const float m_new = grow ? bm : m_run;
                const float corr = (m_run == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
                m_run = m_new;
                l_lane *= corr;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[mt][i] *= corr;
            }
            weights();
        }
        l_lane += psum;

        // ---- O^T += V^T . P^T, transposing V reads one step ahead ----
        if (more) wait_vmcnt<DMA>(); else wait_vmcnt<0>();  // V(t) landed; K(t+1) may still be in flight
        constexpr int PV = MT * 2;
        u32x2 vf[PV][2];
        auto read_v = [&](auto step_c) {
            constexpr int i = decltype(step_c)::value;
            constexpr int kb = 16 * (i & 1);  // step's key base within the block (half adds 4)
            const uint32_t va = vaddr[i >> 1];
            vf[i][0] = lds_read_tr64<kb * (D * 2)>(va);
            vf[i][1] = lds_read_tr64<(kb + 8) * (D * 2)>(va);
        };
        static_for<VA>([&](auto c) { read_v(c); });
        static_for<PV>([&](auto step_c) {
            constexpr int i = decltype(step_c)::value;
            if constexpr (i + VA < PV) {
                read_v(std::integral_constant<int, i + VA>{});
                lgkm_wait<2 * VA>(vf[i][0], vf[i][1]);  // two reads per step
            } else {
                lgkm_wait<2 * (PV - 1 - i)>(vf[i][0], vf[i][1]);
            }
            const u32x4 vw = {vf[i][0].x, vf[i][0].y, vf[i][1].x, vf[i][1].y};
            o[i >> 1] = mfma32(vw, pb[i & 1], o[i >> 1]);
        });
        // Every read of the V tile is complete (lgkmcnt(0) above): it takes the next block's V.
        if (more) issue(j0 + kRowWaves * kRowBN, 1, pr_next);
    }

    // ---- merge the waves: each writes (O^T [D][32 rows], m, l) to its own ring (no DMA pending) ----
    // O^T goes to LDS row-major, [32 rows][D] fp32, as 16-byte granules (four dims) XOR-swizzled by
    // the row so that neither the writes here nor the reads below conflict on banks.
    const float l_row = l_lane + half_swap(l_lane, half);
    constexpr int GR = D / 4;  // granules per row
    float4* mo = reinterpret_cast<float4*>(&lds[wave][0][0]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const int gran = 8 * mt + 2 * i4 + half;  // dims 4*gran .. +3 = mt*32 + 8*i4 + 4*half + 0..3
            mo[col * GR + (gran ^ (col % GR))] =
                make_float4(o[mt][4 * i4], o[mt][4 * i4 + 1], o[mt][4 * i4 + 2], o[mt][4 * i4 + 3]);
        }
    if (half == 0) {
        lds_ml[wave][0][col] = m_run;
        lds_ml[wave][1][col] = l_row;
    }
    __syncthreads();
    // The work-group's threads over 32 rows: each takes DPT dims (at least 8, one 16-byte store).
    constexpr int NDG = kRowWaves * 64 / kRows;
    constexpr int DPT = D / NDG >= 8 ? D / NDG : 8;
    const int r = tid & 31;
    const int dg = tid >> 5;
    const int out_row = rb * kRows + r;
    if (out_row >= a.q_len || dg * DPT >= D) return;
    float wt[kRowWaves];
    float M = -INFINITY, L = 0.f;
#pragma unroll
    for (int w = 0; w < kRowWaves; ++w) M = fmaxf(M, lds_ml[w][0][r]);
#pragma unroll
    for (int w = 0; w < kRowWaves; ++w) {
        const float mw = lds_ml[w][0][r];
        wt[w] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        L = fmaf(wt[w], lds_ml[w][1][r], L);
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint16_t* orow = a.out + ((size_t)hq * a.q_len + out_row) * D + dg * DPT;
#pragma unroll
    for (int d8 = 0; d8 < DPT; d8 += 8) {
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const int g0 = (dg * DPT + d8) / 4;  // first of the two granules of these eight dims
#pragma unroll
        for (int w = 0; w < kRowWaves; ++w) {
            const float4* wo = reinterpret_cast<const float4*>(&lds[w][0][0]) + r * GR;
            const float4 x0 = wo[g0 ^ (r % GR)];
            const float4 x1 = wo[(g0 + 1) ^ (r % GR)];
            v[0] = fmaf(wt[w], x0.x, v[0]);
            v[1] = fmaf(wt[w], x0.y, v[1]);
            v[2] = fmaf(wt[w], x0.z, v[2]);
            v[3] = fmaf(wt[w], x0.w, v[3]);
            v[4] = fmaf(wt[w], x1.x, v[4]);
            v[5] = fmaf(wt[w], x1.y, v[5]);
            v[6] = fmaf(wt[w], x1.z, v[6]);
            v[7] = fmaf(wt[w], x1.w, v[7]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] *= inv;
        uint4 wv;
        wv.x = (uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16);
        wv.y = (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16);
        wv.z = (uint32_t)f32_to_bf16_rne(v[4]) | ((uint32_t)f32_to_bf16_rne(v[5]) << 16);
        wv.w = (uint32_t)f32_to_bf16_rne(v[6]) | ((uint32_t)f32_to_bf16_rne(v[7]) << 16);
        *reinterpret_cast<uint4*>(orow + d8) = wv;
    }
    if (dg == 0 && a.lse != nullptr)
        a.lse[(size_t)hq * a.q_len + out_row] = L > 0.f ? (M + log2f(L)) * kLn2 : -INFINITY;
}

// Row-block kernel shape: 8 waves (two per SIMD: one wave's MFMAs run while the other waits on
// LDS or loads), one K and one V tile each: 128 KiB of LDS at D = 128.
constexpr int kRowWaves = 8;

template <int D>
hipError_t launch_prefill_rows_t(const PrefillArgs& a, const Launch& l) {
    const int n_rb = (a.q_len + kRows - 1) / kRows;
    const int G = a.n_q_heads / a.n_kv_heads;
    dim3 grid(a.n_kv_heads, G * n_rb);
    if (a.block_table != nullptr)
        return launch_kernel(prefill_rows_kernel<D, true, kRowWaves>, grid, dim3(kRowWaves * 64), l, a);
    return launch_kernel(prefill_rows_kernel<D, false, kRowWaves>, grid, dim3(kRowWaves * 64), l, a);
}

// Merge of a row's KV segments.  Segment s holds keys [s*seg_len, (s+1)*seg_len); a row
// reads the segments below its own key limit, which are exactly the ones prefill_kernel
// wrote for it.  A work-group merges kMergeRows rows of one query head; each row is handled
// by D/8 threads owning eight dims (16-byte fp16 loads).  The (m, l, scale) rows and O slices
// of up to kMergeBatch segments are loaded together, so a row pays one memory latency per batch.
constexpr int kMergeRows = 16;
constexpr int kMergeBatch = 8;
constexpr int kMaxMergeSegs = 16;  // segments a launch may have (the host planner's cap)
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <int D>
__global__ __launch_bounds__(kMergeRows * D / 8) void prefill_combine_kernel(PrefillArgs a) {
    constexpr int TPR = D / 8;  // threads per row
    const int hq = blockIdx.y;
    const int row = blockIdx.x * kMergeRows + threadIdx.x / TPR;
    const int d8 = threadIdx.x % TPR;
    if (row >= a.q_len) return;
    int hi = a.kv_len;
    if (a.causal) hi = min(hi, a.q_pos_base + row - a.kv_pos_base + 1);
    hi = max(hi, 0);
    const int n_valid = min(a.n_segs, (hi + a.seg_len - 1) / a.seg_len);
    const size_t seg_stride = (size_t)a.n_q_heads * a.q_len;
    const size_t prow = (size_t)hq * a.q_len + row;
    const float4* ml = reinterpret_cast<const float4*>(a.part_ml) + prow;
    const uint4* po = reinterpret_cast<const uint4*>(a.part_o) + prow * TPR + d8;
    // Segment s contributes 2^(m_s - M) * v_s * 2^(e_s) (M the largest m).  Split its log2 weight
    // into an integer n_s and a fraction: the contribution's exponent is x_s = e_s + n_s, and O
    // accumulates relative to X = max_s x_s, so the dominant contributions are scaled by about one
    // and every term is scaled down by an exact power of two: nothing overflows, and nothing that
    // matters to the sum is flushed, whatever the partials' magnitudes.
    float4 e[kMaxMergeSegs];  // (m, l, exponent, -) of each segment
#pragma unroll
    for (int j = 0; j < kMaxMergeSegs; ++j)
        e[j] = j < n_valid ? ml[(size_t)j * seg_stride] : make_float4(-INFINITY, 0.f, 0.f, 0.f);
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMaxMergeSegs; ++j) M = fmaxf(M, e[j].x);
    uint4 w = {0u, 0u, 0u, 0u};
    float Ls = 0.f;
    if (M != -INFINITY) {
        int n[kMaxMergeSegs];
        int X = INT_MIN;
#pragma unroll
        for (int j = 0; j < kMaxMergeSegs; ++j) {
            n[j] = (int)fmaxf(floorf(e[j].x - M), -1024.f);  // -1024 for an empty segment (m = -inf)
            if (e[j].x != -INFINITY) X = max(X, (int)e[j].z + n[j]);
            Ls = fmaf(__builtin_amdgcn_exp2f(e[j].x - M), e[j].y, Ls);
        }
        float O[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j0 = 0; j0 < kMaxMergeSegs; j0 += kMergeBatch) {
            if (j0 >= n_valid) break;
            f16x8 v[kMergeBatch];
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j)
                v[j] = j0 + j < n_valid ? __builtin_bit_cast(f16x8, po[(size_t)(j0 + j) * seg_stride * TPR])
                                        : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) {
                const float4& ej = e[j0 + j];
                const float wo = ej.x == -INFINITY ? 0.f
                                                   : ldexpf(__builtin_amdgcn_exp2f(ej.x - M - (float)n[j0 + j]),
                                                            (int)ej.z + n[j0 + j] - X);
#pragma unroll
                for (int i = 0; i < 8; ++i) O[i] = fmaf(wo, (float)v[j][i], O[i]);
            }
        }
        // out = O * 2^X / Ls, scaled back in one exact step after the division.
        const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
        float r8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) r8[i] = ldexpf(O[i] * inv, X);
        w.x = (uint32_t)f32_to_bf16_rne(r8[0]) | ((uint32_t)f32_to_bf16_rne(r8[1]) << 16);
        w.y = (uint32_t)f32_to_bf16_rne(r8[2]) | ((uint32_t)f32_to_bf16_rne(r8[3]) << 16);
        w.z = (uint32_t)f32_to_bf16_rne(r8[4]) | ((uint32_t)f32_to_bf16_rne(r8[5]) << 16);
        w.w = (uint32_t)f32_to_bf16_rne(r8[6]) | ((uint32_t)f32_to_bf16_rne(r8[7]) << 16);
    }
    *reinterpret_cast<uint4*>(a.out + prow * D + 8 * d8) = w;
    if (d8 == 0 && a.lse != nullptr) a.lse[prow] = Ls > 0.f ? (M + log2f(Ls)) * kLn2 : -INFINITY;
}

template <int D, int G>
hipError_t launch_prefill_t(const PrefillArgs& a, const Launch& l) {
    const int n_rb = (a.q_len + kRows - 1) / kRows;
    const int n_tasks = n_rb * G;
    dim3 grid((n_tasks + kWaves - 1) / kWaves, a.n_kv_heads, a.n_segs);
    if constexpr (G == 4) {
        if (a.pair) {
            // Paired row blocks: causal, one segment (the whole key range in one launch).
            if (!a.causal || a.n_segs != 1) return hipErrorInvalidValue;
            if (a.block_table != nullptr)
                return launch_kernel(prefill_kernel<D, G, true, true>, grid, dim3(kWaves * 64), l, a);
            return launch_kernel(prefill_kernel<D, G, false, true>, grid, dim3(kWaves * 64), l, a);
        }
    }
    if (a.block_table != nullptr) return launch_kernel(prefill_kernel<D, G, true, false>, grid, dim3(kWaves * 64), l, a);
    return launch_kernel(prefill_kernel<D, G, false, false>, grid, dim3(kWaves * 64), l, a);
}

}  // namespace

constexpr int kMinSegBlocks = 2;  // key blocks per KV segment, at least

PrefillPlan plan_prefill(int q_len, int kv_span, int group, int n_kv_heads, int target_wgs, int max_segs) {
    const int n_rb = (q_len + kRows - 1) / kRows;
    const int base = ((n_rb * group + kWaves - 1) / kWaves) * n_kv_heads;
    const int blocks = (kv_span + kBN - 1) / kBN;
    int segs = (target_wgs + base - 1) / base;
    segs = min(segs, max_segs);
    segs = min(segs, blocks / kMinSegBlocks);  // a segment of one block pays a whole work-group's fixed cost
    if (segs <= 1) return PrefillPlan{blocks > 0 ? blocks * kBN : kBN, 1};
    const int seg_blocks = (blocks + segs - 1) / segs;
    const int seg_len = seg_blocks * kBN;
    return PrefillPlan{seg_len, (blocks + seg_blocks - 1) / seg_blocks};
}

size_t prefill_workspace_floats(const PrefillPlan& p, int q_len, int n_q_heads, int head_dim) {
    if (p.n_segs <= 1) return 0;
    return (size_t)p.n_segs * n_q_heads * q_len * (head_dim / 2 + 4);  // fp16 O row + (m, l, scale, -)
}

hipError_t launch_prefill_combine(int head_dim, const PrefillArgs& a, const Launch& l) {
    if (a.n_segs > kMaxMergeSegs) return hipErrorInvalidValue;
    const dim3 grid((a.q_len + kMergeRows - 1) / kMergeRows, a.n_q_heads);
    if (head_dim == 128) return launch_kernel(prefill_combine_kernel<128>, grid, dim3(kMergeRows * 16), l, a);
    if (head_dim == 64) return launch_kernel(prefill_combine_kernel<64>, grid, dim3(kMergeRows * 8), l, a);
    return hipErrorInvalidValue;
}

hipError_t launch_prefill_rows(int head_dim, const PrefillArgs& a, const Launch& l) {
    if ((a.q_len + kRows - 1) / kRows * (a.n_q_heads / a.n_kv_heads) > 65535) return hipErrorInvalidValue;
    if (head_dim == 128) return launch_prefill_rows_t<128>(a, l);
    if (head_dim == 64) return launch_prefill_rows_t<64>(a, l);
    return hipErrorInvalidValue;
}

int prefill_shared_wgs(int q_len, int group, int n_kv_heads) {
    return ((q_len + kRows - 1) / kRows * group + kWaves - 1) / kWaves * n_kv_heads;
}

bool prefill_supported(int head_dim, int group) {
    return (head_dim == 64 || head_dim == 128) && (group == 1 || group == 2 || group == 4 || group == 8 || group == 16);
}

hipError_t launch_prefill(int head_dim, int group, const PrefillArgs& a, const Launch& l) {
    if (head_dim == 128) {
        if (group == 4) return launch_prefill_t<128, 4>(a, l);
        if (group == 8) return launch_prefill_t<128, 8>(a, l);
        if (group == 2) return launch_prefill_t<128, 2>(a, l);
        if (group == 1) return launch_prefill_t<128, 1>(a, l);
        if (group == 16) return launch_prefill_t<128, 16>(a, l);
    } else if (head_dim == 64) {
        if (group == 4) return launch_prefill_t<64, 4>(a, l);
        if (group == 8) return launch_prefill_t<64, 8>(a, l);
        if (group == 2) return launch_prefill_t<64, 2>(a, l);
        if (group == 1) return launch_prefill_t<64, 1>(a, l);
        if (group == 16) return launch_prefill_t<64, 16>(a, l);
    }
    return hipErrorInvalidValue;
}

}  // namespace lara
