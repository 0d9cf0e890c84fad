// K/V cache row append for the GQA engine.
//
// The KV260 writes its per-group cache at address token*HEAD_DIM + dim from a scalar
// bf16 stream and reloads the whole cache on every transaction
// (hw/rtl/mem/kv_cache_ram.sv:77-91, sw/attn_driver.py:418-422).  Here the cache is
// resident in HBM as [B][H_kv][L_cap][D] and a decode step appends one row per
// (sequence, kv head).  The copy moves whole 16-byte words, so it is bit-exact.
#include "gqa_internal.h"

namespace lara {

// One thread per 16-byte word of the [B][H_kv][D] source rows.  Contiguous cache: row pos of
// (b, h) at (b*H_kv + h)*l_cap + pos; paged cache: see paged_row.
__global__ __launch_bounds__(256) void append_kv_kernel(const u32x4* __restrict__ k_rows,
                                                        const u32x4* __restrict__ v_rows,
                                                        const int32_t* __restrict__ positions,
                                                        u32x4* __restrict__ kc, u32x4* __restrict__ vc,
                                                        int n_words, int words_per_row, int n_kv_heads,
                                                        int l_cap, int l_max, const int32_t* __restrict__ table,
                                                        int page_shift, int max_pages) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_words) return;
    const int unit = idx / words_per_row;  // b * H_kv + h
    const int w = idx - unit * words_per_row;
    const int b = unit / n_kv_heads;
    const int pos = positions[b];
    if (pos < 0 || pos >= l_max) return;
    int64_t row;
    if (table != nullptr) {
        row = paged_row(table + (size_t)b * max_pages, page_shift, n_kv_heads, unit - b * n_kv_heads, pos);
        if (row < 0) return;  // unmapped page: nothing to write
    } else {
        row = (int64_t)unit * l_cap + pos;
    }
    const size_t dst = (size_t)row * words_per_row + w;
    kc[dst] = k_rows[idx];
    vc[dst] = v_rows[idx];
}

hipError_t launch_append(const uint16_t* k_rows, const uint16_t* v_rows, const int32_t* positions,
                         uint16_t* kc, uint16_t* vc, int batch, int n_kv_heads, int head_dim,
                         int l_cap, int l_max, const int32_t* block_table, int page_shift, int max_pages,
                         const Launch& l) {
    const int words_per_row = head_dim / 8;
    const int n_words = batch * n_kv_heads * words_per_row;
    const int block = 256;
    const int grid = (n_words + block - 1) / block;
    return launch_kernel(append_kv_kernel, dim3(grid), dim3(block), l, reinterpret_cast<const u32x4*>(k_rows),
                         reinterpret_cast<const u32x4*>(v_rows), positions, reinterpret_cast<u32x4*>(kc),
                         reinterpret_cast<u32x4*>(vc), n_words, words_per_row, n_kv_heads, l_cap, l_max, block_table,
                         page_shift, max_pages);
}

}  // namespace lara
