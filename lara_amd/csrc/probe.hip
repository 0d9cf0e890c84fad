// Streaming-read ceiling probe for gfx950: the HBM read rate the decode kernel's roofline
// fraction is compared with, measured with the decode kernel's own access pattern.
//
// Each 512-thread work-group reads one contiguous share of the buffer in 16-byte nontemporal
// loads (1 KiB per wave instruction), UNROLL loads in flight per thread.  The loaded words are
// folded with XOR and written only when the fold hits one particular value, so the loads stay
// live but the probe writes (almost) nothing: the measured rate is a pure read rate.
#include "gqa_internal.h"

namespace lara {
namespace {

constexpr int kProbeThreads = 512;
constexpr uint32_t kSinkTrigger = 0x9E3779B9u;

template <int UNROLL>
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n_words,
                                                                    int64_t words_per_wg, uint32_t* __restrict__ sink) {
    const int64_t begin = (int64_t)blockIdx.x * words_per_wg;
    const int64_t end = begin + words_per_wg < n_words ? begin + words_per_wg : n_words;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (int64_t i = begin + threadIdx.x; i < end; i += (int64_t)kProbeThreads * UNROLL) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t j = i + (int64_t)u * kProbeThreads;
            v[u] = j < end ? __builtin_nontemporal_load(src + j) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u];
    }
    const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (x == kSinkTrigger) sink[blockIdx.x] = x;
}

}  // namespace

hipError_t launch_stream_read(const void* src, int64_t n_bytes, int n_wgs, int unroll, uint32_t* sink,
                              const Launch& l) {
    const int64_t n_words = n_bytes / 16;
    const int64_t per_wg = (n_words + n_wgs - 1) / n_wgs;
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
    const dim3 grid(n_wgs), block(kProbeThreads);
    switch (unroll) {
        case 1: return launch_kernel(stream_read_kernel<1>, grid, block, l, s, n_words, per_wg, sink);
        case 2: return launch_kernel(stream_read_kernel<2>, grid, block, l, s, n_words, per_wg, sink);
        case 4: return launch_kernel(stream_read_kernel<4>, grid, block, l, s, n_words, per_wg, sink);
        case 8: return launch_kernel(stream_read_kernel<8>, grid, block, l, s, n_words, per_wg, sink);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace lara
