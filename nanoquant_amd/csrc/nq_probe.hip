// Measurement aids for the decode GEMV's latency floor: an empty launch and a bare streaming
// read, the two things every launch of a decode-sized kernel pays before any arithmetic.
//
// probe_read_kernel reads `bytes` in equal contiguous runs, one per block, 16 bytes a lane, with
// every load of a lane issued before the first use (as the GEMV kernels issue theirs). The loads
// go through a buffer resource sized to the array, so lanes past the end read zeros and touch no
// memory. Without kStore, the xor of what a block read reaches memory only if it equals a
// constant, which keeps the loads alive without a store; with kStore, every block stores one word
// of it (as a GEMV stage stores its few outputs), so the launch also pays for a store.
#include "nq_common.h"

namespace nq {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeChunks = 16;  // 16-byte chunks per lane: up to 64 KB per block

__device__ inline uint32_t wave_xor(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v ^= __shfl_xor(v, off, 64);
    return v;
}

__global__ void probe_empty_kernel() {}

template <bool kStore>
__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const void* src, uint32_t bytes,
                                                                   uint32_t per_block, uint32_t* sink) {
    const rsrc_t rs = make_rsrc(src, bytes);
    const uint32_t base = blockIdx.x * per_block;
    const uint32_t end = min(base + per_block, bytes);
    u32x4 v[kProbeChunks];
#pragma unroll
    for (int k = 0; k < kProbeChunks; ++k) {
        const uint32_t off = base + 16u * (threadIdx.x + kProbeThreads * k);
        v[k] = load_b128_stream(rs, off < end ? off : bytes);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < kProbeChunks; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    if (kStore) {
        acc = wave_xor(acc);
        if (threadIdx.x == 0) sink[blockIdx.x] = acc;
    } else if (acc == 0x9E3779B9u) {
        sink[blockIdx.x] = acc;
    }
}

}  // namespace
}  // namespace nq

extern "C" {

int nq_probe_empty(int64_t blocks, int64_t threads, nq_stream_t stream) {
    if (blocks < 1 || blocks > (1 << 20) || threads < 1 || threads > 1024)
        return nq::fail(NQ_ERR_INVALID_ARGUMENT, "nq_probe_empty: blocks %lld threads %lld", (long long)blocks,
                        (long long)threads);
    nq::probe_empty_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(static_cast<unsigned>(threads)), 0,
                             nq::as_stream(stream)>>>();
    return nq::check_launch("nq_probe_empty");
}

int nq_probe_read(const void* src, int64_t bytes, int64_t blocks, uint32_t* sink, int store, nq_stream_t stream) {
    if (!src || !sink || bytes < 16 || blocks < 1 || blocks > (1 << 20))
        return nq::fail(NQ_ERR_INVALID_ARGUMENT, "nq_probe_read: null pointer, empty read or blocks out of range");
    if (bytes % 16 || !nq::aligned(src, 16))
        return nq::fail(NQ_ERR_ALIGNMENT, "nq_probe_read: bytes and src must be multiples of 16");
    if (bytes >= (int64_t(1) << 31))
        return nq::fail(NQ_ERR_SHAPE, "nq_probe_read: %lld bytes past the 2 GiB offset range", (long long)bytes);
    const int64_t per_block = nq::ceil_div(nq::ceil_div(bytes, blocks), 16) * 16;
    if (per_block > int64_t(16) * nq::kProbeThreads * nq::kProbeChunks)
        return nq::fail(NQ_ERR_SHAPE, "nq_probe_read: %lld bytes per block past 64 KB", (long long)per_block);
    const dim3 grid(static_cast<unsigned>(blocks));
    const uint32_t b = static_cast<uint32_t>(bytes), pb = static_cast<uint32_t>(per_block);
    if (store) nq::probe_read_kernel<true><<<grid, nq::kProbeThreads, 0, nq::as_stream(stream)>>>(src, b, pb, sink);
    else nq::probe_read_kernel<false><<<grid, nq::kProbeThreads, 0, nq::as_stream(stream)>>>(src, b, pb, sink);
    return nq::check_launch("nq_probe_read");
}

}  // extern "C"
