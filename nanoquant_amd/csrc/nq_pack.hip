// Sign-bit packing kernels: the two 32-column word orders (lsb_first, half2),
// the reorder between them, and the Marlin GEMM layout.
//
// All of them are HBM-bound integer work: one thread owns one output word (the
// unpacker of whole-word rows: two 16-byte halves of int8 output) so every load
// and store is a plain coalesced vector access and no thread needs another
// thread's data.
#include "nq_common.h"

namespace nq {
namespace {

constexpr int kThreads = 256;

// --------------------------------------------------------------------------- bit order transforms
// lsb_first word L: element j at bit j. half2 word H: element j at bit 15 - j/2 + 16*(j%2),
// i.e. the even elements bit-reversed into the low half and the odd ones into the high half:
// H = brev((even(L) << 16) | odd(L)) where even/odd compress every other bit.

__device__ inline uint32_t compress_even_bits(uint32_t x) {
    x &= 0x55555555u;
    x = (x | (x >> 1)) & 0x33333333u;
    x = (x | (x >> 2)) & 0x0F0F0F0Fu;
    x = (x | (x >> 4)) & 0x00FF00FFu;
    x = (x | (x >> 8)) & 0x0000FFFFu;
    return x;
}

__device__ inline uint32_t spread_to_even_bits(uint32_t x) {
    x &= 0x0000FFFFu;
    x = (x | (x << 8)) & 0x00FF00FFu;
    x = (x | (x << 4)) & 0x0F0F0F0Fu;
    x = (x | (x << 2)) & 0x33333333u;
    x = (x | (x << 1)) & 0x55555555u;
    return x;
}

__device__ inline uint32_t lsb_to_half2(uint32_t L) {
    return __builtin_bitreverse32((compress_even_bits(L) << 16) | compress_even_bits(L >> 1));
}

__device__ inline uint32_t half2_to_lsb(uint32_t H) {
    const uint32_t t = __builtin_bitreverse32(H);
    return spread_to_even_bits(t >> 16) | (spread_to_even_bits(t) << 1);
}

__device__ inline uint32_t to_method(uint32_t L, int method) { return method == NQ_PACK_HALF2 ? lsb_to_half2(L) : L; }
__device__ inline uint32_t from_method(uint32_t W, int method) { return method == NQ_PACK_HALF2 ? half2_to_lsb(W) : W; }

// Four int8 values packed little-endian in a dword -> 4 bits (1 where the byte is negative).
__device__ inline uint32_t sign_nibble(uint32_t four_bytes) {
    const uint32_t m = (four_bytes >> 7) & 0x01010101u;
    return (m * 0x10204080u) >> 28;
}

// 4 bits -> four int8 values (+1 for a clear bit, -1 for a set bit), little-endian.
__device__ inline uint32_t nibble_to_signs(uint32_t nib) {
    const uint32_t m = ((nib & 0xFu) * 0x00204081u) & 0x01010101u;
    return 0x01010101u + m * 0xFEu;
}

// --------------------------------------------------------------------------- 32-column words

// Whole-word rows (cols = 32 * words) from a 16-byte aligned source: word t's 32 bytes sit at
// src + 32 t, so no row index is needed; one thread per word, two 16-byte loads.
__global__ __launch_bounds__(kThreads) void pack_signs_words_kernel(const int8_t* __restrict__ src,
                                                                    uint32_t* __restrict__ dst, int64_t total,
                                                                    int method) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= total) return;
    const u32x4 a = *reinterpret_cast<const u32x4*>(src + t * 32);
    const u32x4 b = *reinterpret_cast<const u32x4*>(src + t * 32 + 16);
    const uint32_t L = sign_nibble(a.x) | (sign_nibble(a.y) << 4) | (sign_nibble(a.z) << 8) |
                       (sign_nibble(a.w) << 12) | (sign_nibble(b.x) << 16) | (sign_nibble(b.y) << 20) |
                       (sign_nibble(b.z) << 24) | (sign_nibble(b.w) << 28);
    dst[t] = to_method(L, method);
}

// The inverse, whole-word rows into a 16-byte aligned destination: a block owns 256 words and
// thread j writes the 16-byte halves j and j + 256 of their 512, so each store of a wave covers
// 1 KB contiguously (one thread per word storing both halves left every store 32-byte strided).
// Over 8 rotating [1632, 11008] copies: 6.8 us before, 5.75 us; packing 4.78 -> 4.58 us without
// the per-thread 64-bit row division.
__global__ __launch_bounds__(kThreads) void unpack_signs_words_kernel(const uint32_t* __restrict__ src,
                                                                      int8_t* __restrict__ dst, int64_t total,
                                                                      int method) {
    const int j = static_cast<int>(threadIdx.x);
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads;
    const int half = j & 1;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int64_t w = base + 128 * s + (j >> 1);
        if (w < total) {
            const uint32_t L = from_method(src[w], method) >> (16 * half);
            u32x4 a;
            a.x = nibble_to_signs(L);
            a.y = nibble_to_signs(L >> 4);
            a.z = nibble_to_signs(L >> 8);
            a.w = nibble_to_signs(L >> 12);
            *reinterpret_cast<u32x4*>(dst + w * 32 + half * 16) = a;
        }
    }
}

// Any other shape or alignment: one thread per word, bytewise over the row's valid columns.
__global__ __launch_bounds__(kThreads) void pack_signs_kernel(const int8_t* __restrict__ src,
                                                              uint32_t* __restrict__ dst, int64_t rows,
                                                              int64_t cols, int64_t words, int method) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= rows * words) return;
    const int64_t row = t / words;
    const int64_t w = t - row * words;
    const int8_t* p = src + row * cols + w * 32;
    uint32_t L = 0;
    const int64_t valid = cols - w * 32 < 32 ? cols - w * 32 : 32;
    for (int e = 0; e < valid; ++e) L |= static_cast<uint32_t>(p[e] < 0) << e;
    dst[t] = to_method(L, method);
}

__global__ __launch_bounds__(kThreads) void unpack_signs_kernel(const uint32_t* __restrict__ src,
                                                                int8_t* __restrict__ dst, int64_t rows,
                                                                int64_t cols, int64_t words, int method) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= rows * words) return;
    const int64_t row = t / words;
    const int64_t w = t - row * words;
    const uint32_t L = from_method(src[t], method);
    int8_t* p = dst + row * cols + w * 32;
    const int64_t valid = cols - w * 32 < 32 ? cols - w * 32 : 32;
    for (int e = 0; e < valid; ++e) p[e] = ((L >> e) & 1u) ? int8_t(-1) : int8_t(1);
}

template <bool kWhole>
__global__ __launch_bounds__(kThreads) void repack_signs_kernel(const uint32_t* __restrict__ src,
                                                                 uint32_t* __restrict__ dst, int64_t rows,
                                                                 int64_t cols, int64_t words, int src_method,
                                                                 int dst_method) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= rows * words) return;
    uint32_t L = from_method(src[t], src_method);
    if (!kWhole) {  // cols % 32 != 0: the row's last word has padding columns
        const int64_t w = t % words;
        const int64_t valid = cols - w * 32;
        if (valid < 32) L &= (1u << valid) - 1u;  // padding columns stay +1
    }
    dst[t] = to_method(L, dst_method);
}

// --------------------------------------------------------------------------- Marlin layout
// Word (tr, col) of the [K/16, O/2] array holds, for tile_out = col/32, o1 = (col%32)/4 and
// r2 = col%4, the 32 elements o = 64*tile_out + 16*o16 + 8*o8 + o1 (o16 < 4, o8 < 2) by
// k = 16*tr + 8*r8 + 2*r2 + r1 (r8, r1 < 2), element (o16, o8, r8, r1) at bit
// 15 - (2*o8 + r8) + 16*r1 - 4*o16. Each (o, r8) pair of k-adjacent int8 values is one
// 2-byte access.

__global__ __launch_bounds__(kThreads) void pack_marlin_kernel(const int8_t* __restrict__ w,
                                                               uint32_t* __restrict__ dst, int64_t O,
                                                               int64_t K) {
    const int64_t half_o = O / 2;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= (K / 16) * half_o) return;
    const int64_t tr = t / half_o;
    const int64_t col = t - tr * half_o;
    const int64_t tile_out = col / 32;
    const int o1 = static_cast<int>((col % 32) / 4);
    const int r2 = static_cast<int>(col % 4);
    uint32_t word = 0;
#pragma unroll
    for (int o16 = 0; o16 < 4; ++o16) {
#pragma unroll
        for (int o8 = 0; o8 < 2; ++o8) {
            const int64_t o = tile_out * 64 + o16 * 16 + o8 * 8 + o1;
#pragma unroll
            for (int r8 = 0; r8 < 2; ++r8) {
                const int64_t k = tr * 16 + r8 * 8 + r2 * 2;
                const uint16_t pair = *reinterpret_cast<const uint16_t*>(w + o * K + k);
                const uint32_t neg_lo = (pair >> 7) & 1u;   // element k   (r1 = 0)
                const uint32_t neg_hi = (pair >> 15) & 1u;  // element k+1 (r1 = 1)
                const int bit = 15 - (2 * o8 + r8) - 4 * o16;
                word |= (neg_lo << bit) | (neg_hi << (bit + 16));
            }
        }
    }
    dst[t] = word;
}

// The same words from a 16-byte aligned matrix, one block per 64 outputs x kMarlinTileK k: the
// block's 64 row segments reach LDS by 16-byte loads (16 lanes over a row's 256 bytes, where one
// thread per word made 2-byte loads spread over eight rows), then each thread assembles words
// from LDS and a tile row's 32 words go out as one 128-byte run. V^T [1792, 11008] over 8
// rotating copies: 25.4 us one thread per word, 6.34 us tiled, 5.77 us with each thread's four
// loads issued before their LDS stores (a 512-k tile with eight: 6.42).
constexpr int kMarlinTileK = 256;
constexpr int kMarlinRowStride = kMarlinTileK + 16;  // bytes: rows 4 banks apart, 16-byte aligned

__global__ __launch_bounds__(kThreads) void pack_marlin_tiled_kernel(const int8_t* __restrict__ w,
                                                                     uint32_t* __restrict__ dst, int64_t O,
                                                                     int64_t K) {
    __shared__ __attribute__((aligned(16))) int8_t tile[64 * kMarlinRowStride];
    const int t = static_cast<int>(threadIdx.x);
    const int64_t tile_out = blockIdx.y;
    const int64_t k0 = static_cast<int64_t>(blockIdx.x) * kMarlinTileK;
    const int kn = static_cast<int>(K - k0 < kMarlinTileK ? K - k0 : kMarlinTileK);  // a multiple of 16
    constexpr int kChunks = kMarlinTileK / 16;  // 16-byte chunks of a full row segment
    constexpr int kPer = 64 * kChunks / kThreads;  // 16-byte loads per thread, all issued before their stores
    u32x4 v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = t + j * kThreads;
        const int r = i / kChunks, c = i - r * kChunks;
        v[j] = 16 * c < kn ? *reinterpret_cast<const u32x4*>(w + (tile_out * 64 + r) * K + k0 + 16 * c) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = t + j * kThreads;
        const int r = i / kChunks, c = i - r * kChunks;
        if (16 * c < kn) *reinterpret_cast<u32x4*>(tile + r * kMarlinRowStride + 16 * c) = v[j];
    }
    __syncthreads();
    const int64_t half_o = O / 2;
    for (int i = t; i < (kn / 16) * 32; i += kThreads) {
        const int trl = i / 32, cl = i - trl * 32;
        const int o1 = cl / 4, r2 = cl % 4;
        uint32_t word = 0;
#pragma unroll
        for (int o16 = 0; o16 < 4; ++o16) {
#pragma unroll
            for (int o8 = 0; o8 < 2; ++o8) {
#pragma unroll
                for (int r8 = 0; r8 < 2; ++r8) {
                    const int row = o16 * 16 + o8 * 8 + o1;
                    const int kk = trl * 16 + r8 * 8 + r2 * 2;
                    const uint16_t pair = *reinterpret_cast<const uint16_t*>(tile + row * kMarlinRowStride + kk);
                    const uint32_t neg_lo = (pair >> 7) & 1u;   // element k   (r1 = 0)
                    const uint32_t neg_hi = (pair >> 15) & 1u;  // element k+1 (r1 = 1)
                    const int bit = 15 - (2 * o8 + r8) - 4 * o16;
                    word |= (neg_lo << bit) | (neg_hi << (bit + 16));
                }
            }
        }
        dst[(k0 / 16 + trl) * half_o + tile_out * 32 + cl] = word;
    }
}

// Marlin words [K_pad/16, O_pad/2] straight from the sign words of a [O, K] matrix (lsb_first
// or half2, ceil(K/32) words a row), as a checkpoint stores V [r, n] and U [m, r]; elements past
// O or K are +1 (bit 0). Each output word's four k lie in one 16-k group, so in one source word
// per row.
__global__ __launch_bounds__(kThreads) void repack_marlin_kernel(const uint32_t* __restrict__ src, int64_t O,
                                                                 int64_t K, int64_t words, int method,
                                                                 uint32_t* __restrict__ dst, int64_t O_pad,
                                                                 int64_t K_pad) {
    const int64_t half_o = O_pad / 2;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= (K_pad / 16) * half_o) return;
    const int64_t tr = t / half_o;
    const int64_t col = t - tr * half_o;
    const int64_t tile_out = col / 32;
    const int o1 = static_cast<int>((col % 32) / 4);
    const int r2 = static_cast<int>(col % 4);
    const int64_t k0 = tr * 16 + r2 * 2;  // the word's k: k0 + 8*r8 + r1
    uint32_t word = 0;
    if (k0 < K) {
        const int64_t kw = k0 / 32;
#pragma unroll
        for (int o16 = 0; o16 < 4; ++o16) {
#pragma unroll
            for (int o8 = 0; o8 < 2; ++o8) {
                const int64_t o = tile_out * 64 + o16 * 16 + o8 * 8 + o1;
                if (o >= O) continue;
                const uint32_t L = from_method(src[o * words + kw], method);
#pragma unroll
                for (int r8 = 0; r8 < 2; ++r8) {
#pragma unroll
                    for (int r1 = 0; r1 < 2; ++r1) {
                        const int64_t k = k0 + 8 * r8 + r1;
                        const uint32_t neg = k < K ? (L >> (k % 32)) & 1u : 0u;
                        word |= neg << (15 - (2 * o8 + r8) - 4 * o16 + 16 * r1);
                    }
                }
            }
        }
    }
    dst[t] = word;
}

__global__ __launch_bounds__(kThreads) void unpack_marlin_kernel(const uint32_t* __restrict__ src,
                                                                 int8_t* __restrict__ w, int64_t O, int64_t K) {
    const int64_t half_o = O / 2;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= (K / 16) * half_o) return;
    const int64_t tr = t / half_o;
    const int64_t col = t - tr * half_o;
    const int64_t tile_out = col / 32;
    const int o1 = static_cast<int>((col % 32) / 4);
    const int r2 = static_cast<int>(col % 4);
    const uint32_t word = src[t];
#pragma unroll
    for (int o16 = 0; o16 < 4; ++o16) {
#pragma unroll
        for (int o8 = 0; o8 < 2; ++o8) {
            const int64_t o = tile_out * 64 + o16 * 16 + o8 * 8 + o1;
#pragma unroll
            for (int r8 = 0; r8 < 2; ++r8) {
                const int64_t k = tr * 16 + r8 * 8 + r2 * 2;
                const int bit = 15 - (2 * o8 + r8) - 4 * o16;
                const uint16_t lo = ((word >> bit) & 1u) ? 0xFFu : 0x01u;
                const uint16_t hi = ((word >> (bit + 16)) & 1u) ? 0xFFu : 0x01u;
                *reinterpret_cast<uint16_t*>(w + o * K + k) = static_cast<uint16_t>(lo | (hi << 8));
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void permute_scales_kernel(const uint16_t* __restrict__ s_in,
                                                                  uint16_t* __restrict__ s_in_out, int64_t K,
                                                                  const uint16_t* __restrict__ s_out,
                                                                  uint16_t* __restrict__ s_out_out, int64_t O) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (s_in != nullptr && i < K) {
        const int64_t c = i / 16, a = (i % 16) / 8, b = (i % 8) / 2, d = i % 2;
        s_in_out[16 * c + 4 * b + 2 * a + d] = s_in[i];
    }
    if (s_out != nullptr && i < O) {
        const int64_t c = i / 32, a = (i % 32) / 8, b = (i % 8) / 2, d = i % 2;
        s_out_out[32 * c + 8 * b + 2 * a + d] = s_out[i];
    }
}

inline dim3 grid_for(int64_t items) { return dim3(static_cast<unsigned>(ceil_div(items, kThreads))); }

int check_method(int method, const char* name) {
    if (method != NQ_PACK_LSB_FIRST && method != NQ_PACK_HALF2)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: unknown bit order %d", name, method);
    return NQ_OK;
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" {

int nq_pack_signs(const int8_t* src, uint32_t* dst, int64_t rows, int64_t cols, int method, nq_stream_t stream) {
    if (int s = check_method(method, "nq_pack_signs")) return s;
    if (rows < 0 || cols < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_pack_signs: negative size");
    const int64_t words = ceil_div(cols, 32);
    if (rows == 0 || words == 0) return NQ_OK;
    if (!src || !dst) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_pack_signs: null pointer");
    const bool vec = (cols % 32 == 0) && aligned(src, 16);
    if (vec)
        pack_signs_words_kernel<<<grid_for(rows * words), kThreads, 0, as_stream(stream)>>>(src, dst, rows * words,
                                                                                             method);
    else
        pack_signs_kernel<<<grid_for(rows * words), kThreads, 0, as_stream(stream)>>>(src, dst, rows, cols, words,
                                                                                      method);
    return check_launch("nq_pack_signs");
}

int nq_unpack_signs(const uint32_t* src, int8_t* dst, int64_t rows, int64_t cols, int method, nq_stream_t stream) {
    if (int s = check_method(method, "nq_unpack_signs")) return s;
    if (rows < 0 || cols < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_unpack_signs: negative size");
    const int64_t words = ceil_div(cols, 32);
    if (rows == 0 || words == 0) return NQ_OK;
    if (!src || !dst) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_unpack_signs: null pointer");
    const bool vec = (cols % 32 == 0) && aligned(dst, 16);
    if (vec)
        unpack_signs_words_kernel<<<grid_for(rows * words), kThreads, 0, as_stream(stream)>>>(src, dst,
                                                                                               rows * words, method);
    else
        unpack_signs_kernel<<<grid_for(rows * words), kThreads, 0, as_stream(stream)>>>(src, dst, rows, cols, words,
                                                                                        method);
    return check_launch("nq_unpack_signs");
}

int nq_repack_signs(const uint32_t* src, uint32_t* dst, int64_t rows, int64_t cols, int src_method, int dst_method,
                    nq_stream_t stream) {
    if (int s = check_method(src_method, "nq_repack_signs")) return s;
    if (int s = check_method(dst_method, "nq_repack_signs")) return s;
    if (rows < 0 || cols < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_repack_signs: negative size");
    const int64_t words = ceil_div(cols, 32);
    if (rows == 0 || words == 0) return NQ_OK;
    if (!src || !dst) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_repack_signs: null pointer");
    if (cols % 32 == 0)
        repack_signs_kernel<true><<<grid_for(rows * words), kThreads, 0, as_stream(stream)>>>(
            src, dst, rows, cols, words, src_method, dst_method);
    else
        repack_signs_kernel<false><<<grid_for(rows * words), kThreads, 0, as_stream(stream)>>>(
            src, dst, rows, cols, words, src_method, dst_method);
    return check_launch("nq_repack_signs");
}

int nq_pack_marlin(const int8_t* weight, uint32_t* dst, int64_t O, int64_t K, nq_stream_t stream) {
    if (O < 0 || K < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_pack_marlin: negative size");
    if (O % 64 || K % 16) return fail(NQ_ERR_SHAPE, "nq_pack_marlin: need O %% 64 == 0 and K %% 16 == 0, got O=%lld K=%lld",
                                      (long long)O, (long long)K);
    if (O == 0 || K == 0) return NQ_OK;
    if (!weight || !dst) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_pack_marlin: null pointer");
    if (!aligned(weight, 2)) return fail(NQ_ERR_ALIGNMENT, "nq_pack_marlin: weight must be 2-byte aligned");
    if (aligned(weight, 16))
        pack_marlin_tiled_kernel<<<dim3(static_cast<unsigned>(ceil_div(K, kMarlinTileK)), static_cast<unsigned>(O / 64)),
                                   kThreads, 0, as_stream(stream)>>>(weight, dst, O, K);
    else
        pack_marlin_kernel<<<grid_for((K / 16) * (O / 2)), kThreads, 0, as_stream(stream)>>>(weight, dst, O, K);
    return check_launch("nq_pack_marlin");
}

int nq_repack_marlin(const uint32_t* src, int64_t O, int64_t K, int method, uint32_t* dst, int64_t O_pad,
                     int64_t K_pad, nq_stream_t stream) {
    if (int s = check_method(method, "nq_repack_marlin")) return s;
    if (O < 0 || K < 0 || O_pad < O || K_pad < K)
        return fail(NQ_ERR_INVALID_ARGUMENT, "nq_repack_marlin: need 0 <= O <= O_pad and 0 <= K <= K_pad");
    if (O_pad % 64 || K_pad % 16)
        return fail(NQ_ERR_SHAPE, "nq_repack_marlin: need O_pad %% 64 == 0 and K_pad %% 16 == 0, got O_pad=%lld K_pad=%lld",
                    (long long)O_pad, (long long)K_pad);
    if (O_pad == 0 || K_pad == 0) return NQ_OK;
    if (!dst || (O > 0 && K > 0 && !src)) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_repack_marlin: null pointer");
    repack_marlin_kernel<<<grid_for((K_pad / 16) * (O_pad / 2)), kThreads, 0, as_stream(stream)>>>(
        src, O, K, ceil_div(K, 32), method, dst, O_pad, K_pad);
    return check_launch("nq_repack_marlin");
}

int nq_unpack_marlin(const uint32_t* words, int8_t* weight, int64_t O, int64_t K, nq_stream_t stream) {
    if (O < 0 || K < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_unpack_marlin: negative size");
    if (O % 64 || K % 16) return fail(NQ_ERR_SHAPE, "nq_unpack_marlin: need O %% 64 == 0 and K %% 16 == 0");
    if (O == 0 || K == 0) return NQ_OK;
    if (!weight || !words) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_unpack_marlin: null pointer");
    if (!aligned(weight, 2)) return fail(NQ_ERR_ALIGNMENT, "nq_unpack_marlin: weight must be 2-byte aligned");
    unpack_marlin_kernel<<<grid_for((K / 16) * (O / 2)), kThreads, 0, as_stream(stream)>>>(words, weight, O, K);
    return check_launch("nq_unpack_marlin");
}

int nq_permute_marlin_scales(const uint16_t* scale_in, uint16_t* scale_in_out, int64_t K, const uint16_t* scale_out,
                             uint16_t* scale_out_out, int64_t O, nq_stream_t stream) {
    if ((scale_in == nullptr) != (scale_in_out == nullptr) || (scale_out == nullptr) != (scale_out_out == nullptr))
        return fail(NQ_ERR_INVALID_ARGUMENT, "nq_permute_marlin_scales: give both pointers of a pair or neither");
    if (scale_in == nullptr) K = 0;
    if (scale_out == nullptr) O = 0;
    if (K < 0 || O < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_permute_marlin_scales: negative size");
    if (K % 16 || O % 32)
        return fail(NQ_ERR_SHAPE, "nq_permute_marlin_scales: need K %% 16 == 0 and O %% 32 == 0");
    const int64_t n = K > O ? K : O;
    if (n == 0) return NQ_OK;
    permute_scales_kernel<<<grid_for(n), kThreads, 0, as_stream(stream)>>>(scale_in, scale_in_out, K, scale_out,
                                                                           scale_out_out, O);
    return check_launch("nq_permute_marlin_scales");
}

}  // extern "C"
