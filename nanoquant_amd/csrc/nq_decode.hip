// Decode attention of one new token per sequence, with the rotary embedding and the KV-cache
// write fused in: the part of a Llama decode step between the q/k/v projections and o_proj.
//
// One block per (sequence b, kv head); it serves the G = heads / kv_heads query heads that
// share the kv head. The position p of the new token is read from device memory, so the
// launch can be replayed from a graph while the position advances.
//   1. rotate q (G heads) and the new k with the cos/sin rows of p, as the unfused path rounds
//      it: (x * cos) and (rotate_half(x) * sin) each rounded to T, then their sum; write k and
//      v into the cache at p;
//   2. scores s[g][j] = T(q_g . k_j) * scaling for j <= p, one position per thread (a lane
//      holds the key row in registers and runs the G heads over it; 512 threads, so up to
//      512 keys are in flight at once);
//   3. softmax over j in fp32, probabilities rounded to T;
//   4. out[g][d] = T(sum_j p[g][j] * v[j][d]) in fp32: lane pairs of d, waves over j, the
//      values of 32 positions per wave in flight at once.
// The cache layout is [batch, kv_heads, max_len, head_dim] for both K and V; head_dim 128.
// Row p of the caches is only written here: the block reads the new key and value back from
// LDS, never from the cache it has just written.
#include <algorithm>

#include "nq_common.h"

namespace nq {
namespace {

constexpr int kHeadDim = 128;
constexpr int kAttnThreads = 512;
constexpr int kPvChunk = 32;  // positions whose values a wave loads before using them
constexpr size_t kAttnLdsBudget = 64 * 1024;

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Block-wide max or sum of one value per thread (every thread gets the result).
template <bool kMax>
__device__ inline float block_reduce(float v, float* buf) {
    v = kMax ? wave_max(v) : wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) buf[wave] = v;
    __syncthreads();
    float r = buf[0];
#pragma unroll
    for (int w = 1; w < kAttnThreads / 64; ++w) r = kMax ? fmaxf(r, buf[w]) : r + buf[w];
    __syncthreads();
    return r;
}

template <typename T, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int qkv_stride,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, const uint16_t* __restrict__ rope_cos,
    const uint16_t* __restrict__ rope_sin, const int64_t* __restrict__ position, uint16_t* __restrict__ out,
    int kv_heads, int max_len, float scaling) {
    // every rounding below is meant: no product may be fused into a following add
#pragma clang fp contract(off)
    constexpr int D = kHeadDim;
    constexpr int NW = kAttnThreads / 64;
    // [G][max_len]: scores, then probabilities; afterwards the waves' partial outputs
    // [NW][G][D] (the host sizes it for the larger of the two)
    extern __shared__ float sc[];
    __shared__ __attribute__((aligned(16))) uint16_t qs[G][D];
    __shared__ __attribute__((aligned(16))) uint16_t knew[D];  // the new key and value, read
    __shared__ __attribute__((aligned(16))) uint16_t vnew[D];  // back from here, not the cache
    __shared__ float rbuf[NW];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int b = blockIdx.x / kv_heads;
    const int kvh = blockIdx.x - b * kv_heads;
    const int heads = kv_heads * G;
    uint16_t* orow = out + (static_cast<size_t>(b) * heads + static_cast<size_t>(kvh) * G) * D;
    const int64_t p64 = *position;
    if (p64 < 0 || p64 >= max_len) {  // a position outside the cache: zeros, nothing written
        for (int e = t; e < G * D; e += kAttnThreads) orow[e] = 0;
        return;
    }
    const int p = static_cast<int>(p64);
    const size_t head_base = (static_cast<size_t>(b) * kv_heads + kvh) * static_cast<size_t>(max_len) * D;

    // 1. rotary embedding, cache write
    const uint16_t* qrow = q + static_cast<size_t>(b) * qkv_stride + static_cast<size_t>(kvh) * G * D;
    const uint16_t* krow = k + static_cast<size_t>(b) * qkv_stride + static_cast<size_t>(kvh) * D;
    const uint16_t* vrow = v + static_cast<size_t>(b) * qkv_stride + static_cast<size_t>(kvh) * D;
    for (int e = t; e < (G + 2) * D; e += kAttnThreads) {
        const int hh = e / D;
        const int d = e - hh * D;
        if (hh <= G) {  // G query heads, then the key
            const uint16_t* src = hh < G ? qrow + hh * D : krow;
            const float x = T::to_float(src[d]);
            const float xr = d < D / 2 ? -T::to_float(src[d + D / 2]) : T::to_float(src[d - D / 2]);
            const float c = T::to_float(rope_cos[static_cast<size_t>(p) * D + d]);
            const float s = T::to_float(rope_sin[static_cast<size_t>(p) * D + d]);
            const float a0 = T::to_float(T::from_float(x * c));
            const float a1 = T::to_float(T::from_float(xr * s));
            const uint16_t r = T::from_float(a0 + a1);
            if (hh < G) {
                qs[hh][d] = r;
            } else {
                knew[d] = r;
                k_cache[head_base + static_cast<size_t>(p) * D + d] = r;
            }
        } else {
            const uint16_t vd = vrow[d];
            vnew[d] = vd;
            v_cache[head_base + static_cast<size_t>(p) * D + d] = vd;
        }
    }
    __syncthreads();

    // 2. scores
    const uint16_t* kb = k_cache + head_base;
    for (int j = t; j <= p; j += kAttnThreads) {
        u32x4 kr[D / 8];
#pragma unroll
        for (int i = 0; i < D / 8; ++i) kr[i] = *reinterpret_cast<const u32x4*>(kb + static_cast<size_t>(j) * D + 8 * i);
        if (j == p) {
#pragma unroll
            for (int i = 0; i < D / 8; ++i) kr[i] = *reinterpret_cast<const u32x4*>(&knew[8 * i]);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            // the query comes from LDS head by head (broadcast reads); without this the compiler
            // keeps all G heads in registers across the loop and spills from G = 2 on
            asm volatile("" ::: "memory");
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int i = 0; i < D / 8; ++i) {
                const u32x4 qv = *reinterpret_cast<const u32x4*>(&qs[g][8 * i]);
                a0 = T::dot2(qv.x, kr[i].x, a0);
                a1 = T::dot2(qv.y, kr[i].y, a1);
                a0 = T::dot2(qv.z, kr[i].z, a0);
                a1 = T::dot2(qv.w, kr[i].w, a1);
            }
            sc[g * max_len + j] = T::to_float(T::from_float(a0 + a1)) * scaling;
        }
    }
    __syncthreads();

    // 3. softmax over positions 0..p, per head
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float* row = sc + g * max_len;
        float mx = -INFINITY;
        for (int j = t; j <= p; j += kAttnThreads) mx = fmaxf(mx, row[j]);
        mx = block_reduce<true>(mx, rbuf);
        float sum = 0.0f;
        for (int j = t; j <= p; j += kAttnThreads) {
            const float e = expf(row[j] - mx);
            row[j] = e;
            sum += e;
        }
        sum = block_reduce<false>(sum, rbuf);
        for (int j = t; j <= p; j += kAttnThreads) row[j] = T::to_float(T::from_float(row[j] / sum));
    }
    __syncthreads();

    // 4. probabilities times values: lane holds d = 2 lane, 2 lane + 1; wave w takes positions
    //    w, w + NW, ...; each round loads kPvChunk positions' values (clamped addresses, so the
    //    loads are unconditional) before the first multiply-add
    float acc[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.0f;
    const uint16_t* vb = v_cache + head_base + 2 * lane;
    const uint32_t vl = *reinterpret_cast<const uint32_t*>(&vnew[2 * lane]);
    for (int j0 = wave; j0 <= p; j0 += NW * kPvChunk) {
        uint32_t vv[kPvChunk];
#pragma unroll
        for (int u = 0; u < kPvChunk; ++u)
            vv[u] = *reinterpret_cast<const uint32_t*>(vb + static_cast<size_t>(min(j0 + NW * u, p)) * D);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kPvChunk; ++u) {
            const int j = j0 + NW * u;
            if (j <= p) {
                const uint32_t w = j == p ? vl : vv[u];
                const float v0 = T::to_float(static_cast<uint16_t>(w & 0xFFFFu));
                const float v1 = T::to_float(static_cast<uint16_t>(w >> 16));
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float pj = sc[g * max_len + j];
                    acc[g][0] = fmaf(pj, v0, acc[g][0]);
                    acc[g][1] = fmaf(pj, v1, acc[g][1]);
                }
            }
        }
    }
    __syncthreads();  // every wave is done with the probabilities
    float* part = sc;  // [NW][G][D]
#pragma unroll
    for (int g = 0; g < G; ++g) {
        part[(wave * G + g) * D + 2 * lane] = acc[g][0];
        part[(wave * G + g) * D + 2 * lane + 1] = acc[g][1];
    }
    __syncthreads();
    for (int e = t; e < G * D; e += kAttnThreads) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) s += part[w * G * D + e];
        orow[e] = T::from_float(s);
    }
}

template <typename T, int G>
void launch_attn(const void* q, const void* k, const void* v, int64_t qkv_stride, void* k_cache, void* v_cache,
                 const void* rope_cos, const void* rope_sin, const int64_t* position, void* out, int64_t batch,
                 int64_t kv_heads, int64_t max_len, float scaling, size_t lds, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(batch * kv_heads));
    attn_decode_kernel<T, G><<<grid, kAttnThreads, lds, st>>>(
        static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
        static_cast<int>(qkv_stride), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
        static_cast<const uint16_t*>(rope_cos), static_cast<const uint16_t*>(rope_sin), position,
        static_cast<uint16_t*>(out), static_cast<int>(kv_heads), static_cast<int>(max_len), scaling);
}

template <typename T>
bool launch_attn_g(int g, const void* q, const void* k, const void* v, int64_t qkv_stride, void* k_cache,
                   void* v_cache, const void* rope_cos, const void* rope_sin, const int64_t* position, void* out,
                   int64_t batch, int64_t kv_heads, int64_t max_len, float scaling, size_t lds, hipStream_t st) {
    switch (g) {
        case 1: launch_attn<T, 1>(q, k, v, qkv_stride, k_cache, v_cache, rope_cos, rope_sin, position, out, batch, kv_heads, max_len, scaling, lds, st); return true;
        case 2: launch_attn<T, 2>(q, k, v, qkv_stride, k_cache, v_cache, rope_cos, rope_sin, position, out, batch, kv_heads, max_len, scaling, lds, st); return true;
        case 4: launch_attn<T, 4>(q, k, v, qkv_stride, k_cache, v_cache, rope_cos, rope_sin, position, out, batch, kv_heads, max_len, scaling, lds, st); return true;
        case 8: launch_attn<T, 8>(q, k, v, qkv_stride, k_cache, v_cache, rope_cos, rope_sin, position, out, batch, kv_heads, max_len, scaling, lds, st); return true;
        default: return false;
    }
}

// LDS of attn_decode_kernel<G>: static (queries, new key and value, reduction slots) and
// dynamic (score rows, reused for the waves' partial outputs).
inline size_t attn_static_lds(int64_t g) { return static_cast<size_t>(g) * kHeadDim * 2 + 4 * kHeadDim + 64; }
inline size_t attn_dynamic_lds(int64_t g, int64_t max_len) {
    return static_cast<size_t>(std::max<int64_t>(g * max_len, (kAttnThreads / 64) * g * kHeadDim)) * sizeof(float);
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" {

int nq_attention_decode(int dtype, const void* q, const void* k, const void* v, int64_t qkv_stride, void* k_cache,
                        void* v_cache, const void* rope_cos, const void* rope_sin, const int64_t* position, void* out,
                        int64_t batch, int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t max_len,
                        float scaling, nq_stream_t stream) {
    const char* name = "nq_attention_decode";
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "%s: unsupported dtype %d", name, dtype);
    if (batch < 0 || heads <= 0 || kv_heads <= 0 || max_len <= 0 || head_dim <= 0)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: bad sizes", name);
    if (head_dim != kHeadDim) return fail(NQ_ERR_UNSUPPORTED, "%s: head_dim must be %d", name, kHeadDim);
    if (heads % kv_heads) return fail(NQ_ERR_SHAPE, "%s: heads must be a multiple of kv_heads", name);
    const int64_t g = heads / kv_heads;
    if (g != 1 && g != 2 && g != 4 && g != 8)
        return fail(NQ_ERR_UNSUPPORTED, "%s: heads / kv_heads must be 1, 2, 4 or 8", name);
    const size_t lds = attn_dynamic_lds(g, max_len);
    if (lds + attn_static_lds(g) > kAttnLdsBudget)
        return fail(NQ_ERR_UNSUPPORTED, "%s: max_len %lld too long for (heads / kv_heads) = %lld", name,
                    (long long)max_len, (long long)g);
    if (qkv_stride < heads * head_dim)
        return fail(NQ_ERR_SHAPE, "%s: qkv_stride %lld too small", name, (long long)qkv_stride);
    if (batch * kv_heads > INT32_MAX / 2 || batch * kv_heads * max_len * head_dim > ((int64_t)1 << 40) ||
        batch * qkv_stride > INT32_MAX / 2)
        return fail(NQ_ERR_UNSUPPORTED, "%s: sizes too large", name);
    if (batch == 0) return NQ_OK;
    if (!q || !k || !v || !k_cache || !v_cache || !rope_cos || !rope_sin || !position || !out)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(q, 2) || !aligned(k, 2) || !aligned(v, 2) ||
        !aligned(out, 2) || !aligned(rope_cos, 2) || !aligned(rope_sin, 2) || !aligned(position, 8))
        return fail(NQ_ERR_ALIGNMENT, "%s: misaligned operand (the caches need 16 bytes)", name);
    hipStream_t st = as_stream(stream);
    const bool ok = dtype == NQ_F16 ? launch_attn_g<F16>(static_cast<int>(g), q, k, v, qkv_stride, k_cache, v_cache,
                                                         rope_cos, rope_sin, position, out, batch, kv_heads, max_len,
                                                         scaling, lds, st)
                                    : launch_attn_g<BF16>(static_cast<int>(g), q, k, v, qkv_stride, k_cache, v_cache,
                                                          rope_cos, rope_sin, position, out, batch, kv_heads, max_len,
                                                          scaling, lds, st);
    if (!ok) return fail(NQ_ERR_UNSUPPORTED, "%s: no kernel for this head grouping", name);
    return check_launch(name);
}

}  // extern "C"
