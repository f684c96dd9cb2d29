// Decode attention of one new token per sequence, with the rotary embedding and the KV-cache
// write fused in: the part of a Llama decode step between the q/k/v projections and o_proj.
//
// The positions 0..p of each (sequence, kv head) are split into chunks of 64; one block per
// (sequence, kv head, chunk), for every chunk the cache could hold, so the grid is fixed while
// the position p (read from device memory) advances under graph replay; blocks of chunks wholly
// after p exit once they have read it. A block:
//   1. rotates q (the G = heads / kv_heads query heads of its kv head) with the cos/sin row of
//      p, as the unfused path rounds it: (x * cos) and (rotate_half(x) * sin) each rounded to T,
//      then their sum; the block whose chunk holds p also rotates the new key and writes the key
//      and value into the cache at p (it reads them back from LDS, never from the cache);
//   2. scores s[g][j] = T(q_g . k_j) * scaling for its chunk's positions j <= p, four lanes per
//      position (32 dimensions each, summed with lane swaps);
//   3. per head: m = max_j s, e_j = exp(s_j - m), l = sum_j e_j (fp32);
//   4. o[g][d] = sum_j e_j v[j][d] (fp32; lane pairs of d, waves over j, values loaded ahead);
//   5. writes (m, l, o) to the workspace.
// A second launch (attn_combine_kernel, one block per sequence and kv head) combines the chunks:
// M = max m, L = sum l exp(m - M), out = T(sum o exp(m - M) / L). (Combining inside the first
// launch, by the last block to finish, needs device-scope fences, which write back the L2 of
// each XCD and cost more than the second launch.)
// Unlike the unfused path, probabilities are not rounded to T before the value product (the
// chunks' sums are combined first). The cache layout is [batch, kv_heads, max_len, head_dim]
// for K and V; head_dim 128.
#include <algorithm>

#include "nq_common.h"

namespace nq {
namespace {

constexpr int kHeadDim = 128;
constexpr int kAttnThreads = 256;
constexpr int kChunk = 64;  // positions per block

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

inline int64_t attn_chunks(int64_t max_len) { return ceil_div(max_len, kChunk); }
// floats of one chunk's partial result: (m, l) and o[128] per query head
inline int64_t attn_part_floats(int64_t g) { return g * (2 + kHeadDim); }

template <typename T, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int qkv_stride,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, const uint16_t* __restrict__ rope_cos,
    const uint16_t* __restrict__ rope_sin, const int64_t* __restrict__ position, uint16_t* __restrict__ out,
    int kv_heads, int max_len, float scaling, float* __restrict__ parts) {
    // every rounding below is meant: no product may be fused into a following add
#pragma clang fp contract(off)
    constexpr int D = kHeadDim;
    constexpr int NW = kAttnThreads / 64;
    constexpr int PF = G * (2 + D);
    __shared__ __attribute__((aligned(16))) uint16_t qs[G][D];
    __shared__ __attribute__((aligned(16))) uint16_t knew[D];
    __shared__ __attribute__((aligned(16))) uint16_t vnew[D];
    __shared__ float sc[G][kChunk];
    __shared__ float mls[G][2];
    __shared__ float red[NW][G][D];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n_chunks = (max_len + kChunk - 1) / kChunk;
    const int bh = blockIdx.x / n_chunks;  // sequence * kv_heads + kv head
    const int ch = blockIdx.x - bh * n_chunks;
    const int b = bh / kv_heads;
    const int kvh = bh - b * kv_heads;
    const int heads = kv_heads * G;
    uint16_t* orow = out + (static_cast<size_t>(b) * heads + static_cast<size_t>(kvh) * G) * D;
    const int lo = ch * kChunk;
    const size_t head_base = static_cast<size_t>(bh) * static_cast<size_t>(max_len) * D;
    const uint16_t* qrow = q + static_cast<size_t>(b) * qkv_stride + static_cast<size_t>(kvh) * G * D;
    const uint16_t* krow = k + static_cast<size_t>(b) * qkv_stride + static_cast<size_t>(kvh) * D;
    const uint16_t* vrow = v + static_cast<size_t>(b) * qkv_stride + static_cast<size_t>(kvh) * D;

    // 0. the projection elements the rotary step uses (element e of the G query heads, the key
    //    and the value, with its rotate-half partner), loaded together with the position
    constexpr int PW = kChunk / NW;
    constexpr int E = ((G + 2) * D + kAttnThreads - 1) / kAttnThreads;
    uint16_t xe[E], xp[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int e = min(t + i * kAttnThreads, (G + 2) * D - 1);
        const int hh = e / D;
        const int d = e - hh * D;
        const uint16_t* src = hh < G ? qrow + hh * D : (hh == G ? krow : vrow);
        xe[i] = src[d];
        xp[i] = src[d ^ (D / 2)];
    }
    const int64_t p64 = *position;
    __builtin_amdgcn_sched_barrier(0);
    if (p64 < 0 || p64 >= max_len) {  // a position outside the cache: zeros, nothing written
        if (ch == 0)
            for (int e = t; e < G * D; e += kAttnThreads) orow[e] = 0;
        return;
    }
    const int p = static_cast<int>(p64);
    if (lo > p) return;  // a chunk wholly after p: nothing to do, the combine skips it
    const int count = min(kChunk, p + 1 - lo);  // positions of this chunk that are visible
    const bool owner = p < lo + kChunk;

    // then every load that needs only p, issued before any result is used: this chunk's keys
    // (thread t: row lo + t / 4, dimensions 32 (t % 4) .. +31), values (lane pairs of d, PW rows per
    // wave; rows past p read row p, whose result is never used) and the cos/sin entries
    const int jj = t >> 2;
    const int part = t & 3;
    u32x4 kv4[4];
    {
        const uint16_t* kr = k_cache + head_base + static_cast<size_t>(min(lo + jj, p)) * D + 32 * part;
#pragma unroll
        for (int i = 0; i < 4; ++i) kv4[i] = *reinterpret_cast<const u32x4*>(kr + 8 * i);
    }
    uint32_t vv[PW];
#pragma unroll
    for (int u = 0; u < PW; ++u)
        vv[u] = *reinterpret_cast<const uint32_t*>(v_cache + head_base +
                                                   static_cast<size_t>(min(lo + wave + NW * u, p)) * D + 2 * lane);
    uint16_t cs[E], sn[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int e = min(t + i * kAttnThreads, (G + 2) * D - 1);
        const int d = e % D;
        cs[i] = rope_cos[static_cast<size_t>(p) * D + d];
        sn[i] = rope_sin[static_cast<size_t>(p) * D + d];
    }
    __builtin_amdgcn_sched_barrier(0);

    // 1. rotary embedding; the owner writes the new key and value
#pragma unroll
    for (int i = 0; i < E; ++i) {
        const int e = t + i * kAttnThreads;
        if (e < (G + 2) * D) {
            const int hh = e / D;
            const int d = e - hh * D;
            if (hh <= G) {  // G query heads, then the key
                const float x = T::to_float(xe[i]);
                const float xr = d < D / 2 ? -T::to_float(xp[i]) : T::to_float(xp[i]);
                const float a0 = T::to_float(T::from_float(x * T::to_float(cs[i])));
                const float a1 = T::to_float(T::from_float(xr * T::to_float(sn[i])));
                const uint16_t r = T::from_float(a0 + a1);
                if (hh < G) {
                    qs[hh][d] = r;
                } else if (owner) {
                    knew[d] = r;
                    k_cache[head_base + static_cast<size_t>(p) * D + d] = r;
                }
            } else if (owner) {
                vnew[d] = xe[i];
                v_cache[head_base + static_cast<size_t>(p) * D + d] = xe[i];
            }
        }
    }
    __syncthreads();

    // 2. scores: thread t takes position lo + t / 4, dimensions 32 * (t % 4) .. +31; the new
    //    position's key comes from LDS (its row in the prefetched cache is stale)
    if (owner && lo + jj == p) {
#pragma unroll
        for (int i = 0; i < 4; ++i) kv4[i] = *reinterpret_cast<const u32x4*>(&knew[32 * part + 8 * i]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 qv = *reinterpret_cast<const u32x4*>(&qs[g][32 * part + 8 * i]);
            a0 = T::dot2(qv.x, kv4[i].x, a0);
            a1 = T::dot2(qv.y, kv4[i].y, a1);
            a0 = T::dot2(qv.z, kv4[i].z, a0);
            a1 = T::dot2(qv.w, kv4[i].w, a1);
        }
        float sum = a0 + a1;
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        if (part == 0) sc[g][jj] = jj < count ? T::to_float(T::from_float(sum)) * scaling : -INFINITY;
    }
    __syncthreads();

    // 3. chunk softmax statistics, one wave per head
    for (int g = wave; g < G; g += NW) {
        const float s = sc[g][lane];
        const float m = wave_max(s);
        const float e = lane < count ? expf(s - m) : 0.0f;
        sc[g][lane] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            mls[g][0] = m;
            mls[g][1] = l;
        }
    }
    __syncthreads();

    // 4. o[g][d] = sum_j e_j v[j][d]: lane holds d = 2 lane, 2 lane + 1; wave w takes positions
    //    w, w + NW, ...
    {
        float acc[G][2];
#pragma unroll
        for (int g = 0; g < G; ++g) acc[g][0] = acc[g][1] = 0.0f;
        const uint32_t vl = *reinterpret_cast<const uint32_t*>(&vnew[2 * lane]);
#pragma unroll
        for (int u = 0; u < PW; ++u) {
            const int j = wave + NW * u;
            if (j < count) {
                const uint32_t w = (owner && lo + j == p) ? vl : vv[u];
                const float v0 = T::to_float(static_cast<uint16_t>(w & 0xFFFFu));
                const float v1 = T::to_float(static_cast<uint16_t>(w >> 16));
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float pj = sc[g][j];
                    acc[g][0] = fmaf(pj, v0, acc[g][0]);
                    acc[g][1] = fmaf(pj, v1, acc[g][1]);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            red[wave][g][2 * lane] = acc[g][0];
            red[wave][g][2 * lane + 1] = acc[g][1];
        }
    }
    __syncthreads();

    // 5. this chunk's partial result
    float* mypart = parts + (static_cast<size_t>(bh) * n_chunks + ch) * PF;
    for (int e = t; e < G * D; e += kAttnThreads) {
        const int g = e / D;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) s += red[w][g][e - g * D];
        mypart[2 * G + e] = s;
    }
    if (t < 2 * G) mypart[t] = mls[t >> 1][t & 1];
}

// Combine the chunks of one (sequence, kv head): thread e < G * 128 takes output element e.
template <typename T, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(const float* __restrict__ parts,
                                                                    const int64_t* __restrict__ position,
                                                                    uint16_t* __restrict__ out, int kv_heads,
                                                                    int max_len) {
    constexpr int D = kHeadDim;
    constexpr int PF = G * (2 + D);
    const int64_t p64 = *position;
    if (p64 < 0 || p64 >= max_len) return;  // the first launch wrote zeros
    const int n_chunks = (max_len + kChunk - 1) / kChunk;
    const int used = static_cast<int>(p64) / kChunk + 1;  // chunks holding positions <= p
    const int bh = blockIdx.x;
    const int b = bh / kv_heads;
    const int kvh = bh - b * kv_heads;
    uint16_t* orow = out + (static_cast<size_t>(b) * kv_heads * G + static_cast<size_t>(kvh) * G) * D;
    const float* hp = parts + static_cast<size_t>(bh) * n_chunks * PF;
    constexpr int R = 16;  // chunks whose partials are loaded together
    for (int e = threadIdx.x; e < G * D; e += kAttnThreads) {
        const int g = e / D;
        float M = -INFINITY, L = 0.0f, O = 0.0f;  // running combination
        for (int c0 = 0; c0 < used; c0 += R) {
            float m[R], l[R], o[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int c = min(c0 + i, used - 1);
                m[i] = hp[c * PF + 2 * g];
                l[i] = hp[c * PF + 2 * g + 1];
                o[i] = hp[c * PF + 2 * G + e];
            }
            float bm = M;
#pragma unroll
            for (int i = 0; i < R; ++i) bm = fmaxf(bm, m[i]);  // clamped entries repeat a used chunk
            const float scale = expf(M - bm);  // 0 on the first batch (M = -inf, bm finite)
            L *= scale;
            O *= scale;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                if (c0 + i < used) {
                    const float f = expf(m[i] - bm);
                    L = fmaf(l[i], f, L);
                    O = fmaf(o[i], f, O);
                }
            }
            M = bm;
        }
        orow[e] = T::from_float(O / L);
    }
}

// Rotary embedding and KV-cache write of one new token per sequence, for a decode step whose
// attention products run elsewhere: step 1 of attn_decode_kernel on its own. One thread per
// (sequence, head slot, dimension pair d < D/2) of the q, k and v heads of a [batch, qkv_stride]
// row: the query heads are rotated into q_out (which may be the q part of the same row: each
// thread reads and writes only its own pair), the key heads rotated into k_cache[b, kvh, p, :],
// the value heads copied into v_cache[b, kvh, p, :], with p read from device memory (so a graph
// replays it as the position advances). Rounded as the unfused path: T(x cos) and
// T(rotate_half(x) sin), then their sum to T. A position outside [0, max_len) writes zeros to
// q_out and nothing to the caches.
template <typename T>
__global__ __launch_bounds__(256) void rope_kv_kernel(const uint16_t* qkv, int qkv_stride, uint16_t* __restrict__ k_cache,
                                                      uint16_t* __restrict__ v_cache,
                                                      const uint16_t* __restrict__ rope_cos,
                                                      const uint16_t* __restrict__ rope_sin,
                                                      const int64_t* __restrict__ position, uint16_t* q_out,
                                                      int q_stride, int batch, int heads, int kv_heads, int head_dim,
                                                      int max_len) {
#pragma clang fp contract(off)
    const int half = head_dim / 2;
    const int slots = heads + 2 * kv_heads;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<int64_t>(batch) * slots * half) return;
    const int d = static_cast<int>(i % half);
    const int64_t bh = i / half;
    const int hs = static_cast<int>(bh % slots);
    const int b = static_cast<int>(bh / slots);
    const int64_t p64 = *position;
    const uint16_t* src = qkv + static_cast<size_t>(b) * qkv_stride + static_cast<size_t>(hs) * head_dim;
    uint16_t* qdst = q_out + static_cast<size_t>(b) * q_stride + static_cast<size_t>(hs) * head_dim;
    if (p64 < 0 || p64 >= max_len) {
        if (hs < heads) qdst[d] = qdst[d + half] = 0;
        return;
    }
    const size_t p = static_cast<size_t>(p64);
    const uint16_t x0 = src[d], x1 = src[d + half];
    if (hs >= heads + kv_heads) {  // a value head
        const size_t row = ((static_cast<size_t>(b) * kv_heads + (hs - heads - kv_heads)) * max_len + p) * head_dim;
        v_cache[row + d] = x0;
        v_cache[row + d + half] = x1;
        return;
    }
    const float c0 = T::to_float(rope_cos[p * head_dim + d]), c1 = T::to_float(rope_cos[p * head_dim + d + half]);
    const float s0 = T::to_float(rope_sin[p * head_dim + d]), s1 = T::to_float(rope_sin[p * head_dim + d + half]);
    const float f0 = T::to_float(x0), f1 = T::to_float(x1);
    // rotate_half: element d < D/2 takes -x[d + D/2], element d + D/2 takes x[d]
    const uint16_t r0 = T::from_float(T::to_float(T::from_float(f0 * c0)) + T::to_float(T::from_float(-f1 * s0)));
    const uint16_t r1 = T::from_float(T::to_float(T::from_float(f1 * c1)) + T::to_float(T::from_float(f0 * s1)));
    if (hs < heads) {
        qdst[d] = r0;
        qdst[d + half] = r1;
    } else {
        const size_t row = ((static_cast<size_t>(b) * kv_heads + (hs - heads)) * max_len + p) * head_dim;
        k_cache[row + d] = r0;
        k_cache[row + d + half] = r1;
    }
}

template <typename T, int G>
void launch_attn(const void* q, const void* k, const void* v, int64_t qkv_stride, void* k_cache, void* v_cache,
                 const void* rope_cos, const void* rope_sin, const int64_t* position, void* out, int64_t batch,
                 int64_t kv_heads, int64_t max_len, float scaling, float* parts, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(batch * kv_heads * attn_chunks(max_len)));
    attn_decode_kernel<T, G><<<grid, kAttnThreads, 0, st>>>(
        static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
        static_cast<int>(qkv_stride), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
        static_cast<const uint16_t*>(rope_cos), static_cast<const uint16_t*>(rope_sin), position,
        static_cast<uint16_t*>(out), static_cast<int>(kv_heads), static_cast<int>(max_len), scaling, parts);
    attn_combine_kernel<T, G><<<dim3(static_cast<unsigned>(batch * kv_heads)), kAttnThreads, 0, st>>>(
        parts, position, static_cast<uint16_t*>(out), static_cast<int>(kv_heads), static_cast<int>(max_len));
}

template <typename T>
bool launch_attn_g(int g, const void* q, const void* k, const void* v, int64_t qkv_stride, void* k_cache,
                   void* v_cache, const void* rope_cos, const void* rope_sin, const int64_t* position, void* out,
                   int64_t batch, int64_t kv_heads, int64_t max_len, float scaling, float* parts, hipStream_t st) {
#define NQ_ATTN(G_)                                                                                              \
    launch_attn<T, G_>(q, k, v, qkv_stride, k_cache, v_cache, rope_cos, rope_sin, position, out, batch, kv_heads, \
                       max_len, scaling, parts, st)
    switch (g) {
        case 1: NQ_ATTN(1); return true;
        case 2: NQ_ATTN(2); return true;
        case 4: NQ_ATTN(4); return true;
        case 8: NQ_ATTN(8); return true;
        default: return false;
    }
#undef NQ_ATTN
}

// ---- dense GEMV: the lm_head of a decode step
//
// y[b][j] = T(sum_k W[j][k] xn[b][k]) (fp32 sum, one rounding), W [m][n] row-major in T, where xn is
// x itself or, with a norm weight g, its RMS norm as the decoder's torch path rounds it:
// T(g[k] * T(x[k] * rsqrt(mean(x^2) + eps))) (mean and product in fp32). A decode step reaches its
// lm_head after its layers have streamed their weights through the caches, so W comes from HBM, and
// streaming it at speed takes many bytes in flight per CU: a wave takes RPW rows of W one after the
// other and issues every 16-byte load of a 4096-column group at once (8 per lane, non-temporal),
// the next group's (or next row's) before the current one's arithmetic; the first row's loads go
// out before the block stages its NB batch rows of x (or xn) in LDS, so their latency covers the
// staging, which serves the block's 4 RPW rows. Loads past the row's end read zeros (buffer resource
// bounds), so n need only be a multiple of 8. grid.y covers the batch.
constexpr int kDenseCols = 4096;      // columns of W a wave has in flight: 64 lanes x 8 x 8 elements
constexpr int kDenseLdsBytes = 64512;  // staged rows of x, NB * n * 2 bytes: within 64 KB with the static part

template <typename T, int NB, bool NORM, int RPW>
__global__ __launch_bounds__(256) void dense_gemv_kernel(const uint16_t* __restrict__ w, const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ norm_w, float eps,
                                                         void* __restrict__ y, int y_f32, int m, int n, int batch,
                                                         int ldy) {
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [NB][n]
    __shared__ float part[NB][4];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    // wave w of the block takes rows row0 + 4 rr (rr < RPW), one after the other, the next row's
    // loads in flight during the current row's arithmetic; every wave stages its share of x, so
    // none leaves early
    const int row0 = static_cast<int>(blockIdx.x) * 4 * RPW + wave;
    const int b0 = static_cast<int>(blockIdx.y) * NB;
    // the 8 loads of one 4096-column group of a row (rows past m read row m - 1 and store nothing)
    auto issue = [&](u32x4 (&dst)[8], int row, int c0) {
        const rsrc_t wr = make_rsrc(w + static_cast<size_t>(min(row, m - 1)) * static_cast<size_t>(n),
                                    static_cast<uint32_t>(n) * 2u);
#pragma unroll
        for (int k = 0; k < 8; ++k)
            dst[k] = load_b128_stream(wr, static_cast<uint32_t>(c0 + (k * 64 + lane) * 8) * 2u);
    };
    u32x4 wv[8], wq[8];
    issue(wv, row0, 0);

    // x's batch rows into LDS (16-byte chunks; every thread keeps to its own chunks throughout)
    const int chunks = n / 8;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint16_t* xr = x + static_cast<size_t>(min(b0 + b, batch - 1)) * static_cast<size_t>(n);
        float ss = 0.0f;
        for (int c = t; c < chunks; c += 256) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(xr + c * 8);
            *reinterpret_cast<u32x4*>(xs + b * n + c * 8) = v;
            if (NORM) {
                const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float lo = T::to_float(static_cast<uint16_t>(d[q] & 0xFFFFu));
                    const float hi = T::to_float(static_cast<uint16_t>(d[q] >> 16));
                    ss += lo * lo;
                    ss += hi * hi;
                }
            }
        }
        if (NORM) {
            ss = wave_sum(ss);
            if (lane == 0) part[b][wave] = ss;
        }
    }
    if (NORM) {
        __syncthreads();
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float r = rsqrtf((part[b][0] + part[b][1] + part[b][2] + part[b][3]) / static_cast<float>(n) + eps);
            for (int c = t; c < chunks; c += 256) {
                u32x4 v = *reinterpret_cast<const u32x4*>(xs + b * n + c * 8);
                const u32x4 g = *reinterpret_cast<const u32x4*>(norm_w + c * 8);
                uint32_t d[4] = {v.x, v.y, v.z, v.w};
                const uint32_t gd[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint16_t h[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const uint16_t xe = static_cast<uint16_t>(d[q] >> (16 * e));
                        const uint16_t ge = static_cast<uint16_t>(gd[q] >> (16 * e));
                        const float xn = T::to_float(T::from_float(T::to_float(xe) * r));
                        h[e] = T::from_float(T::to_float(ge) * xn);
                    }
                    d[q] = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
                }
                v = u32x4{d[0], d[1], d[2], d[3]};
                *reinterpret_cast<u32x4*>(xs + b * n + c * 8) = v;
            }
        }
    }
    __syncthreads();

#pragma unroll 1
    for (int rr = 0; rr < RPW; ++rr) {
        const int row = row0 + 4 * rr;
        float acc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
        for (int c0 = 0; c0 < n; c0 += kDenseCols) {
            // the next group's loads go out before this group's arithmetic: the rest of this row,
            // else the start of the wave's next row
            const bool next_group = c0 + kDenseCols < n;
            const bool next_row = !next_group && rr + 1 < RPW;
            if (next_group) issue(wq, row, c0 + kDenseCols);
            else if (next_row) issue(wq, row + 4, 0);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int col = c0 + (k * 64 + lane) * 8;
                    const u32x4 xv =
                        col < n ? *reinterpret_cast<const u32x4*>(xs + b * n + col) : u32x4{0u, 0u, 0u, 0u};
                    acc[b] = T::dot2(wv[k].x, xv.x, acc[b]);
                    acc[b] = T::dot2(wv[k].y, xv.y, acc[b]);
                    acc[b] = T::dot2(wv[k].z, xv.z, acc[b]);
                    acc[b] = T::dot2(wv[k].w, xv.w, acc[b]);
                }
            }
            if (next_group || next_row) {
#pragma unroll
                for (int k = 0; k < 8; ++k) wv[k] = wq[k];
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float s = wave_sum(acc[b]);
            if (lane == 0 && row < m && b0 + b < batch) {
                const uint16_t v = T::from_float(s);
                const size_t at = static_cast<size_t>(b0 + b) * static_cast<size_t>(ldy) + static_cast<size_t>(row);
                if (y_f32) static_cast<float*>(y)[at] = T::to_float(v);
                else static_cast<uint16_t*>(y)[at] = v;
            }
        }
    }
}

// Batch rows per block: up to 4, as many as the batch has, as fit the staging LDS.
inline int dense_rows_per_block(int64_t batch, int64_t n) {
    int nb = batch >= 4 ? 4 : (batch >= 2 ? 2 : 1);
    while (nb > 1 && static_cast<int64_t>(nb) * n * 2 > kDenseLdsBytes) nb /= 2;
    return nb;
}

// Rows of W per wave (each block stages x's batch rows once for 4 RPW rows of W). Same-box A/B on the
// Llama-2-7B lm_head (32000 x 4096 fp16, norm prologue, float32 out, 3 rotating weight copies; us at
// batch 1 / 2 / 4 / 8): one row per wave, every block staging x for its 4 rows, 44.5 / 60.4 / 133.6 /
// 260.1; 4 rows 43.5 / 50.2 / 76.3 / 148.1; 8 rows 43.9 / 52.3 / 62.7 / 123.4. Taking a wave's rows
// at once instead (each x chunk read from LDS feeding them all, no next-row prefetch) measured
// slower: 4 rows 46.5 / 54.9 / 108.5 / 207.1.
inline int dense_rows_per_wave(int64_t batch) { return batch >= 3 ? 8 : 4; }

template <typename T, bool NORM, int NB>
void launch_dense_rpw(int rpw, const uint16_t* w, const uint16_t* x, const uint16_t* g, float eps, void* y, int y_f32,
                      int m, int n, int batch, int ldy, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(ceil_div(m, 4 * rpw)), static_cast<unsigned>(ceil_div(batch, NB)));
    const size_t lds = static_cast<size_t>(NB) * n * 2;
    if (rpw == 8) dense_gemv_kernel<T, NB, NORM, 8><<<grid, 256, lds, st>>>(w, x, g, eps, y, y_f32, m, n, batch, ldy);
    else if (rpw == 4) dense_gemv_kernel<T, NB, NORM, 4><<<grid, 256, lds, st>>>(w, x, g, eps, y, y_f32, m, n, batch, ldy);
    else if (rpw == 2) dense_gemv_kernel<T, NB, NORM, 2><<<grid, 256, lds, st>>>(w, x, g, eps, y, y_f32, m, n, batch, ldy);
    else dense_gemv_kernel<T, NB, NORM, 1><<<grid, 256, lds, st>>>(w, x, g, eps, y, y_f32, m, n, batch, ldy);
}

template <typename T, bool NORM>
void launch_dense_gemv(const uint16_t* w, const uint16_t* x, const uint16_t* g, float eps, void* y, int y_f32, int m,
                       int n, int batch, int ldy, hipStream_t st) {
    const int nb = dense_rows_per_block(batch, n);
    const int rpw = dense_rows_per_wave(batch);
    if (nb == 4) launch_dense_rpw<T, NORM, 4>(rpw, w, x, g, eps, y, y_f32, m, n, batch, ldy, st);
    else if (nb == 2) launch_dense_rpw<T, NORM, 2>(rpw, w, x, g, eps, y, y_f32, m, n, batch, ldy, st);
    else launch_dense_rpw<T, NORM, 1>(rpw, w, x, g, eps, y, y_f32, m, n, batch, ldy, st);
}

// ------------------------------------------------------------------ greedy argmax over the logits
//
// One block per batch row: each thread scans every kArgmaxThreads-th logit, then the wave and the
// block reduce (value, index) pairs. The order is torch.argmax's: a NaN beats every number (the
// first NaN wins), otherwise the larger value, and of equal values (-0 equal to +0) the smaller
// index, so the result is the first maximal logit. One 32000-logit row: 8.4 us graph-replayed
// against 10.5 us for torch.argmax (a variant issuing each thread's 32 loads at once took 9.0).
constexpr int kArgmaxThreads = 1024;

__device__ inline bool argmax_before(float a, int ia, float b, int ib) {
    const bool na = a != a, nb = b != b;
    if (na || nb) return na && (!nb || ia < ib);
    return a > b || (a == b && ia < ib);
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const float* __restrict__ x, int n, int64_t ldx,
                                                                     int64_t* __restrict__ out) {
    const float* row = x + static_cast<int64_t>(blockIdx.x) * ldx;
    float bv = -INFINITY;
    int bi = INT32_MAX;  // loses to every element, a -inf one included (equal value, smaller index)
#pragma unroll 8
    for (int i = static_cast<int>(threadIdx.x); i < n; i += kArgmaxThreads) {
        const float v = row[i];
        if (argmax_before(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (argmax_before(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    __shared__ float wv[kArgmaxThreads / 64];
    __shared__ int wi[kArgmaxThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        wv[wave] = bv;
        wi[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w)
            if (argmax_before(wv[w], wi[w], bv, bi)) {
                bv = wv[w];
                bi = wi[w];
            }
        out[blockIdx.x] = bi;
    }
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" {

size_t nq_attention_decode_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads, int64_t head_dim,
                                           int64_t max_len) {
    if (batch < 0 || heads <= 0 || kv_heads <= 0 || max_len <= 0 || head_dim != kHeadDim || heads % kv_heads)
        return 0;
    const int64_t g = heads / kv_heads;
    return static_cast<size_t>(batch * kv_heads * attn_chunks(max_len) * attn_part_floats(g)) * sizeof(float);
}

int nq_attention_decode(int dtype, const void* q, const void* k, const void* v, int64_t qkv_stride, void* k_cache,
                        void* v_cache, const void* rope_cos, const void* rope_sin, const int64_t* position, void* out,
                        int64_t batch, int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t max_len,
                        float scaling, void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    const char* name = "nq_attention_decode";
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "%s: unsupported dtype %d", name, dtype);
    if (batch < 0 || heads <= 0 || kv_heads <= 0 || max_len <= 0 || head_dim <= 0)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: bad sizes", name);
    if (head_dim != kHeadDim) return fail(NQ_ERR_UNSUPPORTED, "%s: head_dim must be %d", name, kHeadDim);
    if (heads % kv_heads) return fail(NQ_ERR_SHAPE, "%s: heads must be a multiple of kv_heads", name);
    const int64_t g = heads / kv_heads;
    if (g != 1 && g != 2 && g != 4 && g != 8)
        return fail(NQ_ERR_UNSUPPORTED, "%s: heads / kv_heads must be 1, 2, 4 or 8", name);
    if (qkv_stride < heads * head_dim)
        return fail(NQ_ERR_SHAPE, "%s: qkv_stride %lld too small", name, (long long)qkv_stride);
    if (batch * kv_heads * attn_chunks(max_len) > INT32_MAX / 2 || max_len > INT32_MAX / 2 ||
        batch * kv_heads * max_len * head_dim > ((int64_t)1 << 40) || batch * qkv_stride > INT32_MAX / 2)
        return fail(NQ_ERR_UNSUPPORTED, "%s: sizes too large", name);
    if (batch == 0) return NQ_OK;
    if (!q || !k || !v || !k_cache || !v_cache || !rope_cos || !rope_sin || !position || !out || !workspace)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(q, 2) || !aligned(k, 2) || !aligned(v, 2) ||
        !aligned(out, 2) || !aligned(rope_cos, 2) || !aligned(rope_sin, 2) || !aligned(position, 8) ||
        !aligned(workspace, 256))
        return fail(NQ_ERR_ALIGNMENT, "%s: misaligned operand (the caches need 16 bytes, the workspace 256)", name);
    const size_t need = nq_attention_decode_workspace_bytes(batch, heads, kv_heads, head_dim, max_len);
    if (workspace_bytes < need)
        return fail(NQ_ERR_WORKSPACE, "%s: workspace has %zu bytes, needs %zu", name, workspace_bytes, need);
    float* parts = static_cast<float*>(workspace);
    hipStream_t st = as_stream(stream);
    const bool ok = dtype == NQ_F16 ? launch_attn_g<F16>(static_cast<int>(g), q, k, v, qkv_stride, k_cache, v_cache,
                                                         rope_cos, rope_sin, position, out, batch, kv_heads, max_len,
                                                         scaling, parts, st)
                                    : launch_attn_g<BF16>(static_cast<int>(g), q, k, v, qkv_stride, k_cache, v_cache,
                                                          rope_cos, rope_sin, position, out, batch, kv_heads, max_len,
                                                          scaling, parts, st);
    if (!ok) return fail(NQ_ERR_UNSUPPORTED, "%s: no kernel for this head grouping", name);
    return check_launch(name);
}

int nq_rope_kv_write(int dtype, const void* qkv, int64_t qkv_stride, void* k_cache, void* v_cache,
                     const void* rope_cos, const void* rope_sin, const int64_t* position, void* q_out,
                     int64_t q_stride, int64_t batch, int64_t heads, int64_t kv_heads, int64_t head_dim,
                     int64_t max_len, nq_stream_t stream) {
    const char* name = "nq_rope_kv_write";
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "%s: unsupported dtype %d", name, dtype);
    if (batch < 0 || heads <= 0 || kv_heads <= 0 || max_len <= 0 || head_dim <= 0 || head_dim % 2)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: bad sizes (head_dim must be even)", name);
    if (qkv_stride < (heads + 2 * kv_heads) * head_dim || q_stride < heads * head_dim)
        return fail(NQ_ERR_SHAPE, "%s: row strides too small", name);
    if (batch * qkv_stride > INT32_MAX / 2 || batch * q_stride > INT32_MAX / 2 || max_len > INT32_MAX / 2 ||
        batch * kv_heads * max_len * head_dim > ((int64_t)1 << 40) || batch * (heads + 2 * kv_heads) * head_dim > INT32_MAX / 2)
        return fail(NQ_ERR_UNSUPPORTED, "%s: sizes too large", name);
    if (batch == 0) return NQ_OK;
    if (!qkv || !k_cache || !v_cache || !rope_cos || !rope_sin || !position || !q_out)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(qkv, 2) || !aligned(k_cache, 2) || !aligned(v_cache, 2) || !aligned(rope_cos, 2) ||
        !aligned(rope_sin, 2) || !aligned(position, 8) || !aligned(q_out, 2))
        return fail(NQ_ERR_ALIGNMENT, "%s: misaligned operand", name);
    const int64_t threads = batch * (heads + 2 * kv_heads) * (head_dim / 2);
    const dim3 grid(static_cast<unsigned>(ceil_div(threads, 256)));
    hipStream_t st = as_stream(stream);
    const auto* a = static_cast<const uint16_t*>(qkv);
    auto* kc = static_cast<uint16_t*>(k_cache);
    auto* vc = static_cast<uint16_t*>(v_cache);
    const auto* cs = static_cast<const uint16_t*>(rope_cos);
    const auto* sn = static_cast<const uint16_t*>(rope_sin);
    auto* qo = static_cast<uint16_t*>(q_out);
    if (dtype == NQ_F16)
        rope_kv_kernel<F16><<<grid, 256, 0, st>>>(a, static_cast<int>(qkv_stride), kc, vc, cs, sn, position, qo,
                                                  static_cast<int>(q_stride), static_cast<int>(batch),
                                                  static_cast<int>(heads), static_cast<int>(kv_heads),
                                                  static_cast<int>(head_dim), static_cast<int>(max_len));
    else
        rope_kv_kernel<BF16><<<grid, 256, 0, st>>>(a, static_cast<int>(qkv_stride), kc, vc, cs, sn, position, qo,
                                                   static_cast<int>(q_stride), static_cast<int>(batch),
                                                   static_cast<int>(heads), static_cast<int>(kv_heads),
                                                   static_cast<int>(head_dim), static_cast<int>(max_len));
    return check_launch(name);
}

int nq_dense_gemv(int dtype, const void* w, const void* x, const void* norm_weight, float eps, void* y,
                  int y_float32, int64_t batch, int64_t n, int64_t m, int64_t ldy, nq_stream_t stream) {
    const char* name = "nq_dense_gemv";
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "%s: unsupported dtype %d", name, dtype);
    if (batch < 0 || n <= 0 || m <= 0 || ldy < m)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: bad sizes (batch %lld, n %lld, m %lld, ldy %lld)", name,
                    (long long)batch, (long long)n, (long long)m, (long long)ldy);
    if (n % 8) return fail(NQ_ERR_SHAPE, "%s: n must be a multiple of 8, got %lld", name, (long long)n);
    if (n * 2 > kDenseLdsBytes || m > INT32_MAX / 2 || ldy > INT32_MAX / 2 || batch > 65535 ||
        batch * ldy > (int64_t{1} << 40))
        return fail(NQ_ERR_UNSUPPORTED, "%s: sizes too large (n at most %d)", name, kDenseLdsBytes / 2);
    if (batch == 0) return NQ_OK;
    if (!w || !x || !y) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(w, 16) || !aligned(x, 16) || (norm_weight && !aligned(norm_weight, 16)) ||
        !aligned(y, y_float32 ? 4 : 2))
        return fail(NQ_ERR_ALIGNMENT, "%s: w, x and norm_weight must be 16-byte aligned, y aligned to its type",
                    name);
    const auto* wp = static_cast<const uint16_t*>(w);
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* gp = static_cast<const uint16_t*>(norm_weight);
    const int yf = y_float32 ? 1 : 0;
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), bi = static_cast<int>(batch);
    const int li = static_cast<int>(ldy);
    hipStream_t st = as_stream(stream);
    if (dtype == NQ_F16) {
        if (gp) launch_dense_gemv<F16, true>(wp, xp, gp, eps, y, yf, mi, ni, bi, li, st);
        else launch_dense_gemv<F16, false>(wp, xp, gp, eps, y, yf, mi, ni, bi, li, st);
    } else {
        if (gp) launch_dense_gemv<BF16, true>(wp, xp, gp, eps, y, yf, mi, ni, bi, li, st);
        else launch_dense_gemv<BF16, false>(wp, xp, gp, eps, y, yf, mi, ni, bi, li, st);
    }
    return check_launch(name);
}

int nq_argmax_rows(const float* x, int64_t rows, int64_t n, int64_t ldx, int64_t* out, nq_stream_t stream) {
    const char* name = "nq_argmax_rows";
    if (rows < 0 || n <= 0 || ldx < n)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: bad sizes (rows %lld, n %lld, ldx %lld)", name, (long long)rows,
                    (long long)n, (long long)ldx);
    if (n > INT32_MAX / 2 || rows > 65535 * 32) return fail(NQ_ERR_UNSUPPORTED, "%s: sizes too large", name);
    if (rows == 0) return NQ_OK;
    if (!x || !out) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(x, 4) || !aligned(out, 8)) return fail(NQ_ERR_ALIGNMENT, "%s: misaligned x or out", name);
    argmax_rows_kernel<<<static_cast<unsigned>(rows), kArgmaxThreads, 0, as_stream(stream)>>>(
        x, static_cast<int>(n), ldx, out);
    return check_launch(name);
}

}  // extern "C"
