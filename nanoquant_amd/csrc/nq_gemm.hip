// Prefill GEMM on the Marlin sign layout: C[M, N] = sat((A[M, K] * W) * s_out) with
// W[k, o] = sign(k, o) * s_in[k], on gfx950 MFMA (v_mfma_f32_16x16x32_{f16,bf16}).
//
// Marlin word (tr, col) of the [K/16, N/2] array holds o = 64*(col/32) + 16*o16 + 8*o8 + o1
// (o1 = (col%32)/4) by k = 16*tr + 8*r8 + 2*r2 + r1 (r2 = col%4), element at bit
// 15 - (2*o8 + r8) + 16*r1 - 4*o16. Shifting a word left by 2*o8 + r8 + 4*o16 puts the
// signs of (k, k+1) at bits 15 and 31: exactly the sign bits of a packed 16-bit pair.
// The B fragment of one MFMA lane is therefore two adjacent words (r2 = 2g', 2g'+1 of
// its column o) turned into four (+-s_in[k], +-s_in[k+1]) pairs with one shift, one
// and, one xor each; no +-1 matrix is ever materialised.
//
// K-slot order: the 32 k of one MFMA step are split over the 4 lane groups g = 2t + g'
// (t = tile_red of the step, g' = pair of r2 values) and inside a lane over dwords
// d = (r8 = d>>1, r2 = 2g' + (d&1)). A and B use the same order, so the product is the
// plain sum over k. The A fragment of a lane is then k = 16t + 4g' + {0..3} and
// 16t + 8 + 4g' + {0..3}: two 8-byte LDS reads.
//
// Block tile 128 x 128, 4 waves (2 x 2), wave tile 64 x 64 = 4 x 4 MFMA tiles, K step 32.
#include "nq_common.h"

namespace nq {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 32;
constexpr int LDA = BK + 8;  // LDS row stride in 16-bit elements (80 bytes)
constexpr int kThreads = 256;

template <typename T>
struct Mfma;

template <>
struct Mfma<F16> {
    __device__ static inline f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
};

template <>
struct Mfma<BF16> {
    __device__ static inline f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
};

// Position of natural output index o in the permuted output-scale vector.
__device__ inline int perm_out(int o) {
    return 32 * (o >> 5) + 8 * ((o & 7) >> 1) + 2 * ((o & 31) >> 3) + (o & 1);
}

template <typename T, bool kSin, bool kSout>
__global__ __launch_bounds__(kThreads) void gemm_onebit_kernel(const uint16_t* __restrict__ A,
                                                               const uint32_t* __restrict__ W,
                                                               const uint16_t* __restrict__ s_in,
                                                               const uint16_t* __restrict__ s_out,
                                                               uint16_t* __restrict__ C, int M, int K, int N) {
    __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDA];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int t = g >> 1;
    const int gp = g & 1;
    const int half_n = N >> 1;
    const int k_tiles = K >> 4;

    const int o_wave = n0 + wn * 64;  // first output column of this wave (multiple of 64)
    const bool n_valid = o_wave < N;
    // word column of (o, r2 = 2g') for this lane; o%8 = c%8 for every ni
    const int wcol = 32 * (o_wave >> 6) + 4 * (c & 7) + 2 * gp;

    f32x4 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int ld_row = tid >> 1;
    const int ld_col = (tid & 1) * 16;

    for (int k0 = 0; k0 < K; k0 += BK) {
        // ---- A tile -> LDS
        u32x4 v0 = u32x4{0, 0, 0, 0}, v1 = u32x4{0, 0, 0, 0};
        {
            const int gm = m0 + ld_row;
            const int gk = k0 + ld_col;
            if (gm < M && gk < K) {
                const uint16_t* p = A + static_cast<size_t>(gm) * K + gk;
                v0 = *reinterpret_cast<const u32x4*>(p);
                v1 = *reinterpret_cast<const u32x4*>(p + 8);
            }
        }
        // ---- B words and input scales for this lane
        const int tr = (k0 >> 4) + t;
        const bool k_valid = tr < k_tiles;
        uint32_t wlo = 0, whi = 0;
        if (n_valid && k_valid) {
            const uint2 w2 = *reinterpret_cast<const uint2*>(W + static_cast<size_t>(tr) * half_n + wcol);
            wlo = w2.x;
            whi = w2.y;
        }
        uint32_t sp[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            if (kSin) {
                sp[d] = k_valid ? *reinterpret_cast<const uint32_t*>(s_in + k0 + 16 * t + 4 * (2 * gp + (d & 1)) +
                                                                     2 * (d >> 1))
                                : 0u;
            } else {
                sp[d] = T::ONE_PAIR;
            }
        }

        __syncthreads();
        *reinterpret_cast<u32x4*>(&As[ld_row * LDA + ld_col]) = v0;
        *reinterpret_cast<u32x4*>(&As[ld_row * LDA + ld_col + 8]) = v1;
        __syncthreads();

        if (n_valid) {
            u32x4 bfrag[4];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int sh0 = 2 * (c >> 3) + 4 * ni;
                bfrag[ni].x = sp[0] ^ ((wlo << sh0) & 0x80008000u);
                bfrag[ni].y = sp[1] ^ ((whi << sh0) & 0x80008000u);
                bfrag[ni].z = sp[2] ^ ((wlo << (sh0 + 1)) & 0x80008000u);
                bfrag[ni].w = sp[3] ^ ((whi << (sh0 + 1)) & 0x80008000u);
            }
            const int kb = 16 * t + 4 * gp;
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
                const int row = wm * 64 + mi * 16 + c;
                const uint2 a01 = *reinterpret_cast<const uint2*>(&As[row * LDA + kb]);
                const uint2 a23 = *reinterpret_cast<const uint2*>(&As[row * LDA + kb + 8]);
                const u32x4 afrag = u32x4{a01.x, a01.y, a23.x, a23.y};
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = Mfma<T>::run(afrag, bfrag[ni], acc[mi][ni]);
            }
        }
    }

    if (!n_valid) return;
    // ---- epilogue: acc[mi][ni][i] is C[m0 + wm*64 + mi*16 + 4g + i][o_wave + ni*16 + c]
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
        const int o = o_wave + ni * 16 + c;
        const float so = kSout ? T::to_float(s_out[perm_out(o)]) : 1.0f;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + wm * 64 + mi * 16 + 4 * g + i;
                if (row < M) C[static_cast<size_t>(row) * N + o] = saturate_to<T>(acc[mi][ni][i] * so, T::SAT_GEMM);
            }
        }
    }
}

template <typename T>
int launch_onebit(const void* A, const uint32_t* W, const void* s_in, const void* s_out, void* C, int64_t M, int64_t K,
                  int64_t N, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(ceil_div(N, BN)), static_cast<unsigned>(ceil_div(M, BM)));
    const auto* a = static_cast<const uint16_t*>(A);
    const auto* si = static_cast<const uint16_t*>(s_in);
    const auto* so = static_cast<const uint16_t*>(s_out);
    auto* c = static_cast<uint16_t*>(C);
    if (s_in && s_out)
        gemm_onebit_kernel<T, true, true><<<grid, kThreads, 0, stream>>>(a, W, si, so, c, (int)M, (int)K, (int)N);
    else if (s_in)
        gemm_onebit_kernel<T, true, false><<<grid, kThreads, 0, stream>>>(a, W, si, so, c, (int)M, (int)K, (int)N);
    else if (s_out)
        gemm_onebit_kernel<T, false, true><<<grid, kThreads, 0, stream>>>(a, W, si, so, c, (int)M, (int)K, (int)N);
    else
        gemm_onebit_kernel<T, false, false><<<grid, kThreads, 0, stream>>>(a, W, si, so, c, (int)M, (int)K, (int)N);
    return check_launch("nq_gemm_onebit");
}

// ---------------------------------------------------------------------------- 32x32x16 kernel
//
// C[q, o] = sat(s_out[o] * sum_k A[q, k] * sign(k, o) * s_in[k]), computed as C^T = S * A^T on
// v_mfma_f32_32x32x16: the MFMA's A operand is 32 output features by 16 k of +-s_in, made from
// the Marlin words in registers; its B operand is 16 k by 32 rows of A. Lane l = (kg = l / 32,
// c = l % 32).
//   sign operand: feature o = o0 + c; dword d = (r8 = d / 2, r2 = 2kg + d % 2) holds the pair
//     k = 16tr + 8r8 + 2r2 + {0, 1}: Marlin word (tr, 32(o/64) + 4(o%8) + r2) shifted left by
//     2((o%16)/8) + 4((o%64)/16) + r8 has their signs on bits 15 and 31, and they go onto the
//     permuted s_in pair at 16tr + 4r2 + 2r8 (one 16-byte read per (tr, kg) covers all four);
//   A operand: row q0 + c, the same k: A[q][16tr + 4kg .. +3] and A[q][16tr + 8 + 4kg .. +3],
//     one 16-byte LDS read (the tile is stored with each 16-k group as k 0-3, 8-11, 4-7, 12-15);
//   C: lane holds C^T[o0 + 8(i/4) + 4kg + i%4][q0 + c], four consecutive features per group of
//      four registers, stored as one 8-byte write of C[q][o .. o+3].
// Per 64-k step a block needs its A tile (BQ x 64 halves), the sign words of its BP features
// (4 rows of BP/2 consecutive words: 1 KB at BP = 128) and 64 s_in values. Each is loaded once
// per block, coalesced, two steps ahead into registers, and staged through double-buffered
// LDS; lanes then read their words and s_in pairs from LDS (4 and 32 lanes share an address,
// which LDS broadcasts). Loading the words per lane instead (4 lanes and 2 tiles per word,
// and every wave of the block again) kept the texture data path ~70% busy.
// The grid runs q tiles fastest: blocks i, i+8, ... land on one XCD, so with q_tiles dividing
// 8 or a multiple of 8 each XCD streams its own rows of A through its L2.
#ifndef NQ_SX_WAVES_PER_EU
#define NQ_SX_WAVES_PER_EU 2
#endif
template <typename T, bool kSin, bool kSout, int BP, int BQ, int WP, int WQ, int BKK>
__global__ __launch_bounds__((BP / WP) * (BQ / WQ) * 64) __attribute__((amdgpu_waves_per_eu(NQ_SX_WAVES_PER_EU)))
void gemm_sx_kernel(
    const uint16_t* __restrict__ A, const uint32_t* __restrict__ W, const uint16_t* __restrict__ s_in,
    const uint16_t* __restrict__ s_out, uint16_t* __restrict__ C, int M, int K, int N, int q_tiles) {
    constexpr int NWP = BP / WP;
    constexpr int NWQ = BQ / WQ;
    constexpr int NT = NWP * NWQ * 64;
    constexpr int TP = WP / 32;
    constexpr int TQ = WQ / 32;
    constexpr int TG = WP / 64;            // 64-feature word groups per wave
    constexpr int KT = BKK / 16;           // 16-k tiles per step
    constexpr int LDX = BKK + 8;           // LDS row pitch of the A tile in halves
    constexpr int XPIECES = BQ * BKK / 8;  // 16-byte pieces of the A tile
    constexpr int XPT = XPIECES / NT;
    constexpr int WROW = BP / 2;           // sign words per k-tile row of the block
    constexpr int WWORDS = KT * WROW;      // sign words per step
    constexpr int WPT = (WWORDS + NT - 1) / NT;  // sign words per thread (the last round may be partial)
    constexpr int SDW = BKK / 2;           // s_in dwords per step
    static_assert(XPIECES % NT == 0 && (WWORDS % NT == 0 || WWORDS < NT), "tile pieces must divide evenly");
    static_assert(WP % 64 == 0 && BP % 64 == 0, "features come in whole 64-feature word groups");
    static_assert(SDW <= NT, "one s_in dword per thread");
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][BQ * LDX];
    __shared__ __attribute__((aligned(16))) uint32_t ws[2][WWORDS];
    __shared__ __attribute__((aligned(16))) uint32_t ss[2][SDW];
    __shared__ uint16_t sos[BP];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int c = lane & 31;
    const int kg = lane >> 5;
    const int wp = wave % NWP;
    const int wq = wave / NWP;
    const int qt = blockIdx.x % q_tiles;
    const int pt = blockIdx.x / q_tiles;
    const int q0 = qt * BQ;
    const int p0 = pt * BP;
    const uint32_t half_n = static_cast<uint32_t>(N) >> 1;
    const int k_iters = K / BKK;

    // lane constants: the word of feature o (per 64-feature group) and its shift per tile
    int wl[TG], shb[TP];
#pragma unroll
    for (int g = 0; g < TG; ++g) wl[g] = 32 * (wp * TG + g) + 4 * (c & 7) + 2 * kg;
#pragma unroll
    for (int tp = 0; tp < TP; ++tp) {
        const int o = wp * WP + 32 * tp + c;  // feature offset in the block
        shb[tp] = 2 * ((o & 15) >> 3) + 4 * ((o & 63) >> 4);
    }
    // load sources: A pieces, sign words (row kt = word / WROW of the step), s_in dwords
    const uint16_t* xsrc[XPT];
    int xdst[XPT];
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        const int piece = t + j * NT;
        const int row = piece / (BKK / 8);
        const int c8 = piece - row * (BKK / 8);
        xsrc[j] = A + static_cast<size_t>(min(q0 + row, M - 1)) * K + 8 * c8;
        xdst[j] = row * LDX + 8 * c8;  // with the exchange, piece 2m + e holds half e of group m
    }
    uint32_t wsrc[WPT];
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
        const int word = min(t + j * NT, WWORDS - 1);
        const int kt = word / WROW;
        wsrc[j] = kt * half_n + min(static_cast<uint32_t>(p0 / 2 + (word - kt * WROW)), half_n - 1);
    }
    const int sd = t % SDW;
    for (int e = t; e < BP; e += NT) sos[e] = kSout ? s_out[perm_out(min(p0 + e, N - 1))] : uint16_t(0);

    struct Ops {
        u32x4 x[XPT];
        uint32_t w[WPT];
        uint32_t s;  // used with kSin only
    };
    auto load_ops = [&](Ops& o, int iter) {
        const int k0 = iter * BKK;
#pragma unroll
        for (int j = 0; j < XPT; ++j) o.x[j] = *reinterpret_cast<const u32x4*>(xsrc[j] + k0);
        const uint32_t wrow = static_cast<uint32_t>(iter * KT) * half_n;
#pragma unroll
        for (int j = 0; j < WPT; ++j) o.w[j] = W[wrow + wsrc[j]];
        if (kSin) o.s = *reinterpret_cast<const uint32_t*>(s_in + k0 + 2 * sd);
    };
    auto store_ops = [&](const Ops& o, int buf) {
        // A piece is 8 halves of a row; lanes t (even) and t + 1 hold the two pieces of one
        // 16-k group. The tile is stored with each group as k 0-3, 8-11, 4-7, 12-15, so that a
        // lane's B fragment (k 4kg .. +3 and 8 + 4kg .. +3) is one 16-byte read: the even lane
        // keeps its low half and takes its neighbour's low half, the odd lane the high halves.
        const bool odd = t & 1;
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const u32x4 v = o.x[j];
            const uint32_t s0 = odd ? v.x : v.z, s1 = odd ? v.y : v.w;
            const uint32_t r0 = __builtin_amdgcn_mov_dpp(s0, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
            const uint32_t r1 = __builtin_amdgcn_mov_dpp(s1, 0xB1, 0xF, 0xF, false);
            const u32x4 out = odd ? u32x4{r0, r1, v.z, v.w} : u32x4{v.x, v.y, r0, r1};
            *reinterpret_cast<u32x4*>(&xs[buf][xdst[j]]) = out;
        }
#pragma unroll
        for (int j = 0; j < WPT; ++j)
            if (WWORDS % NT == 0 || t + j * NT < WWORDS) ws[buf][t + j * NT] = o.w[j];
        if (kSin && t < SDW) ss[buf][t] = o.s;
    };

    f32x16 acc[TP][TQ];
#pragma unroll
    for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[tp][tq][i] = 0.0f;

    const uint32_t mask = 0x80008000u;
    // One step: issue the loads of step it + 2 into `fill`, run the MFMAs of step it from LDS
    // buffer it % 2, put `nxt` (step it + 1) into the other buffer. The three register sets
    // rotate through a loop unrolled three times, so no register is ever copied (a copy of a
    // just-issued load would wait for it).
    // Loads and stores are unconditional (the tail reloads the last step): a load under a branch
    // makes the wait counts at the merge assume it may be the newest load, and the stores at the
    // end of the step would then wait for the loads just issued for two steps later.
    auto step = [&](Ops& nxt, Ops& fill, int it) {
        load_ops(fill, min(it + 2, k_iters - 1));
        __builtin_amdgcn_sched_barrier(0);
        const int buf = it & 1;
        const uint16_t* xb = &xs[buf][(wq * WQ + c) * LDX + 8 * kg];
        // every LDS read of the step first (one latency per step, not one per k tile), then the
        // sign operands and MFMAs as the reads land
        u32x4 bx[KT][TQ];
        uint2 wv[KT][TG];
        u32x4 sv[KT];
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int g = 0; g < TG; ++g) wv[kt][g] = *reinterpret_cast<const uint2*>(&ws[buf][kt * WROW + wl[g]]);
            sv[kt] = kSin ? *reinterpret_cast<const u32x4*>(&ss[buf][8 * kt + 4 * kg])
                          : u32x4{T::ONE_PAIR, T::ONE_PAIR, T::ONE_PAIR, T::ONE_PAIR};
#pragma unroll
            for (int tq = 0; tq < TQ; ++tq) {
                bx[kt][tq] = *reinterpret_cast<const u32x4*>(xb + 32 * tq * LDX + 16 * kt);
            }
        }
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int tp = 0; tp < TP; ++tp) {
                const uint32_t w0 = wv[kt][tp / 2].x, w1 = wv[kt][tp / 2].y;
                const int sft = shb[tp];
                const u32x4 a = u32x4{sv[kt].x ^ ((w0 << sft) & mask), sv[kt].z ^ ((w1 << sft) & mask),
                                      sv[kt].y ^ ((w0 << (sft + 1)) & mask), sv[kt].w ^ ((w1 << (sft + 1)) & mask)};
#pragma unroll
                for (int tq = 0; tq < TQ; ++tq) acc[tp][tq] = mfma32x32x16<T>(a, bx[kt][tq], acc[tp][tq]);
            }
        }
        store_ops(nxt, buf ^ 1);  // past the last step this writes a buffer nobody reads
        __syncthreads();
    };

    Ops o0, o1, o2;
    load_ops(o0, 0);
    load_ops(o1, min(1, k_iters - 1));
    store_ops(o0, 0);
    __syncthreads();
    int it = 0;
    for (; it + 3 <= k_iters; it += 3) {
        step(o1, o2, it);
        step(o2, o0, it + 1);
        step(o0, o1, it + 2);
    }
    if (it < k_iters) {
        step(o1, o2, it);
        if (it + 1 < k_iters) step(o2, o0, it + 1);
    }

    // epilogue: scale, saturate, four consecutive features per 8-byte store
#pragma unroll
    for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq) {
            const int q = q0 + wq * WQ + 32 * tq + c;
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int ol = wp * WP + 32 * tp + 8 * g4 + 4 * kg;  // feature offset in the block
                const int o = p0 + ol;
                uint16_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float sc = kSout ? T::to_float(sos[ol + e]) : 1.0f;
                    h[e] = saturate_to<T>(acc[tp][tq][4 * g4 + e] * sc, T::SAT_GEMM);
                }
                if (q < M && o < N) {
                    uint2 v;
                    v.x = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
                    v.y = static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16);
                    *reinterpret_cast<uint2*>(C + static_cast<size_t>(q) * N + o) = v;
                }
            }
        }
}

template <typename T, int BP, int BQ, int WP, int WQ, int BKK = 64>
void launch_sx(const void* A, const uint32_t* W, const void* s_in, const void* s_out, void* C, int64_t M, int64_t K,
               int64_t N, hipStream_t stream) {
    const int q_tiles = static_cast<int>(ceil_div(M, BQ));
    const int p_tiles = static_cast<int>(ceil_div(N, BP));
    const dim3 grid(static_cast<unsigned>(q_tiles * p_tiles));
    constexpr int NT = (BP / WP) * (BQ / WQ) * 64;
    const auto* a = static_cast<const uint16_t*>(A);
    const auto* si = static_cast<const uint16_t*>(s_in);
    const auto* so = static_cast<const uint16_t*>(s_out);
    auto* c = static_cast<uint16_t*>(C);
    const int m = static_cast<int>(M), k = static_cast<int>(K), n = static_cast<int>(N);
    if (s_in && s_out)
        gemm_sx_kernel<T, true, true, BP, BQ, WP, WQ, BKK><<<grid, NT, 0, stream>>>(a, W, si, so, c, m, k, n, q_tiles);
    else if (s_in)
        gemm_sx_kernel<T, true, false, BP, BQ, WP, WQ, BKK><<<grid, NT, 0, stream>>>(a, W, si, so, c, m, k, n, q_tiles);
    else if (s_out)
        gemm_sx_kernel<T, false, true, BP, BQ, WP, WQ, BKK><<<grid, NT, 0, stream>>>(a, W, si, so, c, m, k, n, q_tiles);
    else
        gemm_sx_kernel<T, false, false, BP, BQ, WP, WQ, BKK><<<grid, NT, 0, stream>>>(a, W, si, so, c, m, k, n, q_tiles);
}

// The 32x32x16 kernel needs whole 64-k iterations, 16-byte s_in pairs loads, 8-byte output
// stores and 32-bit word offsets; anything else runs on the 16x16x32 kernel.
template <typename T>
int launch_gemm(const char* name, const void* A, const uint32_t* W, const void* s_in, const void* s_out, void* C,
                int64_t M, int64_t K, int64_t N, hipStream_t stream) {
    const bool sx = K % 64 == 0 && K > 0 && (!s_in || aligned(s_in, 16)) && aligned(C, 8) &&
                    (K / 16) * (N / 2) < ((int64_t)1 << 31);
    if (!sx) return launch_onebit<T>(A, W, s_in, s_out, C, M, K, N, stream);
    launch_sx<T, 128, 128, 64, 64, 64>(A, W, s_in, s_out, C, M, K, N, stream);
    return check_launch(name);
}

int check_onebit(const char* name, int dtype, const void* A, const uint32_t* W, const void* s_in, const void* s_out,
                 const void* C, int64_t M, int64_t K, int64_t N) {
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "%s: unsupported dtype %d", name, dtype);
    if (M < 0 || K < 0 || N < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: negative size", name);
    if (K % 16 || N % 64)
        return fail(NQ_ERR_SHAPE, "%s: need K %% 16 == 0 and N %% 64 == 0, got K=%lld N=%lld", name, (long long)K,
                    (long long)N);
    if (M > INT32_MAX / 2 || K > INT32_MAX / 2 || N > INT32_MAX / 2 || M * K > (int64_t)1 << 40)
        return fail(NQ_ERR_UNSUPPORTED, "%s: sizes too large", name);
    if (M == 0 || N == 0) return NQ_OK;
    if (!A || !W || !C) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(A, 16) || !aligned(W, 8) || !aligned(C, 2) || (s_in && !aligned(s_in, 4)) ||
        (s_out && !aligned(s_out, 2)))
        return fail(NQ_ERR_ALIGNMENT, "%s: misaligned operand (A needs 16 bytes, weights 8)", name);
    return NQ_OK;
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" {

int nq_gemm_onebit(int dtype, const void* A, const uint32_t* w_bits, const void* s_in, const void* s_out, void* C,
                   int64_t M, int64_t K, int64_t N, nq_stream_t stream) {
    if (int s = check_onebit("nq_gemm_onebit", dtype, A, w_bits, s_in, s_out, C, M, K, N)) return s;
    if (M == 0 || N == 0) return NQ_OK;
    hipStream_t st = as_stream(stream);
    if (dtype == NQ_F16) return launch_gemm<F16>("nq_gemm_onebit", A, w_bits, s_in, s_out, C, M, K, N, st);
    return launch_gemm<BF16>("nq_gemm_onebit", A, w_bits, s_in, s_out, C, M, K, N, st);
}

int nq_gemm_nanoquant(int dtype, const void* A, const uint32_t* v_bits, const uint32_t* u_bits, const void* s_g,
                      const void* s_l, const void* s_h, void* imm, void* C, int64_t M, int64_t n, int64_t r_pad,
                      int64_t m, nq_stream_t stream) {
    if (int s = check_onebit("nq_gemm_nanoquant stage 1", dtype, A, v_bits, s_g, s_l, imm, M, n, r_pad)) return s;
    if (int s = check_onebit("nq_gemm_nanoquant stage 2", dtype, imm, u_bits, nullptr, s_h, C, M, r_pad, m)) return s;
    if (M == 0 || m == 0) return NQ_OK;
    hipStream_t st = as_stream(stream);
    if (r_pad > 0) {
        const int s1 = dtype == NQ_F16
                           ? launch_gemm<F16>("nq_gemm_nanoquant stage 1", A, v_bits, s_g, s_l, imm, M, n, r_pad, st)
                           : launch_gemm<BF16>("nq_gemm_nanoquant stage 1", A, v_bits, s_g, s_l, imm, M, n, r_pad, st);
        if (s1) return s1;
    }
    return dtype == NQ_F16 ? launch_gemm<F16>("nq_gemm_nanoquant stage 2", imm, u_bits, nullptr, s_h, C, M, r_pad, m, st)
                           : launch_gemm<BF16>("nq_gemm_nanoquant stage 2", imm, u_bits, nullptr, s_h, C, M, r_pad, m, st);
}

}  // extern "C"
