// Prefill GEMM on the Marlin sign layout: C[M, N] = sat((A[M, K] * W) * s_out) with
// W[k, o] = sign(k, o) * s_in[k], on gfx950 MFMA. Two kernels: gemm_dm_kernel
// (v_mfma_f32_32x32x16, operands fetched into LDS by DMA; K a multiple of 64) and
// gemm_onebit_kernel (v_mfma_f32_16x16x32, any K that is a multiple of 16), described here.
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
#include <algorithm>

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

// ------------------------------------------------------------------ LDS-DMA natural-k kernel
//
// The natural-k product with every operand of a 64-k step fetched by global_load_lds (16 bytes
// a lane for the A tile, 4 for sign words and s_in) straight into one of NBUF LDS buffers (three
// to eight), NBUF - 1 steps ahead, so no register holds a tile in flight. A wave's DMA writes 64
// consecutive LDS slots, so the A tile is unpadded (128-byte rows) and bank conflicts are avoided
// by where each lane fetches from: LDS chunk p of row r holds the row's 16-byte chunk
// p ^ ((r / 2) % 8). s_in is fetched in the order the operands read it (every wave keeps its own
// copy, so every wave issues the same number of DMAs per step). The DMAs are issued from inline assembly
// (dma16_lds / dma4_lds), from a per-step scalar base and a fixed byte offset per lane, so the
// compiler does not track them and waits for the LDS reads of a k tile only as far as they are
// needed (with the builtin it waited for every outstanding read at each first use; 5.8% / 5.9% /
// 8.7% off the op at B = 2048 on 7B gate / down / q, 5-8% at B = 256, bit-identical outputs).
// Before the barrier that ends a step each wave waits for its own DMAs of the next step, and only
// for those: the barrier carries no memory fence, so the DMAs of the step after stay in flight.
// With KS = 2 the block holds two groups of waves with buffers of their own, each over half of
// the k steps (for outputs too few to give every SIMD two waves); group 1 hands its accumulators
// to group 0 through LDS at the end. With KS = 4 (long K) four groups each take a quarter of the
// steps and hand their sums to group 0 one group at a time through the step buffers. With kSplit
// the grid repeats the tiles once per k range of split_steps steps, and each block stores its raw
// fp32 sums to its plane of `part` [splits][M][N]; gemm_split_finish_kernel adds the planes in
// order and applies the epilogue. A k range may also be shared by KS groups: contiguous runs of
// steps, the first len % KS groups one step longer; every group runs as many steps as the
// longest (the block's barriers are common), a shorter group's last one without its MFMAs.
template <typename T, bool kSin, bool kSout, int BP, int BQ, int WP, int WQ, int WPE, int KS, bool kSplit,
          int NBUF = 3, int BKK = 64>
__global__ __launch_bounds__((BP / WP) * (BQ / WQ) * 64 * KS) __attribute__((amdgpu_waves_per_eu(WPE)))
void gemm_dm_kernel(
    const uint16_t* __restrict__ A, const uint32_t* __restrict__ W, const uint16_t* __restrict__ s_in,
    const uint16_t* __restrict__ s_out, uint16_t* __restrict__ C, int M, int K, int N, int q_tiles, int p_tiles,
    float* __restrict__ part, int split_steps, const uint16_t* __restrict__ k_scale) {
    static_assert(BKK == 64 || BKK == 128, "64 or 128 k per step");
    constexpr int CPR = BKK / 8;       // 16-byte chunks per A-tile row
    // LDS chunk p of A-tile row r holds the row's chunk p ^ xswz(r). 64 banks of 4 bytes serve a
    // 16-byte read 16 lanes at a time, and the 16 lanes of such a phase read one chunk of 16
    // consecutive rows, so those must fall in 16 different 16-byte bank groups: with 128-byte
    // rows, r % 2 picks the half of the banks and (r / 2) % 8 the group within it (r % 8 alone
    // put rows r and r + 8 on the same banks); 256-byte rows span the banks, so r % 16.
    auto xswz = [](int r) { return BKK == 64 ? (r >> 1) & 7 : r & 15; };
    constexpr int NWP = BP / WP;
    constexpr int NWQ = BQ / WQ;
    constexpr int NTG = NWP * NWQ * 64;  // threads of one k group
    constexpr int NT = NTG * KS;
    constexpr int TP = WP / 32;
    constexpr int TQ = WQ / 32;
    constexpr int TG = WP / 64;        // 64-feature word groups per wave
    constexpr int KT = BKK / 16;       // 16-k tiles per step
    constexpr int XCH = BQ * BKK / 8;  // 16-byte chunks of the A tile
    constexpr int XPT = XCH / NTG;
    constexpr int WROW = BP / 2;       // sign words per k-tile row of the block
    constexpr int WWORDS = KT * WROW;  // sign words per step
    constexpr int WPT = WWORDS / NTG;
    constexpr int kIssued = XPT + WPT + (kSin ? 1 : 0);  // DMAs per step and wave
    constexpr int kAcc = TP * TQ * 16;                   // accumulators per lane
    static_assert(XCH % NTG == 0 && WWORDS % NTG == 0, "tile pieces must divide evenly");
    static_assert(WP % 64 == 0 && BP % 64 == 0, "features come in whole 64-feature word groups");
    static_assert(KS == 1 || KS == 2 || KS == 4, "one, two or four k groups");
    static_assert(!kSplit || !kSout, "k ranges of the grid are scaled later");
    // NBUF step buffers, each step's DMAs issued NBUF - 1 steps ahead
    static_assert(NBUF >= 3 && (NBUF - 2) * kIssued < 64, "the DMAs in flight fit the 6-bit vmcnt");
    __shared__ __attribute__((aligned(16))) uint16_t xsall[NBUF][KS][BQ * BKK];
    auto& xs0 = xsall[0];
    auto& xs1 = xsall[1];
    __shared__ __attribute__((aligned(16))) uint32_t wsall[NBUF][KS][WWORDS];
    __shared__ __attribute__((aligned(16))) uint32_t ssall[NBUF][kSin ? NT : 4];
    __shared__ float red_arr[KS == 2 ? kAcc * NTG : 1];
    // with four groups one group's sums at a time pass through the step buffers, free by then
    static_assert(KS != 4 || NBUF * KS * BQ * BKK * 2 >= kAcc * NTG * 4, "the step buffers hold one group's sums");
    float* red = KS == 4 ? reinterpret_cast<float*>(&xsall[0][0][0]) : red_arr;
    __shared__ uint16_t sos[BP];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int grp = wave / (NWP * NWQ);  // k group
    const int gw = wave - grp * (NWP * NWQ);
    const int tg = t - grp * NTG;
    const int c = lane & 31;
    const int kg = lane >> 5;
    const int wp = gw % NWP;
    const int wq = gw / NWP;
    const int split = kSplit ? static_cast<int>(blockIdx.x) / (q_tiles * p_tiles) : 0;
    const int tile = static_cast<int>(blockIdx.x) - split * (q_tiles * p_tiles);
    const int qt = tile % q_tiles;
    const int pt = tile / q_tiles;
    const int q0 = qt * BQ;
    const int p0 = pt * BP;
    const uint32_t half_n = static_cast<uint32_t>(N) >> 1;
    // steps of this block's k group or k range (the host makes K / 64 divide by KS and leaves no
    // k range empty), and the first of them
    // steps of this wave group (k_iters), the first of them (k_first) and the steps every group of
    // the block runs (k_all). Without kSplit the host makes K / 64 divide by KS. With it, a k range
    // holds len >= 1 steps (the host leaves none empty); with len < KS a group gets none, and its
    // DMAs, clamped to step k_iters - 1 = -1 of its run, re-fetch the range's last step.
    int k_iters, k_first, k_all;
    if (kSplit) {
        const int r0 = split * split_steps;
        const int len = min(split_steps, K / BKK - r0);
        const int q = len / KS, rem = len % KS;
        k_iters = q + (grp < rem ? 1 : 0);
        k_first = r0 + grp * q + min(grp, rem);
        k_all = q + (rem > 0 ? 1 : 0);
    } else {
        k_iters = K / BKK / KS;
        k_first = grp * k_iters;
        k_all = k_iters;
    }
    // k_scale (one block over all of K, K <= 32 * NT): A's columns whose k_scale entry is zero are
    // exact zeros (the previous stage multiplied them by it; the padded rank of the NanoQuant
    // factorisation), so the 64-k steps after the last nonzero entry add nothing and are not run.
    // Its entries are read here and examined once the first steps' DMAs are on their way.
    constexpr int kScaleLoads = 4;
    const bool k_trim = KS == 1 && !kSplit && k_scale != nullptr && K <= 8 * kScaleLoads * NT;
    u32x4 kv[kScaleLoads];
    if (k_trim) {
        const rsrc_t ks_rs = make_rsrc(k_scale, static_cast<uint32_t>(K) * 2u);
#pragma unroll
        for (int i = 0; i < kScaleLoads; ++i) kv[i] = load_b128(ks_rs, static_cast<uint32_t>(t + i * NT) * 16u);
    }
    __shared__ int klast[NT / 64];

    // lane constants: the first of the four words of its feature per 64-feature group, the shift
    // per 32-feature tile, its A-tile rows and the swizzled chunk of its 8 k per k tile
    int wl[TG], shb[TP];
#pragma unroll
    for (int g = 0; g < TG; ++g) wl[g] = 32 * (wp * TG + g) + 4 * (c & 7);
#pragma unroll
    for (int tp = 0; tp < TP; ++tp) {
        const int o = wp * WP + 32 * tp + c;  // feature offset in the block
        shb[tp] = 2 * ((o & 15) >> 3) + 4 * ((o & 63) >> 4) + kg;
    }
    const int xrow = (wq * WQ + c) * BKK;  // halves; rows of tile tq are 32 tq further
    // DMA sources: A chunks (32-bit element offsets), sign words, s_in dwords in read order
    uint32_t xoff[XPT];
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
        const int ci = j * NTG + tg;
        const int r = ci / CPR;
        xoff[j] = static_cast<uint32_t>(min(q0 + r, M - 1)) * static_cast<uint32_t>(K) + 8 * ((ci % CPR) ^ xswz(r));
    }
    uint32_t wsrc[WPT];
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
        const int wi = j * NTG + tg;
        const int kt = wi / WROW;
        wsrc[j] = kt * half_n + min(static_cast<uint32_t>(p0 / 2 + (wi - kt * WROW)), half_n - 1);
    }
    // s_in comes permuted: dword 8tr + 2r2 + r8 holds the pair k = 16tr + 8r8 + 2r2 + {0, 1}; LDS
    // slot 8tr + 4r8 + r2 of the wave's copy takes it, so the pairs r2 = 0..3 of one r8 are adjacent
    const int sl = lane & (BKK / 2 - 1);
    const int sidx = (sl & ~7) | ((sl & 3) << 1) | ((sl >> 2) & 1);
    for (int e = t; e < BP; e += NT) sos[e] = kSout ? s_out[perm_out(min(p0 + e, N - 1))] : uint16_t(0);

    // byte offsets of each lane's DMA sources from the step's base addresses
    uint32_t xoffb[XPT], wsrcb[WPT];
#pragma unroll
    for (int j = 0; j < XPT; ++j) xoffb[j] = 2u * xoff[j];
#pragma unroll
    for (int j = 0; j < WPT; ++j) wsrcb[j] = 4u * wsrc[j];
    const uint32_t sidxb = 4u * static_cast<uint32_t>(sidx);
    // LDS byte addresses of this wave's DMA destinations in each step buffer
    uint32_t lx[NBUF], lw[NBUF], ls[NBUF];
#pragma unroll
    for (int b = 0; b < NBUF; ++b) {
        lx[b] = __builtin_amdgcn_readfirstlane(lds_addr(xsall[b][grp]) + static_cast<uint32_t>(gw) * 1024u);
        lw[b] = __builtin_amdgcn_readfirstlane(lds_addr(wsall[b][grp]) + static_cast<uint32_t>(gw) * 256u);
        ls[b] = __builtin_amdgcn_readfirstlane(lds_addr(ssall[b]) + static_cast<uint32_t>(wave) * 256u);
    }
    auto issue = [&](int iter, int b) {
        const uint32_t k0 = static_cast<uint32_t>((k_first + iter) * BKK);
        const uint16_t* abase = A + k0;
#pragma unroll
        for (int j = 0; j < XPT; ++j) dma16_lds(abase, xoffb[j], lx[b] + static_cast<uint32_t>(j * NTG * 16));
        const uint32_t* wbase = W + static_cast<size_t>(static_cast<uint32_t>((k_first + iter) * KT)) * half_n;
#pragma unroll
        for (int j = 0; j < WPT; ++j) dma4_lds(wbase, wsrcb[j], lw[b] + static_cast<uint32_t>(j * NTG * 4));
        if (kSin) dma4_lds(s_in + k0, sidxb, ls[b]);
    };

    f32x16 acc[TP][TQ];
#pragma unroll
    for (int tp = 0; tp < TP; ++tp)
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[tp][tq][i] = 0.0f;

    // +-1 pairs kept in a register, so that each sign operand dword is one shift and one v_bitop3
    uint32_t one = T::ONE_PAIR;
    asm volatile("" : "+v"(one));
    struct Frag {
        u32x4 w[TG];
        u32x4 s;
        u32x4 x[TQ];
    };
    auto read_kt = [&](Frag& f, const uint16_t* xs, const uint32_t* ws, const uint32_t* ss, int kt) {
        const int pos = (2 * kt + kg) ^ xswz(c);  // the wave's rows start at multiples of 32
#pragma unroll
        for (int g = 0; g < TG; ++g) f.w[g] = *reinterpret_cast<const u32x4*>(ws + kt * WROW + wl[g]);
        f.s = kSin ? *reinterpret_cast<const u32x4*>(ss + wave * 64 + 8 * kt + 4 * kg) : u32x4{one, one, one, one};
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq)
            f.x[tq] = *reinterpret_cast<const u32x4*>(xs + xrow + 32 * tq * BKK + 8 * pos);
    };
    const uint32_t mask = 0x80008000u;
    auto compute_kt = [&](const Frag& f) {
#pragma unroll
        for (int tp = 0; tp < TP; ++tp) {
            // two words per 64-bit shift: sft <= 15, so the bits the shift carries from the low word
            // into the high one land below bit 15 and the mask drops them (one v_lshlrev_b64 for
            // two v_lshlrev_b32; same-box A/B: B = 2048 gate / down 1.5 / 1.9% faster, B = 256 gate 3%)
            const u32x4 w = f.w[tp / 2];
            const int sft = shb[tp];
            const uint64_t w01 = ((static_cast<uint64_t>(w.y) << 32) | w.x) << sft;
            const uint64_t w23 = ((static_cast<uint64_t>(w.w) << 32) | w.z) << sft;
            const u32x4 a = u32x4{f.s.x ^ (static_cast<uint32_t>(w01) & mask),
                                  f.s.y ^ (static_cast<uint32_t>(w01 >> 32) & mask),
                                  f.s.z ^ (static_cast<uint32_t>(w23) & mask),
                                  f.s.w ^ (static_cast<uint32_t>(w23 >> 32) & mask)};
#pragma unroll
            for (int tq = 0; tq < TQ; ++tq) acc[tp][tq] = mfma32x32x16<T>(a, f.x[tq], acc[tp][tq]);
        }
    };
    // One step out of buffer b: DMA step it + NBUF - 1 into the buffer step it - 1 used, run the
    // MFMAs of step it (each k tile's reads issued before the previous tile's MFMAs), wait for this
    // wave's DMAs of step it + 1, barrier. The tail re-fetches the last step into free buffers, so
    // that every step issues the same DMAs.
    auto step = [&](int b, int it) {
        const uint16_t* xc = xsall[b][grp];
        const uint32_t* wc = wsall[b][grp];
        const uint32_t* sc = ssall[b];
        issue(min(it + NBUF - 1, k_iters - 1), (b + NBUF - 1) % NBUF);
        __builtin_amdgcn_sched_barrier(0);  // the DMAs go out first, not after the step's MFMAs
        if (!(kSplit && KS > 1) || it < k_iters) {  // uniform over the wave group
            Frag f[2];
            read_kt(f[0], xc, wc, sc, 0);
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
                if (kt + 1 < KT) read_kt(f[(kt + 1) & 1], xc, wc, sc, kt + 1);
                compute_kt(f[kt & 1]);
            }
        }
        wait_vmcnt<(NBUF - 2) * kIssued>();
        barrier_keep_dma();
    };

#pragma unroll
    for (int b = 0; b + 1 < NBUF; ++b) issue(min(b, k_iters - 1), b);
    if (k_trim) {
        int last = -1;  // the last nonzero entry this thread holds (zeros past K)
#pragma unroll
        for (int i = 0; i < kScaleLoads; ++i) {
            const uint32_t d[4] = {kv[i].x, kv[i].y, kv[i].z, kv[i].w};
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (((d[j >> 1] >> (16 * (j & 1))) & 0x7fffu) != 0) last = 8 * (t + i * NT) + j;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) last = max(last, __shfl_xor(last, off, 64));
        if (lane == 0) klast[wave] = last;
    }
    wait_vmcnt<(NBUF - 2) * kIssued>();
    __syncthreads();
    if (k_trim) {
        int last = -1;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) last = max(last, klast[w]);
        k_iters = max(1, min(k_iters, (last + BKK) / BKK));  // steps up to the one holding `last`
        k_all = k_iters;
    }
    int it = 0;
    for (; it + NBUF <= k_all; it += NBUF) {
#pragma unroll
        for (int b = 0; b < NBUF; ++b) step(b, it + b);
    }
#pragma unroll
    for (int b = 0; b + 1 < NBUF; ++b)
        if (it + b < k_all) step(b, it + b);
    wait_vmcnt<0>();  // the tail's re-fetches land before the block's LDS is reused or released

    if (KS == 4) {  // groups 1, 2 and 3 join group 0's sums in that order (deterministic)
        __syncthreads();  // every wave is done with its last step's buffers
#pragma unroll
        for (int src = 1; src < 4; ++src) {
            if (grp == src) {
#pragma unroll
                for (int tp = 0; tp < TP; ++tp)
#pragma unroll
                    for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
                        for (int i = 0; i < 16; ++i) red[((tp * TQ + tq) * 16 + i) * NTG + tg] = acc[tp][tq][i];
            }
            __syncthreads();
            if (grp == 0) {
#pragma unroll
                for (int tp = 0; tp < TP; ++tp)
#pragma unroll
                    for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
                        for (int i = 0; i < 16; ++i) acc[tp][tq][i] += red[((tp * TQ + tq) * 16 + i) * NTG + tg];
            }
            __syncthreads();
        }
        if (grp != 0) return;
    }
    if (KS == 2) {  // group 1's sums join group 0's (lane-contiguous, conflict-free)
        if (grp == 1) {
#pragma unroll
            for (int tp = 0; tp < TP; ++tp)
#pragma unroll
                for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
                    for (int i = 0; i < 16; ++i) red[((tp * TQ + tq) * 16 + i) * NTG + tg] = acc[tp][tq][i];
        }
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int tp = 0; tp < TP; ++tp)
#pragma unroll
            for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[tp][tq][i] += red[((tp * TQ + tq) * 16 + i) * NTG + tg];
    }

    if (kSplit) {  // raw sums of this k range, four consecutive features per 16-byte store
        float* plane = part + static_cast<size_t>(split) * static_cast<size_t>(M) * static_cast<size_t>(N);
#pragma unroll
        for (int tp = 0; tp < TP; ++tp)
#pragma unroll
            for (int tq = 0; tq < TQ; ++tq) {
                const int q = q0 + wq * WQ + 32 * tq + c;
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int o = p0 + wp * WP + 32 * tp + 8 * g4 + 4 * kg;
                    if (q < M && o < N)
                        *reinterpret_cast<f32x4*>(plane + static_cast<size_t>(q) * N + o) =
                            f32x4{acc[tp][tq][4 * g4], acc[tp][tq][4 * g4 + 1], acc[tp][tq][4 * g4 + 2],
                                  acc[tp][tq][4 * g4 + 3]};
                }
            }
        return;
    }
    if constexpr (WP == 64 && NWP * NWQ == 4 && BQ * BKK >= 4096) {
        // epilogue through LDS. An 8-byte store of four features per lane touches the lines of 32
        // output rows; instead each wave scales and saturates its tile 32 rows at a time into 4 KB
        // of the first two step buffers (128-byte rows, 16-byte chunk ch of row r at ch ^ ((r / 2) % 8):
        // the 16-byte reads below are conflict-free, and 32 lanes' 8-byte writes meet two to a bank
        // group, where r % 8 put four) and stores whole 128-byte row pieces, 16 bytes a lane.
        if constexpr (KS == 1) __syncthreads();  // every wave is done with its last step's buffers
        uint32_t* tb = reinterpret_cast<uint32_t*>(gw < 2 ? &xs0[0][0] : &xs1[0][0]) + (gw & 1) * 1024;
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq) {
#pragma unroll
            for (int tp = 0; tp < TP; ++tp)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int ol = wp * WP + 32 * tp + 8 * g4 + 4 * kg;  // feature offset in the block
                    uint16_t h[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float sc = kSout ? T::to_float(sos[ol + e]) : 1.0f;
                        h[e] = saturate_to<T>(acc[tp][tq][4 * g4 + e] * sc, T::SAT_GEMM);
                    }
                    uint2 v;
                    v.x = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
                    v.y = static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16);
                    *reinterpret_cast<uint2*>(tb + 32 * c + 4 * ((4 * tp + g4) ^ ((c >> 1) & 7)) + 2 * kg) = v;
                }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int rr = (lane >> 3) + 8 * j;  // row of the 32-row piece; 8 lanes a row
                const u32x4 d = *reinterpret_cast<const u32x4*>(tb + 32 * rr + 4 * ((lane & 7) ^ ((rr >> 1) & 7)));
                const int q = q0 + wq * WQ + 32 * tq + rr;
                const int o = p0 + wp * WP + 8 * (lane & 7);
                if (q < M && o < N) *reinterpret_cast<u32x4*>(C + static_cast<size_t>(q) * N + o) = d;
            }
        }
        return;
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

template <typename T, int BP, int BQ, int WP, int WQ, int WPE, int KS, int NBUF = 3>
void launch_dm(const void* A, const uint32_t* W, const void* s_in, const void* s_out, void* C, int64_t M, int64_t K,
               int64_t N, hipStream_t stream, const void* k_scale = nullptr) {
    const auto* ksc = static_cast<const uint16_t*>(k_scale);
    const int q_tiles = static_cast<int>(ceil_div(M, BQ));
    const int p_tiles = static_cast<int>(ceil_div(N, BP));
    const dim3 grid(static_cast<unsigned>(q_tiles * p_tiles));
    constexpr int NT = (BP / WP) * (BQ / WQ) * 64 * KS;
    const auto* a = static_cast<const uint16_t*>(A);
    const auto* si = static_cast<const uint16_t*>(s_in);
    const auto* so = static_cast<const uint16_t*>(s_out);
    auto* c = static_cast<uint16_t*>(C);
    const int m = static_cast<int>(M), k = static_cast<int>(K), n = static_cast<int>(N);
    if (s_in && s_out)
        gemm_dm_kernel<T, true, true, BP, BQ, WP, WQ, WPE, KS, false, NBUF>
            <<<grid, NT, 0, stream>>>(a, W, si, so, c, m, k, n, q_tiles, p_tiles, nullptr, 0, ksc);
    else if (s_in)
        gemm_dm_kernel<T, true, false, BP, BQ, WP, WQ, WPE, KS, false, NBUF>
            <<<grid, NT, 0, stream>>>(a, W, si, so, c, m, k, n, q_tiles, p_tiles, nullptr, 0, ksc);
    else if (s_out)
        gemm_dm_kernel<T, false, true, BP, BQ, WP, WQ, WPE, KS, false, NBUF>
            <<<grid, NT, 0, stream>>>(a, W, si, so, c, m, k, n, q_tiles, p_tiles, nullptr, 0, ksc);
    else
        gemm_dm_kernel<T, false, false, BP, BQ, WP, WQ, WPE, KS, false, NBUF>
            <<<grid, NT, 0, stream>>>(a, W, si, so, c, m, k, n, q_tiles, p_tiles, nullptr, 0, ksc);
}

// C[q, o] = sat(s_out[o] * sum_s part[s][q][o]) (the planes added in order); one thread per four
// consecutive outputs.
template <typename T, bool kSout>
__global__ __launch_bounds__(256) void gemm_split_finish_kernel(const float* __restrict__ part,
                                                                const uint16_t* __restrict__ s_out,
                                                                uint16_t* __restrict__ C, int M, int N, int splits) {
    const int64_t quads = static_cast<int64_t>(M) * (N / 4);
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= quads) return;
    const int64_t q = i / (N / 4);
    const int o = static_cast<int>(i - q * (N / 4)) * 4;
    const size_t plane = static_cast<size_t>(M) * static_cast<size_t>(N);
    const float* src = part + static_cast<size_t>(q) * N + o;
    f32x4 sum = *reinterpret_cast<const f32x4*>(src);
    // the planes' loads go out kBatch at a time before their adds (a dependent load per plane waited
    // out a memory round trip each); the adds keep the order s = 1, 2, ...
    constexpr int kBatch = 16;
    for (int s0 = 1; s0 < splits; s0 += kBatch) {
        f32x4 pv[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i)
            pv[i] = s0 + i < splits ? *reinterpret_cast<const f32x4*>(src + static_cast<size_t>(s0 + i) * plane)
                                    : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < kBatch; ++i)
            if (s0 + i < splits) sum = f32x4{sum[0] + pv[i][0], sum[1] + pv[i][1], sum[2] + pv[i][2], sum[3] + pv[i][3]};
    }
    uint16_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float sc = kSout ? T::to_float(s_out[perm_out(o + e)]) : 1.0f;
        h[e] = saturate_to<T>(sum[e] * sc, T::SAT_GEMM);
    }
    uint2 v;
    v.x = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
    v.y = static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16);
    *reinterpret_cast<uint2*>(C + static_cast<size_t>(q) * N + o) = v;
}

// K split over `splits` ranges of the grid, each range over KS wave groups of a block: the
// ranges' raw sums into part [splits][M][N] fp32, then the finishing launch.
template <typename T, int BP, int BQ, int WP, int WQ, int WPE, int NBUF = 3, int KS = 1>
void launch_dm_split(const void* A, const uint32_t* W, const void* s_in, const void* s_out, void* C, int64_t M,
                     int64_t K, int64_t N, float* part, int splits, int split_steps, hipStream_t stream) {
    const int q_tiles = static_cast<int>(ceil_div(M, BQ));
    const int p_tiles = static_cast<int>(ceil_div(N, BP));
    const dim3 grid(static_cast<unsigned>(q_tiles * p_tiles * splits));
    constexpr int NT = (BP / WP) * (BQ / WQ) * 64 * KS;
    const auto* a = static_cast<const uint16_t*>(A);
    const auto* si = static_cast<const uint16_t*>(s_in);
    const auto* so = static_cast<const uint16_t*>(s_out);
    auto* c = static_cast<uint16_t*>(C);
    const int m = static_cast<int>(M), k = static_cast<int>(K), n = static_cast<int>(N);
    if (s_in)
        gemm_dm_kernel<T, true, false, BP, BQ, WP, WQ, WPE, KS, true, NBUF>
            <<<grid, NT, 0, stream>>>(a, W, si, nullptr, c, m, k, n, q_tiles, p_tiles, part, split_steps, nullptr);
    else
        gemm_dm_kernel<T, false, false, BP, BQ, WP, WQ, WPE, KS, true, NBUF>
            <<<grid, NT, 0, stream>>>(a, W, nullptr, nullptr, c, m, k, n, q_tiles, p_tiles, part, split_steps, nullptr);
    const int64_t quads = M * (N / 4);
    const dim3 fgrid(static_cast<unsigned>(ceil_div(quads, 256)));
    if (s_out)
        gemm_split_finish_kernel<T, true><<<fgrid, 256, 0, stream>>>(part, so, c, m, n, splits);
    else
        gemm_split_finish_kernel<T, false><<<fgrid, 256, 0, stream>>>(part, so, c, m, n, splits);
}

// How one GEMM is launched. The 32x32x16 kernel needs whole 64-k steps, 16-byte output stores
// and 32-bit element offsets into A and the words; anything else runs on the 16x16x32 kernel.
// Block tile 256 features x 64 rows, four waves of 64 x 64, or 256 x 128 with waves of 64 x 128
// (each sign fragment decoded once for four MFMAs instead of two; two waves per SIMD). The grid
// decides (tiles of 256 x 64 counted):
//   1024 tiles or more: one block per 256 x 128 tile (B = 2048, K = 1792, N = 11008: 85.5 -> 77 us;
//     K = 3584, N = 28672: 360 -> 338 us; 5-9% on every such stage 2 measured; at 512 tiles the
//     64-row tile stays ahead, 31.2 against 32.2 us on N = 4096);
//   more than 256 tiles: one block per tile (B = 2048, K = 8192, N = 2304, 288 tiles: 119.0 us
//     with K over two wave groups -> 105.2 us; K = 4096, N = 3072, 384 tiles: 64.3 -> 59.8 us);
//   160-256 tiles: K split over two wave groups inside each block (B = 2048, K = 4096,
//     N = 1792, 224 tiles: 46 -> 38 us against one block per tile; 256 tiles: 42.7 -> 40.3 us),
//     over four from 128 steps;
//   fewer, with at most 64 even 64-k steps and 128+ tiles of 32 rows: 32-row tiles, K over two
//     wave groups (B = 256, K = 1280 -> 1120, N = 4096: 16.6 us split across the grid -> 9.1 us;
//     B = 2048, K = 512, N = 1024: 8.8 -> 6.8 us; up to 32 steps at first, then measured on the
//     op at B = 256 with 36-56 steps: Llama-3-70B q/o 45.4 -> 41.0 us, down 93.4 -> 86.4,
//     Llama-2-7B down at 1.0 bpw 53.9 -> 49.7);
//   128-159 tiles otherwise: as 160-511;
//   fewer: K split across the grid, each range at least 8 steps, fp32 sums into the caller's
//     workspace, then a finishing launch. Up to 128 steps: about one block per CU, on 32-row tiles
//     below 64 tiles of 64 rows (B = 256, K = 4096, N = 1792: 8 ranges of 28 tiles 19.6 us -> 4
//     ranges of 56 tiles 15.8 us; B = 2048, K = 8192, N = 512: 8 ranges 34.6 -> 4 ranges 30.2 us).
//     Where the ranges of one block per CU on 32-row tiles hold 32-96 steps, each range runs over
//     four wave groups (below). Longer K: the same while its ranges hold at most 96 steps, else
//     the same on 64-row tiles (once about two blocks per CU on 64-row tiles in one wave group:
//     B = 256, K = 28672, N = 3584, 9 ranges of 56 tiles 66.8 us, against 93.2 us for 2 ranges of
//     112 32-row tiles in one group). Without that workspace, as the grid's K groups above.
constexpr int64_t kSplitTarget = 256;    // blocks a split grid aims at (one per CU; two for long K)
constexpr int64_t kSplitMinSteps = 8;    // 64-k steps of the shortest range
constexpr int64_t kSplitLongSteps = 128; // beyond this many steps K counts as long
// Step buffers (the DMAs of a step go out that many steps less one ahead): three, except K over
// two wave groups on 64-row tiles (four: 152 KB of LDS with the groups' hand-over) and ranges of 16
// or more steps split across the grid on 32-row tiles (eight). Interleaved same-box A/B through the
// op, fp16, bit-identical, minimum of 8 rounds: B = 256 gate 30.7 -> 29.5 us (each of the two
// changes alone about half of it), Llama-3-70B gate 83.2 -> 80.3; every other Llama-2-7B and
// Llama-3-70B cell at B = 64-2048 within 1%. Deeper buffers elsewhere measured no better (B = 2048
// stage 2 within 0.5%) or slower (the long-K split on 64-row tiles at six or eight: B = 256 down
// 36.0 -> 37.1 / 40.3 us, two blocks a CU no longer fitting at eight; ten-step ranges at eight:
// B = 128 down 34.5 -> 35.0).
constexpr int kBufGroups = 4, kBufSplit32Long = 8, kSplit32LongSteps = 16;
// Long K on small grids: 32-row tiles, one block of 16 waves per CU, each k range over four wave
// groups, when the ranges hold at most kSplitGroupMaxSteps steps (each group at least
// kSplitGroupMinSteps). It writes a quarter to a half of the fp32 partials of the 64-row plan
// below (7B down_proj at B = 256: 4 ranges, 7.3 MB, against 18 ranges, 33 MB). Interleaved same-box
// A/B through the op, fp16: Llama-2-7B down_proj at 0.55 bpw B = 256 33.9 -> 29.1 us, B = 128 34.1
// -> 28.9, B = 64 26.8 -> 24.0, at 1.0 bpw B = 256 42.4 -> 40.3 (2 ranges of 86 steps). With 224-step
// ranges (Llama-3-70B down_proj at B = 256) it was slower, 74.4 -> 78.4 and 66.1 -> 71.9 (mixed
// rank): there the 64-row tiles' MFMA efficiency outweighs the partials' traffic. For K of up to
// 128 steps it runs where its ranges hold 32-96 steps, as many ranges as the one-group plan: B = 256
// Llama-3-70B gate/up 72.8 -> 69.2 us, q/o 32.6 -> 30.3, Llama-2-7B gate/up at 1.0 bpw 38.6 -> 36.6,
// B = 2048 Llama-3-70B k/v 32.7 -> 31.1. Shorter ranges lost (B = 64 gate/up 23.6 -> 24.7,
// q/k/v/o 19.5 -> 21.0, where four steps a group halve the ranges). Long K with longer ranges runs
// the same split on 64-row tiles (each sign fragment feeding twice the MFMAs): Llama-3-70B
// down_proj at B = 256 (4 ranges of 112 steps, 14.7 MB of partials, against 9 ranges and 33 MB on
// one group) 78.9 -> 76.4 us, mixed rank 69.5 -> 67.6. Where the 32-row split applies it stays
// ahead (7B down_proj B = 256 30.4 against 33.3 us on 64-row tiles).
constexpr int64_t kSplitGroupMinSteps = 4, kSplitGroupMaxSteps = 96, kSplitGroupShortMinSteps = 32;
enum GemmMode {
    kModeOnebit,
    kModeTile,
    kModeTile128,
    kModeGroups,
    kModeGroups32,
    kModeSplit,
    kModeSplit32,
    kModeSplitGroups32,
    kModeSplitGroups64
};
struct GemmPlan {
    GemmMode mode = kModeOnebit;
    int splits = 1;
    int split_steps = 0;
    size_t workspace_bytes = 0;  // needed by kModeSplit / kModeSplit32
};

GemmPlan plan_gemm(int64_t M, int64_t K, int64_t N) {
    GemmPlan p;
    if (K % 64 || K <= 0 || M * K >= ((int64_t)1 << 31) || (K / 16) * (N / 2) >= ((int64_t)1 << 31)) return p;
    const int64_t tiles = ceil_div(M, 64) * ceil_div(N, 256);
    const int64_t tiles32 = ceil_div(M, 32) * ceil_div(N, 256);
    const int64_t steps = K / 64;
    const bool even = steps % 2 == 0;
    p.mode = tiles >= 1024 ? kModeTile128 : kModeTile;
    if (tiles > 256) return p;
    if (even) p.mode = kModeGroups;
    if (tiles >= 160) return p;
    if (even && steps <= 64 && tiles32 >= 128) {
        p.mode = kModeGroups32;
        return p;
    }
    if (tiles >= 128) return p;
    const bool long_k = steps > kSplitLongSteps;
    {  // 32-row tiles, a block per CU, each k range over four wave groups
        const int64_t want = std::min<int64_t>(kSplitTarget / tiles32, steps / (4 * kSplitGroupMinSteps));
        const int64_t run = want >= 2 ? ceil_div(steps, want) : 0;  // steps of a range
        if (run > 0 && run <= kSplitGroupMaxSteps && (long_k || run >= kSplitGroupShortMinSteps)) {
            p.split_steps = static_cast<int>(ceil_div(steps, want));
            p.splits = static_cast<int>(ceil_div(steps, p.split_steps));
            if (p.splits >= 2) {
                p.mode = kModeSplitGroups32;
                p.workspace_bytes = static_cast<size_t>(p.splits) * static_cast<size_t>(M) * static_cast<size_t>(N) * 4;
                return p;
            }
        }
    }
    if (long_k) {  // longer ranges: 64-row tiles, a block per CU, each k range over four wave groups
        const int64_t want = std::min<int64_t>(kSplitTarget / tiles, steps / (4 * kSplitGroupMinSteps));
        if (want >= 2) {
            p.split_steps = static_cast<int>(ceil_div(steps, want));
            p.splits = static_cast<int>(ceil_div(steps, p.split_steps));
            if (p.splits >= 2) {
                p.mode = kModeSplitGroups64;
                p.workspace_bytes = static_cast<size_t>(p.splits) * static_cast<size_t>(M) * static_cast<size_t>(N) * 4;
                return p;
            }
        }
    }
    const bool rows32 = !long_k && tiles < 64;
    const int64_t grid_tiles = rows32 ? tiles32 : tiles;
    const int64_t want = std::min<int64_t>((long_k ? 2 : 1) * kSplitTarget / grid_tiles, steps / kSplitMinSteps);
    if (want < 2) return p;
    p.split_steps = static_cast<int>(ceil_div(steps, want));
    p.splits = static_cast<int>(ceil_div(steps, p.split_steps));  // every range non-empty
    if (p.splits < 2) return p;
    p.mode = rows32 ? kModeSplit32 : kModeSplit;
    p.workspace_bytes = static_cast<size_t>(p.splits) * static_cast<size_t>(M) * static_cast<size_t>(N) * 4;
    return p;
}

// k_scale: the scale the previous stage gave A's columns (nullptr if none); see gemm_dm_kernel.
template <typename T>
int launch_gemm(const char* name, const void* A, const uint32_t* W, const void* s_in, const void* s_out, void* C,
                int64_t M, int64_t K, int64_t N, void* workspace, size_t workspace_bytes, hipStream_t stream,
                const void* k_scale = nullptr) {
    GemmPlan p = plan_gemm(M, K, N);
    if (p.mode != kModeOnebit && !aligned(C, 16)) p.mode = kModeOnebit;
    if ((p.mode == kModeSplit || p.mode == kModeSplit32 || p.mode == kModeSplitGroups32 ||
         p.mode == kModeSplitGroups64) &&
        (!workspace || workspace_bytes < p.workspace_bytes || !aligned(workspace, 16)))
        p.mode = (K / 64) % 2 == 0 ? kModeGroups : kModeTile;
    switch (p.mode) {
        case kModeOnebit:
            return launch_onebit<T>(A, W, s_in, s_out, C, M, K, N, stream);
        case kModeTile:
            launch_dm<T, 256, 64, 64, 64, 2, 1>(A, W, s_in, s_out, C, M, K, N, stream, k_scale);
            break;
        case kModeTile128:
            launch_dm<T, 256, 128, 64, 128, 2, 1>(A, W, s_in, s_out, C, M, K, N, stream, k_scale);
            break;
        case kModeGroups:
            // long K over four wave groups (16 waves a block, four per SIMD, 128 VGPRs): B = 2048,
            // K = 11008, N = 1792 (172 steps) 2.5% faster per op, same-box A/B; at 64 steps no change,
            // at 28 steps (B = 256, N = 11008) 5.6% slower
            if ((K / 64) % 4 == 0 && K / 64 >= 128)
                launch_dm<T, 256, 64, 64, 64, 4, 4>(A, W, s_in, s_out, C, M, K, N, stream);
            else
                launch_dm<T, 256, 64, 64, 64, 2, 2, kBufGroups>(A, W, s_in, s_out, C, M, K, N, stream);
            break;
        case kModeGroups32:
            launch_dm<T, 256, 32, 64, 32, 2, 2>(A, W, s_in, s_out, C, M, K, N, stream);
            break;
        case kModeSplit:
            launch_dm_split<T, 256, 64, 64, 64, 2>(A, W, s_in, s_out, C, M, K, N, static_cast<float*>(workspace),
                                                   p.splits, p.split_steps, stream);
            break;
        case kModeSplit32:
            if (p.split_steps >= kSplit32LongSteps)
                launch_dm_split<T, 256, 32, 64, 32, 2, kBufSplit32Long>(
                    A, W, s_in, s_out, C, M, K, N, static_cast<float*>(workspace), p.splits, p.split_steps, stream);
            else
                launch_dm_split<T, 256, 32, 64, 32, 2>(A, W, s_in, s_out, C, M, K, N, static_cast<float*>(workspace),
                                                       p.splits, p.split_steps, stream);
            break;
        case kModeSplitGroups64:
            launch_dm_split<T, 256, 64, 64, 64, 4, 3, 4>(A, W, s_in, s_out, C, M, K, N, static_cast<float*>(workspace),
                                                         p.splits, p.split_steps, stream);
            break;
        case kModeSplitGroups32:
            launch_dm_split<T, 256, 32, 64, 32, 4, 3, 4>(A, W, s_in, s_out, C, M, K, N, static_cast<float*>(workspace),
                                                         p.splits, p.split_steps, stream);
            break;
    }
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

size_t nq_gemm_onebit_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    return plan_gemm(M, K, N).workspace_bytes;
}

int nq_gemm_onebit(int dtype, const void* A, const uint32_t* w_bits, const void* s_in, const void* s_out, void* C,
                   int64_t M, int64_t K, int64_t N, void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    if (int s = check_onebit("nq_gemm_onebit", dtype, A, w_bits, s_in, s_out, C, M, K, N)) return s;
    if (M == 0 || N == 0) return NQ_OK;
    hipStream_t st = as_stream(stream);
    if (dtype == NQ_F16)
        return launch_gemm<F16>("nq_gemm_onebit", A, w_bits, s_in, s_out, C, M, K, N, workspace, workspace_bytes, st);
    return launch_gemm<BF16>("nq_gemm_onebit", A, w_bits, s_in, s_out, C, M, K, N, workspace, workspace_bytes, st);
}

size_t nq_gemm_nanoquant_workspace_bytes(int64_t M, int64_t n, int64_t r_pad, int64_t m) {
    if (M <= 0 || n <= 0 || r_pad <= 0 || m <= 0) return 0;
    return std::max(plan_gemm(M, n, r_pad).workspace_bytes, plan_gemm(M, r_pad, m).workspace_bytes);
}

int nq_gemm_nanoquant(int dtype, const void* A, const uint32_t* v_bits, const uint32_t* u_bits, const void* s_g,
                      const void* s_l, const void* s_h, void* imm, void* C, int64_t M, int64_t n, int64_t r_pad,
                      int64_t m, void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    if (int s = check_onebit("nq_gemm_nanoquant stage 1", dtype, A, v_bits, s_g, s_l, imm, M, n, r_pad)) return s;
    if (int s = check_onebit("nq_gemm_nanoquant stage 2", dtype, imm, u_bits, nullptr, s_h, C, M, r_pad, m)) return s;
    if (M == 0 || m == 0) return NQ_OK;
    hipStream_t st = as_stream(stream);
    const char* n1 = "nq_gemm_nanoquant stage 1";
    const char* n2 = "nq_gemm_nanoquant stage 2";
    if (r_pad > 0) {
        const int s1 = dtype == NQ_F16
                           ? launch_gemm<F16>(n1, A, v_bits, s_g, s_l, imm, M, n, r_pad, workspace, workspace_bytes, st)
                           : launch_gemm<BF16>(n1, A, v_bits, s_g, s_l, imm, M, n, r_pad, workspace, workspace_bytes, st);
        if (s1) return s1;
    }
    // stage 2 reuses the workspace: the finishing launch of stage 1 has read it by then (same stream).
    // It stops at the last rank column with a nonzero s_l (the rank padding gives exact zeros).
    return dtype == NQ_F16
               ? launch_gemm<F16>(n2, imm, u_bits, nullptr, s_h, C, M, r_pad, m, workspace, workspace_bytes, st, s_l)
               : launch_gemm<BF16>(n2, imm, u_bits, nullptr, s_h, C, M, r_pad, m, workspace, workspace_bytes, st, s_l);
}

}  // extern "C"
