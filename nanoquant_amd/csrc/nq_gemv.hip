// Decode GEMV: y = sat(s_out * (U * ((V * (s_in * x)) * s_mid))) with +-1 factors held as
// half2-ordered sign words (element j of a 32-column block at bit 15 - j/2 + 16*(j%2)).
//
// Two launches on the caller's stream. (A grid-wide barrier inside one launch costs more on
// this part than the gap between two dependent launches: the agent-scope fences write back
// and invalidate each XCD's L2, and same-address atomics from every block serialise.)
//
//   stage 1  h[b, j] = s_mid[j] * sum_k sign(V[j,k]) * s_in[k] * x[b,k]
//   stage 2  y[b, i] = sat(s_out[i] * sum_j sign(U[i,j]) * h[b,j])
//
// The intermediate h lives in the workspace as a pair of bf16 arrays (hi, lo), [batch][kpad],
// with h ~= hi + lo to 16 significant bits and the fp32 exponent range.
//
// Stage 1 (s1_reg_kernel): each thread owns a fixed set of words of V's rows and keeps the
// matching s_in and x pairs in registers for all the rows it visits; a word's sign bit pair
// (15-p, 31-p) is moved onto the sign bits of the (s_in[k], s_in[k+1]) pair and v_dot2 forms
// the exact fp16/bf16 products with an fp32 sum; rows are reduced across a wave with DPP.
//
// Stage 2 (s2_mfma_kernel): v_mfma_f32_16x16x32_bf16 with U's signs as the A operand and
// (hi, lo) as two B operands: lane group g of a wave takes sign pairs 4g..4g+3 of each word,
// each a shift and an or away from a +-1 bf16 pair, and the matrix core does the sum. Batch
// columns ride in the MFMA's N dimension.
//
// Generic kernels (one wave per output row) cover shapes the fast ones do not.
#include <algorithm>

#include "nq_common.h"

namespace nq {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxNB = 8;
constexpr size_t kHeaderBytes = 256;  // reserved at the start of the workspace

// Bit of element e (0..31) of a half2 word.
__device__ inline int half2_bit(int e) { return 15 - (e >> 1) + 16 * (e & 1); }

__device__ inline uint16_t bf16_bits(float v) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v)); }
__device__ inline float bf16_value(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// Store h[b, j] as (hi, lo).
__device__ inline void store_h(uint16_t* __restrict__ z_hi, uint16_t* __restrict__ z_lo, int kpad, int b, int j,
                               float v) {
    const size_t at = static_cast<size_t>(b) * kpad + j;
    const uint16_t hi = bf16_bits(v);
    z_hi[at] = hi;
    z_lo[at] = bf16_bits(v - bf16_value(hi));
}

// Sum over the 64 lanes of a wave with DPP; every lane gets the total.
// quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and row_mirror leave each 16-lane row
// holding its row sum; row_bcast:15 (rows 1, 3) and row_bcast:31 (rows 2, 3) then carry the
// row sums into lane 63.
template <int kCtrl, int kRowMask>
__device__ inline float dpp_step(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, kRowMask, 0xF, false);
    return v + __int_as_float(moved);
}

__device__ inline float wave_sum_dpp(float v) {
    v = dpp_step<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_step<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_step<0x141, 0xF>(v);  // row_half_mirror
    v = dpp_step<0x140, 0xF>(v);  // row_mirror
    v = dpp_step<0x142, 0xA>(v);  // row_bcast:15
    v = dpp_step<0x143, 0xC>(v);  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// --------------------------------------------------------------------------- generic kernels

// Stage 1, one wave per row j < kpad (rows in [r, kpad) store zeros).
template <typename T, int NB, bool kVec>
__global__ __launch_bounds__(kThreads) void gemv_stage1_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ s_in,
                                                               const uint32_t* __restrict__ vbits,
                                                               const uint16_t* __restrict__ s_mid,
                                                               uint16_t* __restrict__ z_hi,
                                                               uint16_t* __restrict__ z_lo, int batch, int n, int r,
                                                               int wn, int kpad) {
    const int lane = threadIdx.x & 63;
    const int j = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (j >= kpad) return;
    const int b0 = blockIdx.y * NB;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    const uint32_t* row = vbits + static_cast<size_t>(j) * wn;
    for (int w = lane; j < r && w < wn; w += 64) {
        const uint32_t bits = __builtin_nontemporal_load(row + w);
        const int k0 = w * 32;
        if (kVec && k0 + 32 <= n) {
            uint32_t sp[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(s_in + k0 + 8 * q);
                sp[4 * q + 0] = v.x;
                sp[4 * q + 1] = v.y;
                sp[4 * q + 2] = v.z;
                sp[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int p = 0; p < 16; ++p) sp[p] ^= (bits << p) & 0x80008000u;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b0 + b < batch) {
                    const uint16_t* xr = x + static_cast<size_t>(b0 + b) * n + k0;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const u32x4 v = *reinterpret_cast<const u32x4*>(xr + 8 * q);
                        acc[b] = T::dot2(sp[4 * q + 0], v.x, acc[b]);
                        acc[b] = T::dot2(sp[4 * q + 1], v.y, acc[b]);
                        acc[b] = T::dot2(sp[4 * q + 2], v.z, acc[b]);
                        acc[b] = T::dot2(sp[4 * q + 3], v.w, acc[b]);
                    }
                }
            }
        } else {
            const int valid = n - k0 < 32 ? n - k0 : 32;
            for (int e = 0; e < valid; ++e) {
                float sv = T::to_float(s_in[k0 + e]);
                if ((bits >> half2_bit(e)) & 1u) sv = -sv;
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    if (b0 + b < batch) acc[b] = fmaf(sv, T::to_float(x[static_cast<size_t>(b0 + b) * n + k0 + e]), acc[b]);
            }
        }
    }
    const float mid = (j < r && s_mid != nullptr) ? T::to_float(s_mid[j]) : 1.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float v = wave_sum_dpp(acc[b]);
        if (lane == 0 && b0 + b < batch) store_h(z_hi, z_lo, kpad, b0 + b, j, j < r ? v * mid : 0.0f);
    }
}

// Stage 2, one wave per row i; lanes stride the row's words.
template <typename T, int NB>
__global__ __launch_bounds__(kThreads) void gemv_stage2_kernel(const uint16_t* __restrict__ z_hi,
                                                               const uint16_t* __restrict__ z_lo,
                                                               const uint32_t* __restrict__ ubits,
                                                               const uint16_t* __restrict__ s_out,
                                                               uint16_t* __restrict__ y, int batch, int m, int wr,
                                                               int kpad) {
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (i >= m) return;
    const int b0 = blockIdx.y * NB;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    const uint32_t* row = ubits + static_cast<size_t>(i) * wr;
    for (int q = lane; q < wr; q += 64) {
        const uint32_t bits = __builtin_nontemporal_load(row + q);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b0 + b < batch) {
                const size_t at = static_cast<size_t>(b0 + b) * kpad + 32 * q;
#pragma unroll 4
                for (int e = 0; e < 32; ++e) {
                    const float v = bf16_value(z_hi[at + e]) + bf16_value(z_lo[at + e]);
                    acc[b] += ((bits >> half2_bit(e)) & 1u) ? -v : v;
                }
            }
        }
    }
    const float so = T::to_float(s_out[i]);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float v = wave_sum_dpp(acc[b]);
        if (lane == 0 && b0 + b < batch) y[static_cast<size_t>(b0 + b) * m + i] = saturate_to<T>(v * so, T::SAT);
    }
}

// --------------------------------------------------------------------------- stage 1, registers

// x and s_in pairs of one 32-column word as 16 dwords each; columns past n read as zero.
template <int NB>
__device__ inline void load_word_pairs(const uint16_t* __restrict__ x, const uint16_t* __restrict__ s_in, int n,
                                       int batch, int b0, int w, uint32_t (&sp)[16], uint32_t (&xp)[NB][16]) {
    const int k0 = w * 32;
    if (k0 + 32 <= n) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(s_in + k0 + 8 * q);
            sp[4 * q + 0] = v.x;
            sp[4 * q + 1] = v.y;
            sp[4 * q + 2] = v.z;
            sp[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b0 + b < batch) {
                const uint16_t* xr = x + static_cast<size_t>(b0 + b) * n + k0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + 8 * q);
                    xp[b][4 * q + 0] = v.x;
                    xp[b][4 * q + 1] = v.y;
                    xp[b][4 * q + 2] = v.z;
                    xp[b][4 * q + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int p = 0; p < 16; ++p) xp[b][p] = 0u;
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < 16; ++p) {
            const int c0 = k0 + 2 * p;
            const uint32_t lo = c0 < n ? s_in[c0] : 0u;
            const uint32_t hi = c0 + 1 < n ? s_in[c0 + 1] : 0u;
            sp[p] = lo | (hi << 16);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint16_t* xr = x + static_cast<size_t>(b0 + b) * n;
                const bool ok = b0 + b < batch;
                const uint32_t xl = ok && c0 < n ? xr[c0] : 0u;
                const uint32_t xh = ok && c0 + 1 < n ? xr[c0 + 1] : 0u;
                xp[b][p] = xl | (xh << 16);
            }
        }
    }
}

// Thread t = (group g, slot u) with tpg = 1 << tpg_log2 threads per group and rg = 256 / tpg
// groups; it owns words u + tpg*k (k < WPT) of rows j0 + g + rg*i (i < RPT) of the block's
// rg*RPT rows. Rows in [r, kpad) store zeros.
template <typename T, int NB, int WPT, int RPT>
__global__ __launch_bounds__(256) void s1_reg_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ s_in,
                                                     const uint32_t* __restrict__ vbits,
                                                     const uint16_t* __restrict__ s_mid, uint16_t* __restrict__ z_hi,
                                                     uint16_t* __restrict__ z_lo, int batch, int n, int r, int wn,
                                                     int kpad, int tpg_log2) {
    __shared__ float part[4][RPT * NB];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int tpg = 1 << tpg_log2;
    const int rg = 256 >> tpg_log2;
    const int g = t >> tpg_log2;
    const int u = t & (tpg - 1);
    const int j0 = blockIdx.x * rg * RPT;
    const int b0 = blockIdx.y * NB;

    uint32_t bits[RPT][WPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int j = j0 + g + rg * i;
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            const int w = u + tpg * k;
            bits[i][k] = (j < r && w < wn) ? __builtin_nontemporal_load(vbits + static_cast<size_t>(j) * wn + w) : 0u;
        }
    }

    // the epilogue's mid scale, fetched with the rest
    const int rows_pb = rg * RPT;
    const int ep_j = j0 + t / NB;
    const float ep_mid = (t < rows_pb * NB && ep_j < r && s_mid != nullptr) ? T::to_float(s_mid[ep_j]) : 1.0f;

    float acc[RPT][NB];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[i][b] = 0.0f;

#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int w = u + tpg * k;
        if (w < wn) {
            uint32_t sp[16];
            uint32_t xp[NB][16];
            load_word_pairs<NB>(x, s_in, n, batch, b0, w, sp, xp);
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
                const uint32_t wb = bits[i][k];
#pragma unroll
                for (int p = 0; p < 16; ++p) {
                    const uint32_t sg = sp[p] ^ ((wb << p) & 0x80008000u);
#pragma unroll
                    for (int b = 0; b < NB; ++b) acc[i][b] = T::dot2(sg, xp[b][p], acc[i][b]);
                }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float v = wave_sum_dpp(acc[i][b]);
            if (lane == 0) part[wave][i * NB + b] = v;
        }
    __syncthreads();
    if (t < rows_pb * NB) {
        const int jj = t / NB;
        const int b = t - jj * NB;
        const int gg = jj % rg;
        const int i = jj / rg;
        const int j = j0 + jj;
        const int waves_per_group = tpg >> 6;
        if (j < kpad && b0 + b < batch) {
            float v = 0.0f;
            if (j < r) {
                for (int wv = gg * waves_per_group; wv < (gg + 1) * waves_per_group; ++wv) v += part[wv][i * NB + b];
                v *= ep_mid;
            }
            store_h(z_hi, z_lo, kpad, b0 + b, j, v);
        }
    }
}

// --------------------------------------------------------------------------- stage 2, MFMA

// One block per 16 rows of U and up to 16 batch columns. Its W waves split the row's words in
// groups of four (wave w takes words 4w..4w+3, 4(w+W).., ...). Lane l: row i0 + l%16 of U
// (A operand) and batch column b0 + l%16 (B operand) for k-slots 8g..8g+7, g = l/16: the
// elements 8g..8g+7 of each 32-element word, i.e. the sign pairs p = 4g + d (bits 15-p and
// 31-p) that a shift by p moves onto the sign bits of a bf16 pair. The B operand is then
// eight consecutive elements of h.
// Everything a block reads from memory goes to LDS first, with 16-byte loads that are all
// issued before any is waited for: the block's rows of U (one contiguous run of words, laid
// out with rows padded to a multiple of four words), the (hi, lo) intermediate of its batch
// columns (one contiguous run in each array) and the output scales. Global loads are
// unconditional (clamped addresses): a load under a branch is waited for where the branch
// merges. Lanes past m or past the batch compute rows or columns that are never stored.
constexpr int kS2MaxWr = 192;

template <typename T, int W>
__global__ __launch_bounds__(W * 64) void s2_mfma_kernel(const uint16_t* __restrict__ z_hi,
                                                         const uint16_t* __restrict__ z_lo,
                                                         const uint32_t* __restrict__ ubits,
                                                         const uint16_t* __restrict__ s_out, uint16_t* __restrict__ y,
                                                         int batch, int m, int wr, int kpad) {
    constexpr int kThreadsK = W * 64;
    constexpr int kTileLoads = (16 * kS2MaxWr / 4 + kThreadsK - 1) / kThreadsK;
    extern __shared__ __attribute__((aligned(16))) uint32_t dyn[];  // [2][ncols][kpad/2]: hi, then lo
    __shared__ f32x4 red[W][64];
    __shared__ __attribute__((aligned(16))) uint32_t tile[16 * kS2MaxWr];  // [16][wr4]
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int i0 = blockIdx.x * 16;
    const int b0 = blockIdx.y * 16;
    const int ncols = min(16, batch - b0);
    const int wr4 = (wr + 3) & ~3;

    // 1. issue every global load
    const int64_t total = static_cast<int64_t>(m) * wr;
    const int64_t vec_end = total & ~static_cast<int64_t>(3);  // 16-byte loads stay below this
    const int64_t base = static_cast<int64_t>(i0) * wr;
    const int nwords = min(16, m - i0) * wr;
    u32x4 tv[kTileLoads];
#pragma unroll
    for (int it = 0; it < kTileLoads; ++it) {
        const int64_t at = min(base + (t + it * kThreadsK) * 4, vec_end - 4);
        tv[it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ubits + at));
    }
    const int zvec = ncols * kpad / 8;  // 16-byte pieces per half
    const u32x4* zsrc_hi = reinterpret_cast<const u32x4*>(z_hi + static_cast<size_t>(b0) * kpad);
    const u32x4* zsrc_lo = reinterpret_cast<const u32x4*>(z_lo + static_cast<size_t>(b0) * kpad);
    constexpr int kZLoads = 2;  // pieces per thread per half issued up front; more are copied after
    u32x4 zvh[kZLoads], zvl[kZLoads];
#pragma unroll
    for (int it = 0; it < kZLoads; ++it) {
        const int v = min(t + it * kThreadsK, zvec - 1);
        zvh[it] = zsrc_hi[v];
        zvl[it] = zsrc_lo[v];
    }
    float so[4];  // branch-free (clamped) so that the four loads issue together
#pragma unroll
    for (int i = 0; i < 4; ++i) so[i] = T::to_float(s_out[min(i0 + 4 * g + i, m - 1)]);

    // 2. LDS: U words with rows padded to wr4 (pad words zero), then h
#pragma unroll
    for (int it = 0; it < kTileLoads; ++it) {
        const int e4 = (t + it * kThreadsK) * 4;
        if (e4 < nwords) {
            const u32x4 v = tv[it];
            const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
            const bool vec_ok = base + e4 + 4 <= vec_end;
#pragma unroll
            for (int z = 0; z < 4; ++z) {
                const int e = e4 + z;
                if (e < nwords) {
                    const int rrow = e / wr;
                    tile[rrow * wr4 + (e - rrow * wr)] = vec_ok ? vv[z] : ubits[base + e];
                }
            }
        }
    }
    if (wr4 != wr)
        for (int e = t; e < 16 * (wr4 - wr); e += kThreadsK) {
            const int rrow = e / (wr4 - wr);
            tile[rrow * wr4 + wr + (e - rrow * (wr4 - wr))] = 0u;
        }
    u32x4* zdst = reinterpret_cast<u32x4*>(dyn);
#pragma unroll
    for (int it = 0; it < kZLoads; ++it) {
        const int v = t + it * kThreadsK;
        if (v < zvec) {
            zdst[v] = zvh[it];
            zdst[zvec + v] = zvl[it];
        }
    }
    for (int v = t + kZLoads * kThreadsK; v < zvec; v += kThreadsK) {
        zdst[v] = zsrc_hi[v];
        zdst[zvec + v] = zsrc_lo[v];
    }
    __syncthreads();

    // 3. MFMAs, four words at a time: one 16-byte read of words, eight of h, 2 VALU ops per
    //    A dword, two accumulators (hi, lo)
    const int zc = min(c, ncols - 1);
    const uint32_t* zrow_hi = dyn + zc * (kpad / 2) + 4 * g;
    const uint32_t* zrow_lo = dyn + (ncols + zc) * (kpad / 2) + 4 * g;
    const uint32_t* trow = tile + c * wr4;
    const int sh = 4 * g;
    f32x4 ah = f32x4{0.f, 0.f, 0.f, 0.f}, al = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int q0 = 4 * wave; q0 < wr; q0 += 4 * W) {
        const u32x4 w4 = *reinterpret_cast<const u32x4*>(trow + q0);
        u32x4 bh[4], bl[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int q = min(q0 + k, wr - 1);
            bh[k] = *reinterpret_cast<const u32x4*>(zrow_hi + 16 * q);
            bl[k] = *reinterpret_cast<const u32x4*>(zrow_lo + 16 * q);
        }
        const uint32_t ws[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (q0 + k < wr) {
                const uint32_t w = ws[k] << sh;
                u32x4 a;
                a.x = 0x3F803F80u | (w & 0x80008000u);
                a.y = 0x3F803F80u | ((w << 1) & 0x80008000u);
                a.z = 0x3F803F80u | ((w << 2) & 0x80008000u);
                a.w = 0x3F803F80u | ((w << 3) & 0x80008000u);
                ah = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                             __builtin_bit_cast(bf16x8, bh[k]), ah, 0, 0, 0);
                al = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                             __builtin_bit_cast(bf16x8, bl[k]), al, 0, 0, 0);
            }
        }
    }
    {
        const f32x4 a0 = ah, a1 = al;
        red[wave][lane] = f32x4{a0.x + a1.x, a0.y + a1.y, a0.z + a1.z, a0.w + a1.w};
    }
    __syncthreads();

    // 4. wave 0 sums over the W waves and stores
    const int col = b0 + c;
    if (wave == 0 && col < batch) {
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const f32x4 p = red[w][lane];
            const float p0 = p.x, p1 = p.y, p2 = p.z, p3 = p.w;
            s[0] += p0;
            s[1] += p1;
            s[2] += p2;
            s[3] += p3;
        }
        // C layout: lane l holds column l%16 and rows 4*(l/16) + i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ro = i0 + 4 * g + i;
            if (ro < m) y[static_cast<size_t>(col) * m + ro] = saturate_to<T>(s[i] * so[i], T::SAT);
        }
    }
}

inline size_t s2_dyn_lds(int ncols, int kpad) { return static_cast<size_t>(ncols) * 2 * kpad * sizeof(uint16_t); }

// --------------------------------------------------------------------------- dispatch

inline int64_t kpad_of(int64_t r) { return ceil_div(r, 32) * 32; }
inline size_t z_bytes(int64_t batch, int64_t r) {
    return (static_cast<size_t>(batch) * static_cast<size_t>(kpad_of(r)) * 2 + 255) / 256 * 256;
}

struct GemvArgs {
    const uint16_t* x;
    const uint16_t* s_in;
    const uint32_t* v_bits;
    const uint16_t* s_mid;
    const uint32_t* u_bits;
    const uint16_t* s_out;
    uint16_t* y;
    int batch, n, r, m, wn, wr, kpad;
    uint16_t* z_hi;
    uint16_t* z_lo;
    hipStream_t stream;
};

template <typename T, int NB>
void launch_stage1_generic(const GemvArgs& a) {
    const dim3 g1(static_cast<unsigned>(ceil_div(a.kpad, kWaves)), static_cast<unsigned>(ceil_div(a.batch, NB)));
    const bool vec = (a.n % 8 == 0) && aligned(a.x, 16) && aligned(a.s_in, 16);
    if (vec)
        gemv_stage1_kernel<T, NB, true><<<g1, kThreads, 0, a.stream>>>(a.x, a.s_in, a.v_bits, a.s_mid, a.z_hi, a.z_lo,
                                                                        a.batch, a.n, a.r, a.wn, a.kpad);
    else
        gemv_stage1_kernel<T, NB, false><<<g1, kThreads, 0, a.stream>>>(a.x, a.s_in, a.v_bits, a.s_mid, a.z_hi,
                                                                         a.z_lo, a.batch, a.n, a.r, a.wn, a.kpad);
}

template <typename T, int NB>
void launch_stage2_generic(const GemvArgs& a) {
    const dim3 g2(static_cast<unsigned>(ceil_div(a.m, kWaves)), static_cast<unsigned>(ceil_div(a.batch, NB)));
    gemv_stage2_kernel<T, NB><<<g2, kThreads, 0, a.stream>>>(a.z_hi, a.z_lo, a.u_bits, a.s_out, a.y, a.batch, a.m,
                                                             a.wr, a.kpad);
}

template <typename T, int NB, int WPT>
void launch_s1_reg(const GemvArgs& a, int tpg_log2) {
    const int rg = 256 >> tpg_log2;
    // two rows per thread when that still gives a full wave of blocks, else four
    const bool two = ceil_div(a.kpad, rg * 2) >= 256;
    const int rows_pb = rg * (two ? 2 : 4);
    const dim3 grid(static_cast<unsigned>(ceil_div(a.kpad, rows_pb)), static_cast<unsigned>(ceil_div(a.batch, NB)));
    if (two)
        s1_reg_kernel<T, NB, WPT, 2><<<grid, 256, 0, a.stream>>>(a.x, a.s_in, a.v_bits, a.s_mid, a.z_hi, a.z_lo,
                                                                 a.batch, a.n, a.r, a.wn, a.kpad, tpg_log2);
    else
        s1_reg_kernel<T, NB, WPT, 4><<<grid, 256, 0, a.stream>>>(a.x, a.s_in, a.v_bits, a.s_mid, a.z_hi, a.z_lo,
                                                                 a.batch, a.n, a.r, a.wn, a.kpad, tpg_log2);
}

template <typename T>
void launch_stage1(const GemvArgs& a) {
    const bool fast = (a.n % 8 == 0) && aligned(a.x, 16) && aligned(a.s_in, 16) && a.wn <= 1024;
    if (!fast) {
        if (a.batch <= 1) launch_stage1_generic<T, 1>(a);
        else if (a.batch <= 2) launch_stage1_generic<T, 2>(a);
        else if (a.batch <= 4) launch_stage1_generic<T, 4>(a);
        else launch_stage1_generic<T, kMaxNB>(a);
        return;
    }
    const int wpt = a.wn <= 256 ? 1 : (a.wn <= 512 ? 2 : 4);
    const int slots = static_cast<int>(ceil_div(a.wn, wpt));
    const int tpg_log2 = slots <= 64 ? 6 : (slots <= 128 ? 7 : 8);
    // batch rows per pass: registers hold WPT * NB * 16 x dwords, keep that <= 64
    const int nb_cap = 4 / wpt;
    const int nb = a.batch >= 4 && nb_cap >= 4 ? 4 : (a.batch >= 2 && nb_cap >= 2 ? 2 : 1);
    if (wpt == 1) {
        if (nb == 4) launch_s1_reg<T, 4, 1>(a, tpg_log2);
        else if (nb == 2) launch_s1_reg<T, 2, 1>(a, tpg_log2);
        else launch_s1_reg<T, 1, 1>(a, tpg_log2);
    } else if (wpt == 2) {
        if (nb == 2) launch_s1_reg<T, 2, 2>(a, tpg_log2);
        else launch_s1_reg<T, 1, 2>(a, tpg_log2);
    } else {
        launch_s1_reg<T, 1, 4>(a, tpg_log2);
    }
}

template <typename T, int W>
void launch_s2_mfma(const GemvArgs& a) {
    const dim3 grid(static_cast<unsigned>(ceil_div(a.m, 16)), static_cast<unsigned>(ceil_div(a.batch, 16)));
    const size_t lds = s2_dyn_lds(std::min(16, a.batch), a.kpad);
    static const bool lds_ok = [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(&s2_mfma_kernel<T, W>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024) == hipSuccess;
    }();
    (void)lds_ok;
    s2_mfma_kernel<T, W><<<grid, W * 64, lds, a.stream>>>(a.z_hi, a.z_lo, a.u_bits, a.s_out, a.y, a.batch, a.m, a.wr,
                                                          a.kpad);
}

template <typename T>
void launch_stage2(const GemvArgs& a) {
    const bool fast = aligned(a.z_hi, 16) && aligned(a.z_lo, 16) && aligned(a.u_bits, 16) && a.wr <= kS2MaxWr &&
                      static_cast<int64_t>(a.m) * a.wr >= 4 && s2_dyn_lds(std::min(16, a.batch), a.kpad) <= 96 * 1024;
    if (!fast) {
        if (a.batch <= 1) launch_stage2_generic<T, 1>(a);
        else if (a.batch <= 2) launch_stage2_generic<T, 2>(a);
        else if (a.batch <= 4) launch_stage2_generic<T, 4>(a);
        else launch_stage2_generic<T, kMaxNB>(a);
        return;
    }
    if (a.wr <= 64) launch_s2_mfma<T, 4>(a);
    else launch_s2_mfma<T, 8>(a);
}

template <typename T>
int run_gemv(const GemvArgs& a) {
    if (a.kpad > 0) {
        launch_stage1<T>(a);
        if (int s = check_launch("nq_gemv stage 1")) return s;
    }
    launch_stage2<T>(a);
    return check_launch("nq_gemv stage 2");
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" {

size_t nq_gemv_workspace_bytes(int64_t batch, int64_t n, int64_t r, int64_t m) {
    (void)n;
    (void)m;
    if (batch < 0 || r < 0) return 0;
    return kHeaderBytes + 2 * z_bytes(batch, r);
}

int nq_gemv(int dtype, const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid,
            const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n, int64_t r, int64_t m,
            void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "nq_gemv: unsupported dtype %d", dtype);
    if (batch < 0 || n < 0 || r < 0 || m < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_gemv: negative size");
    if (n > INT32_MAX / 2 || r > INT32_MAX / 2 || m > INT32_MAX / 2 || batch > INT32_MAX / 2 ||
        batch * kpad_of(r) > INT32_MAX / 2)
        return fail(NQ_ERR_UNSUPPORTED, "nq_gemv: sizes beyond 2^30 are not supported");
    if (batch == 0 || m == 0) return NQ_OK;
    if (!x || !s_in || !v_bits || !u_bits || !s_out || !y || !workspace)
        return fail(NQ_ERR_INVALID_ARGUMENT, "nq_gemv: null pointer");
    if (!aligned(workspace, 256)) return fail(NQ_ERR_ALIGNMENT, "nq_gemv: workspace must be 256-byte aligned");
    if (!aligned(x, 2) || !aligned(s_in, 2) || !aligned(s_out, 2) || !aligned(y, 2) || !aligned(v_bits, 4) ||
        !aligned(u_bits, 4) || (s_mid && !aligned(s_mid, 2)))
        return fail(NQ_ERR_ALIGNMENT, "nq_gemv: misaligned operand");
    const size_t need = nq_gemv_workspace_bytes(batch, n, r, m);
    if (workspace_bytes < need)
        return fail(NQ_ERR_WORKSPACE, "nq_gemv: workspace has %zu bytes, needs %zu", workspace_bytes, need);
    GemvArgs a;
    a.x = static_cast<const uint16_t*>(x);
    a.s_in = static_cast<const uint16_t*>(s_in);
    a.v_bits = v_bits;
    a.s_mid = static_cast<const uint16_t*>(s_mid);
    a.u_bits = u_bits;
    a.s_out = static_cast<const uint16_t*>(s_out);
    a.y = static_cast<uint16_t*>(y);
    a.batch = static_cast<int>(batch);
    a.n = static_cast<int>(n);
    a.r = static_cast<int>(r);
    a.m = static_cast<int>(m);
    a.wn = static_cast<int>(ceil_div(n, 32));
    a.wr = static_cast<int>(ceil_div(r, 32));
    a.kpad = static_cast<int>(kpad_of(r));
    char* base = static_cast<char*>(workspace) + kHeaderBytes;
    a.z_hi = reinterpret_cast<uint16_t*>(base);
    a.z_lo = reinterpret_cast<uint16_t*>(base + z_bytes(batch, r));
    a.stream = as_stream(stream);
    return dtype == NQ_F16 ? run_gemv<F16>(a) : run_gemv<BF16>(a);
}

}  // extern "C"
