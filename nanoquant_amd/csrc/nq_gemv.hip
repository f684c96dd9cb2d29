// Decode GEMV: y = sat(s_out * (U * ((V * (s_in * x)) * s_mid))) with +-1 factors held as
// half2-ordered sign words (element e of a 32-column block at bit 15 - e/2 + 16*(e%2)).
//
// Two launches on the caller's stream:
//   stage 1  h[b, j] = s_mid[j] * sum_k sign(V[j,k]) * s_in[k] * x[b,k]
//   stage 2  y[b, i] = sat(s_out[i] * sum_j sign(U[i,j]) * h[b,j])
// A grid-wide barrier inside one launch costs more on this part than the gap between two
// dependent launches (same-address device-scope atomics from every block serialise, and the
// agent-scope fences write back and invalidate each XCD's L2), so the stages stay separate.
//
// The intermediate h lives in the workspace as a pair of bf16 arrays (hi, lo), each
// [batch][zpitch]: h ~= hi + lo to 16 significant bits with the fp32 exponent range. Columns
// [r, zpitch) are zero (stage 1 writes them every call), so stage 2 may read past the rank.
//
// What bounds these kernels at decode sizes is latency and instruction issue, not HBM
// bandwidth: a 3 MB read is ~0.4 us of bandwidth against ~2 us of launch plus memory latency.
// So every global load of a kernel is issued before the first use (unconditional loads from
// clamped addresses; __builtin_amdgcn_sched_barrier keeps the scheduler from sinking them to
// their uses), nothing waits on a branch, and the per-wave instruction count is kept small.
//
// Stage 1 (s1w_kernel, VALU): a group of WR waves owns R rows of V; each lane holds WPL words
// of a row and the matching s_in and x pairs in registers for all R rows. The sign of s_in is
// moved onto x once, a word's sign pair p then replaces the sign bits of the s_in pair (one
// v_bfi) and v_dot2 adds the two exact products in fp32. Rows are summed with DPP.
//
// Stage 2 (s2t_kernel, MFMA): v_mfma_f32_16x16x32_bf16 with 16 rows of U as A, built from the
// sign words with a shift and a v_and_or per dword, and the intermediate as B, whose columns
// are (batch row, hi or lo): up to 8 batch rows per pass, hi and lo added after the MFMAs. A
// block stages its rows of U and the intermediate in LDS with non-redundant 16-byte loads:
// the number of vector-memory instructions per CU is what this size pays for.
//
// Generic kernels (one wave per output row) cover the shapes the fast ones do not.
#include <algorithm>
#include <cstdint>
#include <mutex>
#include <type_traits>

#include "nq_common.h"

// Phase marks of the fast kernels; empty in the library (a timing build may define them).
#ifndef NQ_STAMP
#define NQ_STAMP(k)
#endif

namespace nq {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxNB = 8;
constexpr size_t kHeaderBytes = 256;  // reserved at the start of the workspace
constexpr uint32_t kSignPair = 0x80008000u;
constexpr uint32_t kBf16OnePair = 0x3F803F80u;

// ceil(2^32 / d): n / d == __umulhi(n, magic) for n * d < 2^32.
__host__ __device__ inline uint32_t div_magic(uint32_t d) {
    return static_cast<uint32_t>(((1ULL << 32) + d - 1) / d);
}

// LDS row stride (words) of s1m_kernel's tile of V rows wn words wide. A multiple of 64 puts the
// 16 rows one MFMA fragment reads in one bank; from 256 words such rows get the odd stride wn + 1
// (Llama-3-70B, 4 batch rows: q/o 12.7 -> 12.2 us, k/v 11.05 -> 10.55, mixed-rank gate 30.3 ->
// 26.9). On 128-word rows the padded staging measured 6% slower at 16 batch rows, and rows whose
// stride does not share banks gain nothing from it; both keep wn. (Four row tiles of padded wide
// rows do not fit the staging buffer; rows whose padded tile would not fit keep wn, so that the
// MFMA kernel still takes them: 1024-word rows at one row tile, 512-word rows at two.)
// s1m_kernel stages up to kS1mMaxStaged dwords in LDS: 16 rows of sign words per row tile, and the
// s_in pairs when they fit too (64 KB, 16 dwords per thread of a 1024-thread block).
constexpr int kS1mMaxStaged = 16 * 16 * 64;
__host__ __device__ inline int s1m_row_stride(int wn, int rt = 1) {
    return rt <= 2 && wn % 64 == 0 && wn >= 256 && 16 * rt * (wn | 1) <= kS1mMaxStaged ? (wn | 1) : wn;
}

// Bit of element e (0..31) of a half2 word.
__device__ inline int half2_bit(int e) { return 15 - (e >> 1) + 16 * (e & 1); }

__device__ inline uint16_t bf16_bits(float v) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v)); }
__device__ inline float bf16_value(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// Store h[b, j] as (hi, lo).
__device__ inline void store_h(uint16_t* __restrict__ z_hi, uint16_t* __restrict__ z_lo, int zpitch, int b, int j,
                               float v) {
    const size_t at = static_cast<size_t>(b) * zpitch + j;
    const uint16_t hi = bf16_bits(v);
    z_hi[at] = hi;
    z_lo[at] = bf16_bits(v - bf16_value(hi));
}

// Zero columns [kpad, zpitch) of batch rows b0 .. b0+nb-1 (with the block's threads).
__device__ inline void zero_h_pad(uint16_t* __restrict__ z_hi, uint16_t* __restrict__ z_lo, int zpitch, int kpad,
                                  int b0, int nb, int batch) {
    const int width = zpitch - kpad;
    for (int e = threadIdx.x; e < width * nb; e += blockDim.x) {
        const int b = e / width;
        if (b0 + b < batch) {
            const size_t at = static_cast<size_t>(b0 + b) * zpitch + kpad + (e - b * width);
            z_hi[at] = 0;
            z_lo[at] = 0;
        }
    }
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
                                                               int wn, int kpad, int zpitch) {
    const int lane = threadIdx.x & 63;
    const int b0 = blockIdx.y * NB;
    if (blockIdx.x == 0) zero_h_pad(z_hi, z_lo, zpitch, kpad, b0, NB, batch);
    const int j = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (j >= kpad) return;
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
            for (int p = 0; p < 16; ++p) sp[p] ^= (bits << p) & kSignPair;
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
        if (lane == 0 && b0 + b < batch) store_h(z_hi, z_lo, zpitch, b0 + b, j, j < r ? v * mid : 0.0f);
    }
}

// Stage 2, one wave per row i; lanes stride the row's words.
template <typename T, int NB>
__global__ __launch_bounds__(kThreads) void gemv_stage2_kernel(const uint16_t* __restrict__ z_hi,
                                                               const uint16_t* __restrict__ z_lo,
                                                               const uint32_t* __restrict__ ubits,
                                                               const uint16_t* __restrict__ s_out,
                                                               uint16_t* __restrict__ y, int batch, int m, int wr,
                                                               int zpitch) {
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
                const size_t at = static_cast<size_t>(b0 + b) * zpitch + 32 * q;
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

// --------------------------------------------------------------------------- item tables
//
// The fast kernels take a table of up to kMaxItems linears launched together (one block
// range per item): the q, k, v projections of an attention layer share their input, so do
// gate and up. A single GEMV is a one-item table.
constexpr int kMaxItems = 4;

struct S1Item {
    const uint32_t* v_bits;
    const uint16_t* s_in;
    const uint16_t* s_mid;  // or nullptr
    uint16_t* z_hi;
    uint16_t* z_lo;
    int r, kpad, zpitch;
    int blocks;  // blockIdx.x < blocks do the item's rows (each item has a grid plane, blockIdx.z)
};

struct S1Table {
    S1Item item[kMaxItems];
    int count;
};

struct S2Item {
    const uint32_t* u_bits;
    const uint16_t* s_out;
    uint16_t* y;
    const uint16_t* resid;  // residual added in the epilogue, or nullptr
    const uint16_t* z_hi;
    const uint16_t* z_lo;
    int m, wr, zpitch;
    int ystride;  // elements between batch rows of y and resid
    int blocks;  // blockIdx.x < blocks do the item's rows (each item has a grid plane, blockIdx.z)
    int rope;         // kEpiRope, kEpiKv: 0 store into y, 1 rotate into y (queries), 2 rotate into cache
                      // (keys), 3 copy into cache (values)
    uint16_t* cache;  // kinds 2 and 3: [batch, m / head_dim, max_len, head_dim]
};

// The rotary step of kEpiRope: position p = *pos (device), cos/sin rows [max_len, head_dim] (null for
// kEpiKv, which rotates nothing).
struct S2Rope {
    const int64_t* pos;
    const uint16_t* cos;
    const uint16_t* sin;
    int head_dim, max_len;
    uint16_t* mask;       // optional: the step's additive causal mask [rows][max_len][groups]
    uint32_t mask_total;  // elements of mask
    int mask_groups;      // query heads per kv head
};

struct S2Table {
    S2Item item[kMaxItems];
    int count;
    S2Rope rope;
};

// The step position of kEpiRope and kEpiKv as a vector (buffer) load. Scalar loads may return out of order,
// so the compiler waits for every outstanding one at the first use of any: this load, which
// follows a pointer from the kernel arguments, would hold up the block's first reads of its item.
// Vector loads are counted in order, and the wait for this one falls where its value is used.
__device__ inline int64_t load_position(const int64_t* pos) {
    const rsrc_t rs = make_rsrc(pos, 8);
    const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b32(rs, 0, 0, 0);
    const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b32(rs, 4, 0, 0);
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Stage-2 epilogues: y = sat(s_out * acc); y = resid + that (rounded as two T operations);
// gated pair (items 0 and 1 over the same rows): y0 = silu(gate) * up, each a T value;
// kEpiStoreOne is kEpiStore for a one-item table (no item lookup); kEpiRope: the q, k, v
// projections of a decode step with the rotary embedding at position p applied to q and k, q stored
// to y, k and v written into their caches at row p.
// kEpiKv: the same three projections with no rotation, q and k stored to y, v written into its
// cache at row p (S2Item::rope 0 and 3).
enum Epilogue { kEpiStore = 0, kEpiResidual = 1, kEpiGated = 2, kEpiStoreOne = 3, kEpiRope = 4, kEpiKv = 5 };

// The item of this block: a table launch gives each item a grid plane of its own (blockIdx.z), so
// the item's fields are one round of scalar loads at an offset known when the wave starts. (A
// single plane, the item found by comparing blockIdx.x with the items' first blocks, took several
// dependent rounds of scalar loads: ~0.5-0.8 us of each launch.) Blocks of a plane past the item's
// own count exit at once (item_done).
template <typename Item, typename Table>
__device__ inline Item pick_item(const Table& tab) {
    return tab.item[blockIdx.z];
}
template <typename Item>
__device__ inline bool item_done(const Item& it) {
    return static_cast<int>(blockIdx.x) >= it.blocks;
}

// --------------------------------------------------------------------------- stage 1, VALU rows
//
// Block = G groups of WR waves; group gi owns rows j0 .. j0+R-1 (j0 = block row base + gi*R) of
// its item. Lane p = (wave % WR)*64 + lane of a group holds words
// q_w = p + 64*WR*w (w < WPL) of those rows: consecutive lanes read consecutive words.
// Requires n % 8 == 0 (an 8-column piece is wholly inside or outside a row) and 16-byte
// aligned x and s_in.
//
// Every operand comes through a buffer resource sized to its array (x per batch row), so a
// lane's loads past the row or past the rank return zero: a zero s_in pair makes the lane's
// products zero, so nothing is clamped or masked. The signs of a word's pair p are the word
// shifted left by p under the sign mask; xor-ing them onto the s_in pair (one v_bitop3) gives
// +-s_in exactly whatever the sign of s_in, and v_dot2 adds the two exact products in fp32.
//
// kNorm folds an RMSNorm of x into the stage: every group also sums x^2 over the whole row
// (the lanes hold all of x anyway) and h is multiplied by rsqrt(sum / n + eps); the norm's
// weight is expected inside s_in.
template <typename T, int NB, int WPL, int WR, int R, int G, bool kNorm, bool kOne>
__global__ __launch_bounds__(G * WR * 64) void s1w_kernel(const S1Table tab, const uint16_t* __restrict__ x, int batch,
                                                          int n, int wn, float eps) {
    constexpr int kGroups = G;
    constexpr int kRows = kGroups * R;
    constexpr int kPartRows = R + (kNorm ? 1 : 0);
    __shared__ float part[kGroups * kPartRows * NB * WR];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int grp = wave / WR;
    const int p = (wave % WR) * 64 + lane;
    const S1Item it = kOne ? tab.item[0] : pick_item<S1Item>(tab);
    if (!kOne && item_done(it)) return;
    const int r = it.r;
    const int j0 = static_cast<int>(blockIdx.x) * kRows + grp * R;
    const int b0 = blockIdx.y * NB;
    NQ_STAMP(0);

    const uint32_t row_bytes = static_cast<uint32_t>(n) * 2u;
    const rsrc_t s_rs = make_rsrc(it.s_in, row_bytes);
    const rsrc_t v_rs = make_rsrc(it.v_bits, static_cast<uint32_t>(r) * static_cast<uint32_t>(wn) * 4u);
    rsrc_t x_rs[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
        x_rs[b] = make_rsrc(x + static_cast<size_t>(min(b0 + b, batch - 1)) * static_cast<size_t>(n),
                            b0 + b < batch ? row_bytes : 0u);
    // the mid scales, raw until the end; without s_mid the (unused) loads read s_in
    const uint16_t* msrc = it.s_mid != nullptr ? it.s_mid : it.s_in;
    const int mlim = (it.s_mid != nullptr ? r : n) - 1;
    uint16_t mid[R];
#pragma unroll
    for (int k = 0; k < R; ++k) mid[k] = msrc[min(j0 + k, mlim)];
    uint32_t sp[WPL][16];
    uint32_t xp[WPL][NB][16];
    // a lane past the row's last word loads nothing (an offset past the resource touches no memory)
    const uint32_t v_end = static_cast<uint32_t>(r) * static_cast<uint32_t>(wn) * 4u;
    uint32_t vb[R][WPL];
    auto load_v = [&]() {
#pragma unroll
        for (int k = 0; k < R; ++k)
#pragma unroll
            for (int w = 0; w < WPL; ++w) {
                const int q = p + 64 * WR * w;
                const uint32_t off =
                    (static_cast<uint32_t>(j0 + k) * static_cast<uint32_t>(wn) + static_cast<uint32_t>(q)) * 4u;
                vb[k][w] = load_b32_stream(v_rs, q < wn ? off : v_end);
            }
    };
    // s_in and x first (from L2), then V's words (from HBM), each in 16- and 4-byte pieces
#pragma unroll
    for (int w = 0; w < WPL; ++w)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t off = (32u * static_cast<uint32_t>(p + 64 * WR * w) + 8u * v) * 2u;
            const u32x4 sv = load_b128(s_rs, off);
            sp[w][4 * v + 0] = sv.x;
            sp[w][4 * v + 1] = sv.y;
            sp[w][4 * v + 2] = sv.z;
            sp[w][4 * v + 3] = sv.w;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const u32x4 xv = load_b128(x_rs[b], off);
                xp[w][b][4 * v + 0] = xv.x;
                xp[w][b][4 * v + 1] = xv.y;
                xp[w][b][4 * v + 2] = xv.z;
                xp[w][b][4 * v + 3] = xv.w;
            }
        }
    __builtin_amdgcn_sched_barrier(0);
    load_v();
    __builtin_amdgcn_sched_barrier(0);

    NQ_STAMP(1);
    // Even and odd pairs accumulate separately and rows are innermost, so consecutive dot2
    // instructions do not wait on each other.
    const uint32_t mask = kSignPair;
    float acc[2][R][NB];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int k = 0; k < R; ++k)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[e][k][b] = 0.0f;
#pragma unroll
    for (int w = 0; w < WPL; ++w)
#pragma unroll
        for (int pp = 0; pp < 16; ++pp)
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const uint32_t a = ((vb[k][w] << pp) & mask) ^ sp[w][pp];
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[pp & 1][k][b] = T::dot2(a, xp[w][b][pp], acc[pp & 1][k][b]);
            }
    NQ_STAMP(2);
    // sum of squares of x (lanes past the row hold zeros)
    float ss[2][NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ss[0][b] = ss[1][b] = 0.0f;
    if (kNorm) {
#pragma unroll
        for (int w = 0; w < WPL; ++w)
#pragma unroll
            for (int pp = 0; pp < 16; ++pp)
#pragma unroll
                for (int b = 0; b < NB; ++b) ss[pp & 1][b] = T::dot2(xp[w][b][pp], xp[w][b][pp], ss[pp & 1][b]);
    }

    if (WR == 1) {
        float rs[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b)
            rs[b] = kNorm ? rsqrtf(wave_sum_dpp(ss[0][b] + ss[1][b]) / static_cast<float>(n) + eps) : 1.0f;
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const int j = j0 + k;
            const float mf = it.s_mid != nullptr ? T::to_float(mid[k]) : 1.0f;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float v = wave_sum_dpp(acc[0][k][b] + acc[1][k][b]) * rs[b];
                if (lane == 0 && j < it.kpad && b0 + b < batch)
                    store_h(it.z_hi, it.z_lo, it.zpitch, b0 + b, j, j < r ? v * mf : 0.0f);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < kPartRows; ++k)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float v = wave_sum_dpp(k < R ? acc[0][k][b] + acc[1][k][b] : ss[0][b] + ss[1][b]);
                if (lane == 0) part[((grp * kPartRows + k) * NB + b) * WR + wave % WR] = v;
            }
        __syncthreads();
        if (lane == 0 && wave % WR == 0) {
            float rs[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                rs[b] = 1.0f;
                if (kNorm) {
                    float v = 0.0f;
#pragma unroll
                    for (int s2 = 0; s2 < WR; ++s2) v += part[((grp * kPartRows + R) * NB + b) * WR + s2];
                    rs[b] = rsqrtf(v / static_cast<float>(n) + eps);
                }
            }
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const int j = j0 + k;
                const float mf = it.s_mid != nullptr ? T::to_float(mid[k]) : 1.0f;
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    float v = 0.0f;
#pragma unroll
                    for (int s2 = 0; s2 < WR; ++s2) v += part[((grp * kPartRows + k) * NB + b) * WR + s2];
                    v *= rs[b];
                    if (j < it.kpad && b0 + b < batch)
                        store_h(it.z_hi, it.z_lo, it.zpitch, b0 + b, j, j < r ? v * mf : 0.0f);
                }
            }
        }
    }
    if (blockIdx.x == 0) zero_h_pad(it.z_hi, it.z_lo, it.zpitch, it.kpad, b0, NB, batch);
    NQ_STAMP(3);
}

// --------------------------------------------------------------------------- stage 1, one batch row
//
// s1l_kernel: one batch row, n % 32 == 0, rows of up to 384 words. Block = G groups of WR waves;
// group gi owns rows j0 .. j0+R-1 (R even), lane p = (wave % WR) * 64 + lane of a group holds words
// q = p + 64 WR w (w < WPL) of those rows, so a row's words are split over the group's WR waves.
//
// Order of the memory work: V's words first (HBM, the long wait), then one DMA of the item's s_in
// and of x into LDS (L2), then the block waits for all of it. In LDS, word q of the two arrays takes
// nine 16-byte slots from 9 q: s_in pieces 0..3 (elements 32 q + 8 v .. +7), x pieces 0..3, one pad.
// A quarter wave reads piece v of 16 consecutive words at a 144-byte stride, which lands in 16
// distinct slots mod 16 (no bank conflict), and each piece is an immediate offset from the word's
// slot. Lanes past the row read a zero word placed after the DMA region (zslot), so their products
// are zero; their loads of V run into the next row or past the array (zeros) and need no clamp.
//
// The arithmetic takes two rows per shift: the rows' words as one 64-bit value shifted left by the
// pair index put each row's pair signs on bits 15 and 31 of its half (the bits the shift carries
// from the low word into the high one land below bit 15 - p and are masked off). One v_bitop3 per
// row xors them onto the s_in pair and v_dot2 adds the two exact products in fp32: 2.5 VALU per
// pair and row instead of 3. The LDS reads of word w + 1 are issued before word w's arithmetic.
//
// kNorm: group 0 also sums x^2 over the words it holds, and h is scaled by rsqrt(sum / n + eps).
// Measured against the VALU kernel with x in LDS (same rotation of 128 weight copies, us per
// launch): n = 11008, r = 1632: 4.53 -> 3.86; n = 4096, r = 1632 / 1120: 2.92 / 2.87 -> 2.67 / 2.62;
// n = 8192, r = 2240 / 512: 4.51 / 3.12 -> 4.26 / 2.81.
constexpr int kS1lMaxWords = 384;

// LDS slot (16 bytes) of the zero word, and the dynamic LDS bytes, of s1l_kernel at wn words.
__host__ __device__ inline int s1l_zero_slot(int wn) { return (9 * wn + 63) / 64 * 64; }
inline size_t s1l_lds_bytes(int wn) { return static_cast<size_t>(s1l_zero_slot(wn) + 9) * 16; }

template <typename T, int WPL, int R, int G, int WR, bool kNorm, bool kOne>
__global__ __launch_bounds__(G * WR * 64) void s1l_kernel(const S1Table tab, const uint16_t* __restrict__ x, int n,
                                                          int wn, float eps) {
    static_assert(R % 2 == 0, "rows go in pairs");
    extern __shared__ __attribute__((aligned(16))) uint32_t sx[];
    __shared__ float part[(G * R + 1) * WR];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int grp = wave / WR, h = wave % WR;
    const S1Item it = kOne ? tab.item[0] : pick_item<S1Item>(tab);
    if (!kOne && item_done(it)) return;
    const int r = it.r;
    const int j0 = static_cast<int>(blockIdx.x) * (G * R) + grp * R;
    const int zslot = s1l_zero_slot(wn);
    NQ_STAMP(0);

    // V's words of this wave's rows
    const rsrc_t v_rs = make_rsrc(it.v_bits, static_cast<uint32_t>(r) * static_cast<uint32_t>(wn) * 4u);
    uint32_t vb[WPL][R];
#pragma unroll
    for (int w = 0; w < WPL; ++w)
#pragma unroll
        for (int k = 0; k < R; ++k)
            vb[w][k] = load_b32_stream(v_rs, (static_cast<uint32_t>(j0 + k) * static_cast<uint32_t>(wn) +
                                              static_cast<uint32_t>(h * 64 + lane + 64 * WR * w)) * 4u);
    uint16_t mid[R];
    const uint16_t* msrc = it.s_mid != nullptr ? it.s_mid : it.s_in;
    const int mlim = (it.s_mid != nullptr ? r : n) - 1;
#pragma unroll
    for (int k = 0; k < R; ++k) mid[k] = msrc[min(j0 + k, mlim)];
    // the DMA of s_in and x: slot l = 9 q + v (each wave's lanes fill 64 consecutive slots; the
    // last round's lanes past the region repeat its last piece into slots below zslot)
    const int slots = 9 * wn;
    const uint32_t magic9 = div_magic(9);
    for (int l0 = wave * 64; l0 < slots; l0 += G * WR * 64) {
        const int l = min(l0 + lane, slots - 1);
        const int q = static_cast<int>(__umulhi(static_cast<uint32_t>(l), magic9));
        const int v = l - 9 * q;
        const uint16_t* src = v < 4 ? it.s_in + 32 * q + 8 * v : (v < 8 ? x + 32 * q + 8 * (v - 4) : x + 32 * q);
        dma16(src, sx + 4 * l0);
    }
    if (t < 36) sx[4 * zslot + t] = 0u;
    wait_vmcnt<0>();
    barrier_keep_dma();
    NQ_STAMP(1);

    const uint32_t mask = kSignPair;
    float acc[2][R];
#pragma unroll
    for (int k = 0; k < R; ++k) acc[0][k] = acc[1][k] = 0.0f;
    float ss[2] = {0.0f, 0.0f};
    u32x4 cur[8], nxt[8];
    auto fetch = [&](u32x4* d, int w) {
        const int q = h * 64 + lane + 64 * WR * w;
        const u32x4* p = reinterpret_cast<const u32x4*>(sx) + (q < wn ? 9 * q : zslot);
#pragma unroll
        for (int v = 0; v < 8; ++v) d[v] = p[v];
    };
    fetch(cur, 0);
#pragma unroll
    for (int w = 0; w < WPL; ++w) {
        if (w + 1 < WPL) fetch(nxt, w + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int pp = 0; pp < 16; ++pp) {
            const uint32_t s = cur[pp >> 2][pp & 3], xv = cur[4 + (pp >> 2)][pp & 3];
#pragma unroll
            for (int k = 0; k < R; k += 2) {
                const uint64_t sh = ((static_cast<uint64_t>(vb[w][k + 1]) << 32) | vb[w][k]) << pp;
                const uint32_t a0 = (static_cast<uint32_t>(sh) & mask) ^ s;
                const uint32_t a1 = (static_cast<uint32_t>(sh >> 32) & mask) ^ s;
                acc[pp & 1][k] = T::dot2(a0, xv, acc[pp & 1][k]);
                acc[pp & 1][k + 1] = T::dot2(a1, xv, acc[pp & 1][k + 1]);
            }
            if (kNorm && grp == 0) ss[pp & 1] = T::dot2(xv, xv, ss[pp & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int v = 0; v < 8; ++v) cur[v] = nxt[v];
    }
    NQ_STAMP(2);

    if (WR == 1 && !kNorm) {
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const int j = j0 + k;
            const float v = wave_sum_dpp(acc[0][k] + acc[1][k]);
            const float mf = it.s_mid != nullptr ? T::to_float(mid[k]) : 1.0f;
            if (lane == 0 && j < it.kpad) store_h(it.z_hi, it.z_lo, it.zpitch, 0, j, j < r ? v * mf : 0.0f);
        }
    } else {
        // the waves' row sums (and group 0's x^2 sums, row G R) through LDS
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const float v = wave_sum_dpp(acc[0][k] + acc[1][k]);
            if (lane == 0) part[(grp * R + k) * WR + h] = v;
        }
        if (kNorm && grp == 0) {
            const float v = wave_sum_dpp(ss[0] + ss[1]);
            if (lane == 0) part[G * R * WR + h] = v;
        }
        __syncthreads();
        if (h == 0 && lane < R) {
            const int j = j0 + lane;
            float v = 0.0f, sq = 0.0f;
#pragma unroll
            for (int s2 = 0; s2 < WR; ++s2) {
                v += part[(grp * R + lane) * WR + s2];
                if (kNorm) sq += part[G * R * WR + s2];
            }
            if (kNorm) v *= rsqrtf(sq / static_cast<float>(n) + eps);
            uint16_t mk = mid[0];
#pragma unroll
            for (int k = 1; k < R; ++k) mk = lane == k ? mid[k] : mk;
            const float mf = it.s_mid != nullptr ? T::to_float(mk) : 1.0f;
            if (j < it.kpad) store_h(it.z_hi, it.z_lo, it.zpitch, 0, j, j < r ? v * mf : 0.0f);
        }
    }
    if (blockIdx.x == 0) zero_h_pad(it.z_hi, it.z_lo, it.zpitch, it.kpad, 0, 1, 1);
    NQ_STAMP(3);
}

// s1b_kernel: s1l_kernel for NB = 2..4 batch rows. Each sign word's decode (the 64-bit shift of a
// row pair and the xor of the pair signs onto the s_in pair) is done once and feeds one v_dot2 per
// batch row, so a batch row costs one dot2 per pair and row on top of the decode (1.5 VALU) instead
// of a pass of its own. LDS per word: s_in pieces 0..3, x pieces 0..3 of each batch row, one pad:
// 4 NB + 5 slots, an odd stride, so the quarter-wave reads stay in distinct slots. The LDS reads go
// a quarter word (one piece of s_in and of each batch row) ahead of the arithmetic.
__host__ __device__ inline int s1b_word_slots(int nb) { return 4 * nb + 5; }
__host__ __device__ inline int s1b_zero_slot(int wn, int nb) { return (s1b_word_slots(nb) * wn + 63) / 64 * 64; }
inline size_t s1b_lds_bytes(int wn, int nb) {
    return static_cast<size_t>(s1b_zero_slot(wn, nb) + s1b_word_slots(nb)) * 16;
}

template <typename T, int WPL, int R, int G, int WR, int NB, bool kNorm, bool kOne>
__global__ __launch_bounds__(G * WR * 64) void s1b_kernel(const S1Table tab, const uint16_t* __restrict__ x, int n,
                                                          int wn, float eps) {
    static_assert(R % 2 == 0, "rows go in pairs");
    static_assert(NB >= 2 && NB <= 4, "two to four batch rows");
    constexpr int S = 4 * NB + 5;  // LDS slots per word
    extern __shared__ __attribute__((aligned(16))) uint32_t sx[];
    __shared__ float part[(G * R + 1) * NB * WR];
    static_assert(sizeof(part) <= 1024, "the static LDS the launch leaves aside");
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int grp = wave / WR, h = wave % WR;
    const S1Item it = kOne ? tab.item[0] : pick_item<S1Item>(tab);
    if (!kOne && item_done(it)) return;
    const int r = it.r;
    const int j0 = static_cast<int>(blockIdx.x) * (G * R) + grp * R;
    const int zslot = s1b_zero_slot(wn, NB);

    // V's words of this wave's rows (as s1l_kernel)
    const rsrc_t v_rs = make_rsrc(it.v_bits, static_cast<uint32_t>(r) * static_cast<uint32_t>(wn) * 4u);
    uint32_t vb[WPL][R];
#pragma unroll
    for (int w = 0; w < WPL; ++w)
#pragma unroll
        for (int k = 0; k < R; ++k)
            vb[w][k] = load_b32_stream(v_rs, (static_cast<uint32_t>(j0 + k) * static_cast<uint32_t>(wn) +
                                              static_cast<uint32_t>(h * 64 + lane + 64 * WR * w)) * 4u);
    uint16_t mid[R];
    const uint16_t* msrc = it.s_mid != nullptr ? it.s_mid : it.s_in;
    const int mlim = (it.s_mid != nullptr ? r : n) - 1;
#pragma unroll
    for (int k = 0; k < R; ++k) mid[k] = msrc[min(j0 + k, mlim)];
    // the DMA of s_in and the batch rows of x: slot l = S q + v (each wave's lanes fill 64
    // consecutive slots; the last round's lanes past the region repeat its last piece into slots
    // below zslot)
    const int slots = S * wn;
    const uint32_t magic = div_magic(S);
    for (int l0 = wave * 64; l0 < slots; l0 += G * WR * 64) {
        const int l = min(l0 + lane, slots - 1);
        const int q = static_cast<int>(__umulhi(static_cast<uint32_t>(l), magic));
        const int v = l - S * q;
        const uint16_t* src;
        if (v < 4) src = it.s_in + 32 * q + 8 * v;
        else if (v < 4 + 4 * NB) src = x + static_cast<size_t>((v - 4) >> 2) * n + 32 * q + 8 * ((v - 4) & 3);
        else src = x + 32 * q;  // the pad slot: any valid piece
        dma16(src, sx + 4 * l0);
    }
    if (t < 4 * S) sx[4 * zslot + t] = 0u;
    wait_vmcnt<0>();
    barrier_keep_dma();

    const uint32_t mask = kSignPair;
    float acc[2][R][NB];
    float ss[2][NB];
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[0][k][b] = acc[1][k][b] = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) ss[0][b] = ss[1][b] = 0.0f;
    // one quarter word: piece v of s_in and of each batch row's x
    u32x4 cs, cx[NB], ns, nx[NB];
    auto fetch = [&](u32x4& ds, u32x4* dx, int w, int v) {
        const int q = h * 64 + lane + 64 * WR * w;
        const u32x4* p = reinterpret_cast<const u32x4*>(sx) + (q < wn ? S * q : zslot);
        ds = p[v];
#pragma unroll
        for (int b = 0; b < NB; ++b) dx[b] = p[4 + 4 * b + v];
    };
    fetch(cs, cx, 0, 0);
#pragma unroll
    for (int w = 0; w < WPL; ++w) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (v + 1 < 4) fetch(ns, nx, w, v + 1);
            else if (w + 1 < WPL) fetch(ns, nx, w + 1, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int pp = 4 * v + e;
                const uint32_t sp = cs[e];
#pragma unroll
                for (int k = 0; k < R; k += 2) {
                    const uint64_t sh = ((static_cast<uint64_t>(vb[w][k + 1]) << 32) | vb[w][k]) << pp;
                    const uint32_t a0 = (static_cast<uint32_t>(sh) & mask) ^ sp;
                    const uint32_t a1 = (static_cast<uint32_t>(sh >> 32) & mask) ^ sp;
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        acc[pp & 1][k][b] = T::dot2(a0, cx[b][e], acc[pp & 1][k][b]);
                        acc[pp & 1][k + 1][b] = T::dot2(a1, cx[b][e], acc[pp & 1][k + 1][b]);
                    }
                }
                if (kNorm && grp == 0) {
#pragma unroll
                    for (int b = 0; b < NB; ++b) ss[pp & 1][b] = T::dot2(cx[b][e], cx[b][e], ss[pp & 1][b]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            cs = ns;
#pragma unroll
            for (int b = 0; b < NB; ++b) cx[b] = nx[b];
        }
    }

    // the waves' sums per (row, batch row) and group 0's x^2 sums per batch row, through LDS
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float v = wave_sum_dpp(acc[0][k][b] + acc[1][k][b]);
            if (lane == 0) part[((grp * R + k) * NB + b) * WR + h] = v;
        }
    if (kNorm && grp == 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float v = wave_sum_dpp(ss[0][b] + ss[1][b]);
            if (lane == 0) part[(G * R * NB + b) * WR + h] = v;
        }
    }
    __syncthreads();
    if (h == 0 && lane < R * NB) {
        const int k = lane / NB, b = lane - (lane / NB) * NB;  // row j0 + k of the group, batch row b
        const int j = j0 + k;
        float v = 0.0f, sq = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < WR; ++s2) {
            v += part[((grp * R + k) * NB + b) * WR + s2];
            if (kNorm) sq += part[(G * R * NB + b) * WR + s2];
        }
        if (kNorm) v *= rsqrtf(sq / static_cast<float>(n) + eps);
        uint16_t mk = mid[0];
#pragma unroll
        for (int kk = 1; kk < R; ++kk) mk = k == kk ? mid[kk] : mk;
        const float mf = it.s_mid != nullptr ? T::to_float(mk) : 1.0f;
        if (j < it.kpad) store_h(it.z_hi, it.z_lo, it.zpitch, b, j, j < r ? v * mf : 0.0f);
    }
    if (blockIdx.x == 0) zero_h_pad(it.z_hi, it.z_lo, it.zpitch, it.kpad, 0, NB, NB);
}

// --------------------------------------------------------------------------- stage 1, MFMA (batches)
//
// For three or more batch rows: v_mfma_f32_16x16x32_{f16,bf16} with A = 16 rows of V x 32 k of
// +-s_in and B = 32 k x 16 batch rows of x, so one pass over V serves 16 batch rows (the VALU
// kernel above takes two per pass). Lane l = (c = l % 16, g = l / 16). For word q of row j0 + c,
// lane group g takes the pairs p = 4g .. 4g+3 (k = 32q + 8g .. +7): the word shifted left by p
// carries pair p's signs on the sign bits of a 16-bit pair, and one xor puts them onto the s_in
// pair of those k. B: lane (c, g) holds x[b0 + c][32q + 8g .. +7]. The NW waves split the words
// of the rows and add their tiles in LDS. Each wave issues the loads of CH words before their
// MFMAs. kNorm sums x^2 of each batch row on the way (the B fragments of the block's lanes cover
// every k of a batch row once) and scales h by rsqrt(mean(x^2) + eps).
template <typename T, int NW, bool kNorm, bool kOne, bool kSinLds, int kLoads, int RT = 1, bool kPad = false>
__global__ __launch_bounds__(NW * 64) void s1m_kernel(const S1Table tab, const uint16_t* __restrict__ x, int batch,
                                                      int n, int wn, float eps) {
    constexpr int CH = 8;
    constexpr int NT = NW * 64;
    // dwords per thread staged: the host picks the smallest of 4, 8, 12, 16 that covers the block's
    // words (a fixed 16 issued up to three quarters of redundant, clamped loads at n = 4096)
    constexpr int kMaxLoads = kLoads;
    // [16 RT][wn] sign words, then (kSinLds) s_in as [n / 2] pairs; wider rows read s_in from global
    // (after the MFMAs the same memory holds the waves' partial tiles). With RT row tiles a block
    // runs 16 RT rows of V against the same 16 batch rows, so each fragment of x it fetches feeds
    // RT MFMAs.
    extern __shared__ uint32_t lds[];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int c = lane & 15;
    const int g = lane >> 4;
    const S1Item it = kOne ? tab.item[0] : pick_item<S1Item>(tab);
    if (!kOne && item_done(it)) return;
    const int r = it.r;
    const int j0 = static_cast<int>(blockIdx.x) * 16 * RT;
    const int b0 = blockIdx.y * 16;
    const uint16_t* xrow = x + static_cast<uint32_t>(min(b0 + c, batch - 1)) * static_cast<uint32_t>(n);
    const bool b_ok = b0 + c < batch;
    const uint32_t mask = kSignPair;
    // rows of V sit vs words apart in LDS; kPad (rows of 256 words or more, see s1m_row_stride) makes
    // the stride odd, since with wn = 256, 896 ... the 16 rows one MFMA fragment reads share a bank
    const int vs = kPad ? (wn | 1) : wn;
    uint32_t* vt = lds;
    uint32_t* si = lds + 16 * RT * vs;

    // 1. stage the block's rows of V (consecutive in memory) and s_in, dword by dword, coalesced;
    //    rows past r repeat the last row (their h is never stored)
    const int vwords = 16 * RT * wn;
    const int total = vwords + (kSinLds ? n / 2 : 0);
    const uint32_t vbase = static_cast<uint32_t>(min(j0, r - 1)) * static_cast<uint32_t>(wn);
    const uint32_t vlast = static_cast<uint32_t>(r) * static_cast<uint32_t>(wn) - 1;
    const uint32_t* s_in32 = reinterpret_cast<const uint32_t*>(it.s_in);
    uint32_t vals[kMaxLoads];
#pragma unroll
    for (int i = 0; i < kMaxLoads; ++i) {
        const int e = min(t + i * NT, total - 1);
        vals[i] = (!kSinLds || e < vwords) ? it.v_bits[min(vbase + static_cast<uint32_t>(e), vlast)]
                                           : s_in32[e - vwords];
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kPad) {
        // word e of the rows goes to row e / wn of the padded tile (a multiply-high: e * wn < 2^32)
        const uint32_t wmagic = div_magic(static_cast<uint32_t>(wn));
#pragma unroll
        for (int i = 0; i < kMaxLoads; ++i) {
            const int e = t + i * NT;
            if (e < total) {
                const int at = e < vwords ? e + (vs - wn) * static_cast<int>(__umulhi(static_cast<uint32_t>(e), wmagic))
                                          : e - vwords + 16 * RT * vs;
                lds[at] = vals[i];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < kMaxLoads; ++i)
            if (t + i * NT < total) lds[t + i * NT] = vals[i];
    }
    __syncthreads();

    // 2. MFMAs: wave w takes words w, w + NW, ...; x comes from global CH words at a time
    f32x4 acc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt][0] = acc[rt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss[2] = {0.0f, 0.0f};
    for (int q0 = wave; q0 < wn; q0 += NW * CH) {
        u32x4 xv[CH], sg[CH];
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int qc = min(q0 + NW * u, wn - 1);
            const int k = min(32 * qc + 8 * g, n - 8);
            xv[u] = *reinterpret_cast<const u32x4*>(xrow + k);
            if (!kSinLds) sg[u] = *reinterpret_cast<const u32x4*>(it.s_in + k);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int q = q0 + NW * u;
            const int qc = min(q, wn - 1);
            const bool ok = q < wn && 32 * q + 8 * g < n;
            const u32x4 sp = kSinLds ? *reinterpret_cast<const u32x4*>(&si[min(16 * qc + 4 * g, n / 2 - 4)]) : sg[u];
            const u32x4 s = ok ? sp : u32x4{0u, 0u, 0u, 0u};
            const u32x4 xb = (ok && b_ok) ? xv[u] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const uint32_t ws = vt[(16 * rt + c) * vs + qc] << (4 * g);
                const u32x4 a = u32x4{s.x ^ (ws & mask), s.y ^ ((ws << 1) & mask), s.z ^ ((ws << 2) & mask),
                                      s.w ^ ((ws << 3) & mask)};
                acc[rt][u & 1] = mfma16x16x32<T>(a, xb, acc[rt][u & 1]);
            }
            if (kNorm) {
                ss[u & 1] = T::dot2(xb.x, xb.x, ss[u & 1]);
                ss[u & 1] = T::dot2(xb.y, xb.y, ss[u & 1]);
                ss[u & 1] = T::dot2(xb.z, xb.z, ss[u & 1]);
                ss[u & 1] = T::dot2(xb.w, xb.w, ss[u & 1]);
            }
        }
    }
    __syncthreads();  // every wave is done with the staged words
    f32x4* red = reinterpret_cast<f32x4*>(lds);                    // [RT][NW][64]
    float* ssr = reinterpret_cast<float*>(lds) + 4 * RT * NW * 64;  // [NW][64]
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        red[(rt * NW + wave) * 64 + lane] = f32x4{acc[rt][0].x + acc[rt][1].x, acc[rt][0].y + acc[rt][1].y,
                                                  acc[rt][0].z + acc[rt][1].z, acc[rt][0].w + acc[rt][1].w};
    if (kNorm) ssr[wave * 64 + lane] = ss[0] + ss[1];
    __syncthreads();

    // 3. wave rt sums the waves' tiles of row tile rt, scales, stores
    if (wave < RT) {
        const int rt = wave;
        f32x4 sum = red[rt * NW * 64 + lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const f32x4 pr = red[(rt * NW + w) * 64 + lane];
            sum = f32x4{sum.x + pr.x, sum.y + pr.y, sum.z + pr.z, sum.w + pr.w};
        }
        float rs = 1.0f;
        if (kNorm) {
            float tot = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int gg = 0; gg < 4; ++gg) tot += ssr[w * 64 + 16 * gg + c];
            rs = rsqrtf(tot / static_cast<float>(n) + eps);
        }
        const float v[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = j0 + 16 * rt + 4 * g + i;
            if (b_ok && j < it.kpad) {
                const float mf = (it.s_mid != nullptr && j < r) ? T::to_float(it.s_mid[j]) : 1.0f;
                store_h(it.z_hi, it.z_lo, it.zpitch, b0 + c, j, j < r ? v[i] * rs * mf : 0.0f);
            }
        }
    }
    if (blockIdx.x == 0) zero_h_pad(it.z_hi, it.z_lo, it.zpitch, it.kpad, b0, 16, batch);
}

// --------------------------------------------------------------------------- stage 2, MFMA
//
// v_mfma_f32_16x16x32_bf16, lane l = (g = l / 16, c = l % 16), one block per 16 rows of U.
// Word q of a row holds 32 elements; lane group g takes elements 8g..8g+7, the half2 pairs
// p = 4g..4g+3, whose signs sit at bits 15-p and 31-p: the word shifted left by p carries
// them on the sign bits of a bf16 pair, and an and-or with (+1, +1) makes the A dword.
//   A: row c of the tile, k-slots of word q (from U's word (i0 + c, q));
//   B: column c = (batch row b0 + c/2, hi or lo = c % 2), elements 32q + 8g .. +7 of h;
//   C: column c, tile rows 4g .. 4g+3.
// At decode sizes the vector-memory instruction count per CU, not bytes, is what a kernel
// pays for, so the block first stages its 16 rows of U (one contiguous run of words) and the
// intermediate of its NB batch rows in LDS with non-redundant 16-byte loads. The 4 waves then
// take words q = wave + 4s (s < QW); words past wr meet the zero columns of h (U's row is
// clamped), so every step is valid and the loop has no branch. Columns of batch rows past the
// batch hold finite values that are never stored. The waves' partial tiles are added in LDS,
// then hi + lo of each batch row (adjacent lanes) and s_out.
//
// With the gated epilogue a block runs two items (gate, up) over the same 16 rows, each with
// its own U tile and intermediate, and stores silu(gate) * up.
//
// RT row tiles per block: the block stages 16 * RT rows of U, and each step's B fragment serves
// RT MFMAs, one per tile; wave t < RT runs tile t's epilogue. With several batch rows per pass
// the staged intermediate (2 * NB rows of up to 128 * QW columns) outweighs the block's words of
// U many times over, and more rows per block stage it fewer times.
template <typename T>
__device__ inline float silu_of(float g) {
    return g / (1.0f + expf(-g));
}

template <typename T, int QW, int NB, int EPI, int RT>
__global__ __launch_bounds__(256) void s2t_kernel(const S2Table tab, int batch) {
    constexpr int NW = 4;
    constexpr int kThr = 256;
    constexpr int P = EPI == kEpiGated ? 2 : 1;  // items per block
    constexpr int kRows = 16 * RT;               // rows of U per block
    static_assert(RT >= 1 && RT <= NW, "one epilogue wave per row tile");
    constexpr int kWords = kRows * NW * QW;  // tile words (wr <= NW * QW)
    constexpr int kUPieces = (kWords / 4 + kThr - 1) / kThr;
    constexpr int kCols = 32 * NW * QW;  // h columns used per batch row (<= zpitch)
    constexpr int kRowPieces = kCols / 8;
    constexpr int kZPieces = (2 * NB * kRowPieces + kThr - 1) / kThr;
    __shared__ __attribute__((aligned(16))) uint32_t tile[P][kWords + 4];
    __shared__ __attribute__((aligned(16))) uint16_t hz[P][2 * NB][kCols];  // [hi rows, then lo rows][column]
    __shared__ f32x4 red[P][RT][NW][64];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int c = lane & 15;
    const int g = lane >> 4;
    S2Item its[P];
    its[0] = (EPI == kEpiGated || EPI == kEpiStoreOne) ? tab.item[0] : pick_item<S2Item>(tab);
    if (P == 2) its[P - 1] = tab.item[1];
    const int64_t p64 = EPI == kEpiRope || EPI == kEpiKv ? load_position(tab.rope.pos) : 0;
    // kEpiRope: the additive causal mask of the step into the attention scores, element (row, p,
    // group) 0 for a cache position p <= the step's position and -inf after it; every thread of
    // the grid takes every nthr-th element, once its block's own stores are issued (a block with no
    // rows of its item does it at once)
    auto write_mask = [&]() {
        if (EPI != kEpiRope || tab.rope.mask == nullptr) return;
        const uint32_t nthr = gridDim.x * gridDim.y * gridDim.z * 256u;
        const uint32_t gid = ((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * 256u + threadIdx.x;
        const uint16_t neg_inf = T::from_float(-__builtin_huge_valf());
        for (uint32_t e = gid; e < tab.rope.mask_total; e += nthr) {
            const int p = static_cast<int>((e / static_cast<uint32_t>(tab.rope.mask_groups)) %
                                           static_cast<uint32_t>(tab.rope.max_len));
            tab.rope.mask[e] = p <= p64 ? uint16_t(0) : neg_inf;
        }
    };
    if (EPI != kEpiGated && EPI != kEpiStoreOne && item_done(its[0])) {
        write_mask();
        return;
    }
    const int m = its[0].m;
    const int wr = its[0].wr;  // gated items share m and wr
    const int i0 = static_cast<int>(blockIdx.x) * kRows;
    const int b0 = blockIdx.y * NB;
    // kEpiRope: tile row r (< 16) holds feature d of a head's first half for r < 8 and its rotary
    // partner d + head_dim / 2 for r >= 8, so the epilogue finds the partner of each value in the
    // lane 32 away (rows 4g .. 4g+3 against 4(g ^ 2) ..): block bi of an item takes features
    // head * head_dim + 8 j + (r % 8) + (r / 8) * head_dim / 2, head = bi / (head_dim / 16),
    // j = bi % (head_dim / 16). Otherwise the tile's rows are rows i0 .. of U in order.
    int f0 = i0, fhalf = 8;
    if (EPI == kEpiRope) {
        const int D = tab.rope.head_dim;
        const int bi = static_cast<int>(blockIdx.x);
        f0 = (bi / (D / 16)) * D + 8 * (bi % (D / 16));
        fhalf = D / 2;
    }
    auto feat = [&](int r) { return f0 + (r & 7) + (r >> 3) * fhalf; };  // row of U of tile row r
    const int re = 16 * min(wave, RT - 1);  // first tile row whose epilogue this wave may run
    NQ_STAMP(0);

    // 1. every global load: the tiles' words as 16-byte pieces, h, the output scales
    const uint32_t total = static_cast<uint32_t>(m) * static_cast<uint32_t>(wr);
    const uint32_t vec_end = total & ~3u;  // the host guarantees total >= 4
    // tile word e is word e of U's run from row f0 for e < 8 wr, else word e - 8 wr of the run from
    // row f0 + fhalf (one contiguous run from row i0 without kEpiRope); runs start at multiples of 8
    // rows, so the 16-byte pieces below never straddle them
    const uint32_t base1 = static_cast<uint32_t>(f0) * static_cast<uint32_t>(wr);
    const uint32_t base2 = static_cast<uint32_t>(f0 + fhalf) * static_cast<uint32_t>(wr);
    const uint32_t split = 8u * static_cast<uint32_t>(wr);
    auto gword = [&](uint32_t e) { return e < split ? base1 + e : base2 + (e - split); };
    const int rows = min(kRows, m - i0);
    const int nwords = rows * wr;
    u32x4 pv[P][kUPieces];
    uint32_t tail_word[P];
    u32x4 zv[P][kZPieces];
    uint16_t so[P][4];  // raw until the epilogue
    // The intermediate's pieces first: they come from L2, and loads return in issue order, so the
    // block can put them in LDS and read its first fragments while U's words (issued after them)
    // are still on their way from HBM.
#pragma unroll
    for (int pi = 0; pi < P; ++pi) {
        const S2Item& it = its[pi];
#pragma unroll
        for (int k = 0; k < kZPieces; ++k) {
            const int pc = min(t + k * kThr, 2 * NB * kRowPieces - 1);
            const int arr = pc / (NB * kRowPieces);
            const int rem = pc - arr * (NB * kRowPieces);
            const int b = rem / kRowPieces;
            const int off = (rem - b * kRowPieces) * 8;
            zv[pi][k] = *reinterpret_cast<const u32x4*>((arr ? it.z_lo : it.z_hi) +
                                                        static_cast<uint32_t>(min(b0 + b, batch - 1)) *
                                                            static_cast<uint32_t>(it.zpitch) +
                                                        off);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // then the output scales and the residual (needed only by the epilogue) and U's words
#pragma unroll
    for (int pi = 0; pi < P; ++pi)
#pragma unroll
        for (int i = 0; i < 4; ++i) so[pi][i] = its[pi].s_out[min(feat(re + 4 * g + i), m - 1)];
    // the residual of this lane's outputs (batch row b0 + c/2, rows i0 + 4g + i)
    uint16_t res[4] = {0, 0, 0, 0};
    if (EPI == kEpiResidual) {
        const uint32_t rb = static_cast<uint32_t>(min(b0 + min(c >> 1, NB - 1), batch - 1));
#pragma unroll
        for (int i = 0; i < 4; ++i)
            res[i] = its[0].resid[rb * static_cast<uint32_t>(its[0].ystride) + min(feat(re + 4 * g + i), m - 1)];
    }
    // pieces past the block's run are not needed: their offset lies past the resource, so they load
    // nothing (zeros)
#pragma unroll
    for (int pi = 0; pi < P; ++pi) {
        const S2Item& it = its[pi];
        const rsrc_t u_rs = make_rsrc(it.u_bits, vec_end * 4u);
#pragma unroll
        for (int k = 0; k < kUPieces; ++k) {
            const int e4 = 4 * (t + k * kThr);
            pv[pi][k] = load_b128_stream(u_rs, e4 < nwords ? gword(static_cast<uint32_t>(e4)) * 4u : vec_end * 4u);
        }
        tail_word[pi] = it.u_bits[min(vec_end + static_cast<uint32_t>(t), total - 1u)];  // words past vec_end
    }
    // the rotary cos/sin entries of this lane's epilogue rows (row p of the tables; p outside the
    // tables reads row 0, and those values are never used)
    uint16_t rcos[4] = {0, 0, 0, 0}, rsin[4] = {0, 0, 0, 0};
    if (EPI == kEpiRope) {
        const int D = tab.rope.head_dim;
        const size_t prow = p64 >= 0 && p64 < tab.rope.max_len ? static_cast<size_t>(p64) * D : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = feat(re + 4 * g + i) % D;
            rcos[i] = tab.rope.cos[prow + d];
            rsin[i] = tab.rope.sin[prow + d];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. the intermediate into LDS, then each wave's first CH fragments of it
#pragma unroll
    for (int pi = 0; pi < P; ++pi) {
#pragma unroll
        for (int k = 0; k < kZPieces; ++k) {
            const int pc = t + k * kThr;
            if (pc < 2 * NB * kRowPieces) {
                const int row = pc / kRowPieces;  // arr * NB + b
                *reinterpret_cast<u32x4*>(&hz[pi][row][(pc - row * kRowPieces) * 8]) = zv[pi][k];
            }
        }
    }
    __syncthreads();
    const uint32_t mask = kSignPair, one = kBf16OnePair;
    const int sh = 4 * g;
    const int bcol = c >> 1;
    constexpr int CH = QW < 4 ? QW : 4;
    u32x4 bq0[P][CH];
#pragma unroll
    for (int pi = 0; pi < P; ++pi) {
        const uint16_t* hsrc = &hz[pi][(c & 1) * NB + min(bcol, NB - 1)][8 * g];
#pragma unroll
        for (int s = 0; s < CH; ++s) bq0[pi][s] = *reinterpret_cast<const u32x4*>(hsrc + 32 * (wave + NW * s));
    }
    __builtin_amdgcn_sched_barrier(0);
    //    then U's words; vec_end and base + e4 are multiples of 4, so a piece lies wholly below
    //    vec_end or wholly past it, and words past it come from tail_word
#pragma unroll
    for (int pi = 0; pi < P; ++pi) {
#pragma unroll
        for (int k = 0; k < kUPieces; ++k) {
            const int e4 = 4 * (t + k * kThr);
            if (e4 < nwords && gword(static_cast<uint32_t>(e4)) + 4 <= vec_end)
                *reinterpret_cast<u32x4*>(tile[pi] + e4) = pv[pi][k];
        }
        if (t < 3) {
            const uint32_t w = vec_end + t;
            const uint32_t n1 = min(split, static_cast<uint32_t>(nwords));
            if (w < total && w >= base1 && w < base1 + n1) tile[pi][w - base1] = tail_word[pi];
            else if (w < total && nwords > static_cast<int>(split) && w >= base2 && w < base2 + (nwords - split))
                tile[pi][split + (w - base2)] = tail_word[pi];
        }
    }
    __syncthreads();
    NQ_STAMP(1);

    // 3. MFMAs
    // The LDS operands of step s + CH are read right after step s's MFMA is issued, so each read
    // has CH steps to land; the fences keep the scheduler from sinking the reads next to their
    // uses (which made every step wait out an LDS round trip: ~1 us for 14 steps).
    // (4 steps ahead measured 3.96 us on the 11008 x 1632 shape against 4.03-4.05 for 8 and 4.05 for all 13)
#pragma unroll
    for (int pi = 0; pi < P; ++pi) {
        f32x4 acc[RT][2];
        const uint32_t* trow[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            acc[rt][0] = acc[rt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
            trow[rt] = tile[pi] + min(16 * rt + c, rows - 1) * wr;
        }
        const uint16_t* hsrc = &hz[pi][(c & 1) * NB + min(bcol, NB - 1)][8 * g];
        u32x4 bq[CH];
        uint32_t wq[RT][CH];
#pragma unroll
        for (int s = 0; s < CH; ++s) {
            const int q = wave + NW * s;
            bq[s] = bq0[pi][s];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) wq[rt][s] = trow[rt][min(q, wr - 1)];
        }
        __builtin_amdgcn_sched_barrier(0);
        NQ_STAMP(4);
#pragma unroll
        for (int s = 0; s < QW; ++s) {
            const int j = s % CH;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const uint32_t w = wq[rt][j] << sh;
                const u32x4 a = u32x4{and_or(w, mask, one), and_or(w << 1, mask, one), and_or(w << 2, mask, one),
                                      and_or(w << 3, mask, one)};
                acc[rt][s & 1] = mfma16x16x32<BF16>(a, bq[j], acc[rt][s & 1]);
            }
            if (s + CH < QW) {
                const int q = wave + NW * (s + CH);
                bq[j] = *reinterpret_cast<const u32x4*>(hsrc + 32 * q);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) wq[rt][j] = trow[rt][min(q, wr - 1)];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        NQ_STAMP(5);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            red[pi][rt][wave][lane] = f32x4{acc[rt][0].x + acc[rt][1].x, acc[rt][0].y + acc[rt][1].y,
                                            acc[rt][0].z + acc[rt][1].z, acc[rt][0].w + acc[rt][1].w};
    }
    __syncthreads();
    NQ_STAMP(2);

    // 4. sum the waves' partial tiles, add hi and lo, scale, store (wave t: row tile t)
    if (wave < RT) {
        float v[P][4];
#pragma unroll
        for (int pi = 0; pi < P; ++pi) {
            f32x4 sum = red[pi][wave][0][lane];
#pragma unroll
            for (int w = 1; w < NW; ++w) {
                const f32x4 pr = red[pi][wave][w][lane];
                sum = f32x4{sum.x + pr.x, sum.y + pr.y, sum.z + pr.z, sum.w + pr.w};
            }
            v[pi][0] = sum.x;
            v[pi][1] = sum.y;
            v[pi][2] = sum.z;
            v[pi][3] = sum.w;
        }
        const bool b_ok = (c & 1) == 0 && bcol < NB && b0 + bcol < batch;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // quad_perm [1,0,3,2]: the lo column's value from the neighbouring lane
            float out[P];
#pragma unroll
            for (int pi = 0; pi < P; ++pi) {
                const float lo = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v[pi][i]), 0xB1, 0xF, 0xF, false));
                out[pi] = (v[pi][i] + lo) * T::to_float(so[pi][i]);
            }
            const int row = feat(re + 4 * g + i);
            if (EPI == kEpiRope) {
                // q and k rotated as the unfused path rounds it: T(x cos) + T(rotate_half(x) sin), the
                // partner value from the lane 32 away (every lane takes part in the exchange)
#pragma clang fp contract(off)
                const S2Item& it = its[0];
                const int D = tab.rope.head_dim;
                const uint16_t val = saturate_to<T>(out[0], T::SAT);
                const float x = T::to_float(val);
                const float xp = __shfl_xor(x, 32, 64);
                const int d = row % D;
                const float xr = d < D / 2 ? -xp : xp;
                const uint16_t rot = T::from_float(T::to_float(T::from_float(x * T::to_float(rcos[i]))) +
                                                   T::to_float(T::from_float(xr * T::to_float(rsin[i]))));
                const bool p_ok = p64 >= 0 && p64 < tab.rope.max_len;
                if (b_ok && row < m) {
                    if (it.rope == 0) {
                        its[0].y[static_cast<size_t>(b0 + bcol) * its[0].ystride + row] = val;
                    } else if (it.rope == 1) {
                        its[0].y[static_cast<size_t>(b0 + bcol) * its[0].ystride + row] = p_ok ? rot : uint16_t(0);
                    } else if (p_ok) {
                        const size_t at = ((static_cast<size_t>(b0 + bcol) * (m / D) + row / D) * tab.rope.max_len +
                                           static_cast<size_t>(p64)) * D + d;
                        it.cache[at] = it.rope == 2 ? rot : val;
                    }
                }
                continue;
            }
            if (EPI == kEpiKv) {
                if (b_ok && row < m) {
                    const uint16_t val = saturate_to<T>(out[0], T::SAT);
                    if (its[0].rope != 3) {
                        its[0].y[static_cast<size_t>(b0 + bcol) * its[0].ystride + row] = val;
                    } else if (p64 >= 0 && p64 < tab.rope.max_len) {
                        const int D = tab.rope.head_dim;
                        its[0].cache[((static_cast<size_t>(b0 + bcol) * (m / D) + row / D) * tab.rope.max_len +
                                      static_cast<size_t>(p64)) * D + row % D] = val;
                    }
                }
                continue;
            }
            if (b_ok && row < m) {
                uint16_t val = saturate_to<T>(out[0], T::SAT);
                if (EPI == kEpiResidual) {
                    val = T::from_float(T::to_float(res[i]) + T::to_float(val));
                } else if (EPI == kEpiGated) {
                    const float gate = T::to_float(val);
                    const float up = T::to_float(saturate_to<T>(out[P - 1], T::SAT));
                    val = T::from_float(T::to_float(T::from_float(silu_of<T>(gate))) * up);
                }
                its[0].y[static_cast<size_t>(b0 + bcol) * its[0].ystride + row] = val;
            }
        }
    }
    write_mask();
    NQ_STAMP(3);
}

// --------------------------------------------------------------------------- stage 2, batched
//
// For many batch rows: s2t_kernel makes one pass over U per 8 batch rows, decoding U and staging
// the intermediate again on each. s2b_kernel decodes each A fragment (16 rows of U x 32 k, as in
// s2t_kernel) once for all of its block's batch rows. Block = 4 waves in a WR x (4 / WR) grid: wave
// (wr, wc) runs row tiles wr + WR * j (j < RTW) of the block's RT = WR * RTW tiles of 16 rows
// against column tiles wc * CTW + j2 (j2 < CTW), each 8 batch rows x (hi, lo) as in s2t_kernel.
//
// The block's words of U reach LDS by DMA first, row-major as in memory. The intermediate streams
// through three LDS buffers in chunks of KC words of k (32 KC columns of every batch row, hi and
// lo), each fetched by DMA two chunks ahead, so no register holds a chunk in flight. LDS row
// R = 2 b + (0 hi, 1 lo) of a chunk holds 4 KC pieces of 16 bytes, piece p at slot p ^ (R % 8): the
// eight lanes of a fragment read that share a bank group read eight different rows.
//
// Every chunk runs all of its KC steps: past the rank, the intermediate's columns [kpad, zpitch)
// are zero (stage 1 writes them), and the host only picks KC that keep 32 KC * chunks <= zpitch,
// so the words read past a row (the next row's, or the tile's padding) multiply zeros.
struct S2bArgs {
    const uint32_t* u_bits;
    const uint16_t* s_out;
    uint16_t* y;
    const uint16_t* z_hi;
    const uint16_t* z_lo;
    int m, wr, zpitch, batch, chunks;
    int u_slots;      // LDS dwords of the U tile (its rows' words and the padding, whole DMAs)
    int store8;       // y takes 8-byte stores of four rows (m % 4 == 0, y 8-byte aligned)
};

template <int RT, int WR, int CTW, int KC>
struct S2bShape {
    static constexpr int kRTW = RT / WR;
    static constexpr int kWC = 4 / WR;
    static constexpr int kRows = 16 * RT;            // rows of U per block
    static constexpr int kBatch = 8 * kWC * CTW;      // batch rows per block
    static constexpr int kPieces = 4 * KC;            // 16-byte pieces per LDS row of a chunk
    static constexpr int kSlots = 2 * kBatch * kPieces;  // 16-byte slots per chunk buffer
    static_assert(RT % WR == 0 && (WR == 1 || WR == 2 || WR == 4), "row tiles split evenly over WR");
    static_assert(KC == 2 || KC == 4, "two or four words of k per chunk");
    static_assert(kSlots % 256 == 0, "whole DMAs per thread");
};

template <typename T, int RT, int WR, int CTW, int KC>
__global__ __launch_bounds__(256) void s2b_kernel(const S2bArgs a) {
    using S = S2bShape<RT, WR, CTW, KC>;
    constexpr int RTW = S::kRTW;
    constexpr int NP = S::kPieces;
    constexpr int kDma = S::kSlots / 256;  // 16-byte DMAs per thread per chunk
    // distinct LDS arrays: the compiler's wait before a buffer's reads then counts only the DMAs
    // into that buffer, not the ones in flight into the others
    __shared__ __attribute__((aligned(16))) uint32_t hb0[4 * S::kSlots], hb1[4 * S::kSlots], hb2[4 * S::kSlots];
    extern __shared__ __attribute__((aligned(16))) uint32_t ut[];  // the U tile (a.u_slots dwords)
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int c = lane & 15;
    const int g = lane >> 4;
    const int wrow = wave % WR;
    const int wcol = wave / WR;
    const int i0 = static_cast<int>(blockIdx.x) * S::kRows;
    const int bb = static_cast<int>(blockIdx.y) * S::kBatch;
    NQ_STAMP(0);

    // 1. DMA: the rows' words (clamped to the last word of U: slots past the rows are never used
    //    for a stored output), then the first two chunks of the intermediate
    const uint32_t wtotal = static_cast<uint32_t>(a.m) * static_cast<uint32_t>(a.wr);
    const uint32_t wbase = static_cast<uint32_t>(i0) * static_cast<uint32_t>(a.wr);
    for (int l0 = wave * 64; l0 < a.u_slots; l0 += 256)
        dma4(a.u_bits + min(wbase + static_cast<uint32_t>(l0 + lane), wtotal - 1u), ut + l0);
    // this thread's DMA sources: LDS row R = l / NP of slot l, batch row clamped below batch
    const uint16_t* hsrc[kDma];
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
        const int l = j * 256 + t;
        const int R = l / NP;
        const int p = (l % NP) ^ (R & 7);
        const uint32_t b = static_cast<uint32_t>(min(bb + (R >> 1), a.batch - 1));
        hsrc[j] = ((R & 1) ? a.z_lo : a.z_hi) + b * static_cast<uint32_t>(a.zpitch) + 8 * p;
    }
    auto issue = [&](int ci, uint32_t* buf) {
        const uint32_t k0 = static_cast<uint32_t>(ci) * 32u * KC;
#pragma unroll
        for (int j = 0; j < kDma; ++j) dma16(hsrc[j] + k0, buf + (j * 256 + wave * 64) * 4);
    };
    issue(0, hb0);
    issue(min(1, a.chunks - 1), hb1);
    // the output scales of this lane's rows (needed only by the epilogue)
    uint16_t so[RTW][4];
#pragma unroll
    for (int j = 0; j < RTW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) so[j][i] = a.s_out[min(i0 + 16 * (wrow + WR * j) + 4 * g + i, a.m - 1)];
    wait_vmcnt<kDma>();  // the words and chunk 0 (chunk 1's DMAs may still be in flight)
    barrier_keep_dma();
    NQ_STAMP(1);

    // 2. MFMAs, chunk by chunk
    const uint32_t mask = kSignPair, one = kBf16OnePair;
    const int sh = 4 * g;
    f32x4 acc[RTW][CTW];
#pragma unroll
    for (int j = 0; j < RTW; ++j)
#pragma unroll
        for (int j2 = 0; j2 < CTW; ++j2) acc[j][j2] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t* urow[RTW];
#pragma unroll
    for (int j = 0; j < RTW; ++j) urow[j] = ut + (16 * (wrow + WR * j) + c) * a.wr;
    const int hrow = (16 * wcol * CTW + c) * NP;  // LDS row of column tile wcol * CTW, this lane's column
    const int swz = c & 7;                         // = R % 8 for every column tile of the lane
    struct Ops {
        u32x4 bf[CTW];
        uint32_t w[RTW];
    };
    auto fetch = [&](const uint32_t* buf, int q, int s, Ops& o) {
        const int slot = hrow + ((4 * s + g) ^ swz);
#pragma unroll
        for (int j2 = 0; j2 < CTW; ++j2) o.bf[j2] = *reinterpret_cast<const u32x4*>(buf + (slot + 16 * j2 * NP) * 4);
#pragma unroll
        for (int j = 0; j < RTW; ++j) o.w[j] = urow[j][q];
    };
    auto run = [&](const Ops& o) {
#pragma unroll
        for (int j = 0; j < RTW; ++j) {
            const uint32_t w = o.w[j] << sh;
            const u32x4 av = u32x4{and_or(w, mask, one), and_or(w << 1, mask, one), and_or(w << 2, mask, one),
                                   and_or(w << 3, mask, one)};
#pragma unroll
            for (int j2 = 0; j2 < CTW; ++j2) acc[j][j2] = mfma16x16x32<BF16>(av, o.bf[j2], acc[j][j2]);
        }
    };
    // one chunk: DMA chunk ci + 2 into the buffer chunk ci - 1 used (the last chunk again at the
    // end: every step issues the same DMAs, so the wait below always means chunk ci + 1), the
    // chunk's steps with the next step's operands read first, then chunk ci + 1's DMAs, barrier
    auto chunk = [&](const uint32_t* cur, uint32_t* free_buf, int ci) {
        issue(min(ci + 2, a.chunks - 1), free_buf);
        Ops o[2];
        fetch(cur, ci * KC, 0, o[0]);
#pragma unroll
        for (int s = 0; s < KC; ++s) {
            if (s + 1 < KC) fetch(cur, ci * KC + s + 1, s + 1, o[(s + 1) & 1]);
            run(o[s & 1]);
        }
        wait_vmcnt<kDma>();
        barrier_keep_dma();
    };
    int ci = 0;
    for (; ci + 3 <= a.chunks; ci += 3) {
        chunk(hb0, hb2, ci);
        chunk(hb1, hb0, ci + 1);
        chunk(hb2, hb1, ci + 2);
    }
    if (ci < a.chunks) {
        chunk(hb0, hb2, ci);
        if (ci + 1 < a.chunks) chunk(hb1, hb0, ci + 1);
    }
    wait_vmcnt<0>();  // the re-fetches land before the block's LDS is released
    NQ_STAMP(2);

    // 3. lane (c, g) of tile (j, j2) holds rows 4g .. 4g+3 of column c: batch row 8 (wcol CTW + j2)
    //    + c / 2, hi (c even) or lo; the even lane adds its neighbour's lo, scales and stores
#pragma unroll
    for (int j = 0; j < RTW; ++j) {
        const int row = i0 + 16 * (wrow + WR * j) + 4 * g;
#pragma unroll
        for (int j2 = 0; j2 < CTW; ++j2) {
            const int b = bb + 8 * (wcol * CTW + j2) + (c >> 1);
            const float vv[4] = {acc[j][j2].x, acc[j][j2].y, acc[j][j2].z, acc[j][j2].w};
            uint16_t out[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float lo = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(vv[i]), 0xB1, 0xF, 0xF, false));
                out[i] = saturate_to<T>((vv[i] + lo) * T::to_float(so[j][i]), T::SAT);
            }
            if ((c & 1) == 0 && b < a.batch) {
                uint16_t* yp = a.y + static_cast<size_t>(b) * a.m + row;
                if (a.store8 && row + 3 < a.m) {
                    *reinterpret_cast<uint2*>(yp) = uint2{out[0] | (uint32_t(out[1]) << 16), out[2] | (uint32_t(out[3]) << 16)};
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (row + i < a.m) yp[i] = out[i];
                }
            }
        }
    }
    NQ_STAMP(3);
}

// --------------------------------------------------------------------------- stage 1, batched (k split)
//
// For many batch rows on wide rows of V: h[b][j] = s_mid[j] * sum_k sign(V[j][k]) s_in[k] x[b][k]
// as v_mfma_f32_16x16x32_{f16,bf16} tiles with A = 16 rows of V x 32 k of +-s_in (the word shifted
// left by 4g + d carries pair 4g + d's signs; one xor puts them on the s_in pair, as in s1m_kernel)
// and B = 32 k x 16 batch rows of x. sb_kernel gives one block 16 * NW * RTW rows of V and a range
// of kw words of k for up to 16 * CT batch rows: it copies that slice of x, of s_in and the rows'
// words into LDS by DMA in one go, then wave w runs its RTW row tiles against all CT batch tiles,
// decoding each A fragment once for the CT MFMAs that use it. s1m_kernel, by contrast, decodes V
// again for every 16 batch rows and streams all of x through every block of 16 rows.
//
// With one k range the block applies the epilogue; with several, each block stores its raw fp32
// sums to plane grid.y of `part` ([ks][batch][kpad]) and sb_finish1 adds the planes in order (a
// fixed order: the result does not depend on which block finished first).
//
// x slice layout: column c (batch row bb + c; the last column holds s_in) is kw * 4 chunks of 16
// bytes; chunk p of column c holds x's chunk p ^ (c % 8) (kw is even, so the swizzle stays inside
// the column), which spreads the 16 columns one MFMA fragment read touches over the LDS banks. A
// wave's DMA fills 64 consecutive chunks; lanes past the slice fetch a valid chunk again into the
// rounding slack. Words: row i of the block at i * (kw + 1).
//
// Measured (MI355X, graph-replayed, rotating weights; stage 1 alone, us): n = 11008, r = 1632:
// batch 16 / 64 / 128: 12.9 / 18.7 / 27.7 against 14.3 / 26.6 / 51.3 for s1m_kernel with one row
// tile per block (19.0 at 64 rows with two); n = 4096: batch 64 / 128: 11.5 / 15.6 against 8.9 / 13.4
// for s1m_kernel with two and four row tiles, so it runs on wide rows only. A block
// fetches its slice at 35-45 GB/s (phase stamps), so the plan keeps slices small; the same design
// for stage 2 (slices of h, partial sums of y) lost to s2t_kernel at every batch and is not used.
struct SbArgs {
    const uint32_t* words;  // V's words [M][wpr]
    const uint16_t* s_in;   // [wpr * 32]
    const uint16_t* x;      // [batch][ldx]
    const uint16_t* s_mid;  // or nullptr
    uint16_t* z_hi;
    uint16_t* z_lo;
    float* part;            // [ks][batch][kpad] with several k ranges
    int M, wpr, ldx, batch, kw;
    int kpad, zpitch;       // rows >= M give zeros, rows < kpad are stored, columns [kpad, zpitch) zeroed
    uint32_t kw4_magic;     // ceil(2^32 / (4 kw)): l / (4 kw) == umulhi(l, kw4_magic) for the l used here
    uint32_t ws_magic;      // ceil(2^32 / (kw + 1))
};


// Dwords of LDS an sb_kernel block takes (x slice, then words), each part rounded to whole DMAs.
__host__ __device__ inline int sb_xs_dwords(int xcols, int kw) { return (xcols * kw * 4 + 63) / 64 * 64 * 4; }
__host__ __device__ inline int sb_w_dwords(int rows, int kw) { return (rows * (kw + 1) + 63) / 64 * 64; }

template <typename T, int NW, int RTW, int CT>
__global__ __launch_bounds__(NW * 64) void sb_kernel(const SbArgs a) {
    constexpr int BR = 16 * NW * RTW;  // rows of V per block
    constexpr int NCOL = 16 * CT;      // batch rows per block
    constexpr int XCOLS = NCOL + 1;    // + s_in
    extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int c = lane & 15;
    const int g = lane >> 4;
    const int i0 = static_cast<int>(blockIdx.x) * BR;
    const int q0 = static_cast<int>(blockIdx.y) * a.kw;
    const int qn = min(a.kw, a.wpr - q0);
    const int bb = static_cast<int>(blockIdx.z) * NCOL;  // first batch row of the block
    const int kw4 = a.kw * 4;
    uint32_t* xs = smem;
    uint32_t* wl = smem + sb_xs_dwords(XCOLS, a.kw);
    const int wstride = a.kw + 1;
    NQ_STAMP(0);

    // 1. DMA: the x slice and s_in, and the rows' words (divisions by a multiply: the issue loops
    //    are VALU work before the first MFMA). V's words come from HBM and the x slice mostly from
    //    L2: up to 64 batch rows the words go out first, so that part of their longer latency
    //    passes while the slice is issued (same-box A/B, down_proj and Llama-3-70B q/o at 16-64
    //    rows: 1.1-1.9% faster); with 128 rows the larger slice goes first (1.6-1.9% faster so).
    auto dma_slice = [&]() {
        const uint32_t xchunks = static_cast<uint32_t>(XCOLS * kw4);
        const uint32_t kend = static_cast<uint32_t>(a.wpr) * 32u;  // elements of k
        for (uint32_t l0 = static_cast<uint32_t>(wave) * 64u; l0 < xchunks; l0 += NW * 64) {
            const uint32_t l = min(l0 + static_cast<uint32_t>(lane), xchunks - 1u);
            const uint32_t col = __umulhi(l, a.kw4_magic);
            const uint32_t p = l - col * static_cast<uint32_t>(kw4);
            uint32_t k = static_cast<uint32_t>(q0) * 32u + 8u * (p ^ (col & 7u));
            if (k >= kend) k = 0;  // past the last word: never read
            const uint16_t* src;
            if (col == NCOL) {
                src = a.s_in + k;
            } else {
                const uint32_t b = min(static_cast<uint32_t>(bb) + col, static_cast<uint32_t>(a.batch - 1));
                src = a.x + b * static_cast<uint32_t>(a.ldx) + k;
            }
            dma16(src, xs + l0 * 4);
        }
    };
    auto dma_words = [&]() {
        const uint32_t wtotal = static_cast<uint32_t>(BR * wstride);
        const uint32_t qlast = static_cast<uint32_t>(qn - 1);
        const uint32_t rlast = static_cast<uint32_t>(a.M - 1 - i0);  // >= 0: the grid covers rows below M only
        const uint32_t* wbase = a.words + static_cast<uint32_t>(i0) * static_cast<uint32_t>(a.wpr) + static_cast<uint32_t>(q0);
        for (uint32_t l0 = static_cast<uint32_t>(wave) * 64u; l0 < wtotal; l0 += NW * 64) {
            const uint32_t l = min(l0 + static_cast<uint32_t>(lane), wtotal - 1u);
            const uint32_t row = __umulhi(l, a.ws_magic);
            const uint32_t q = min(l - row * static_cast<uint32_t>(wstride), qlast);  // the pad slot repeats a word
            dma4(wbase + min(row, rlast) * static_cast<uint32_t>(a.wpr) + q, wl + l0);
        }
    };
    if constexpr (CT <= 4) {
        dma_words();
        dma_slice();
    } else {
        dma_slice();
        dma_words();
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's DMAs have landed (vmcnt, expcnt and lgkmcnt all zero)
    __syncthreads();
    NQ_STAMP(1);

    // 2. MFMAs over the range: A fragment of row tile rt from word (row 16 rt' + c, q) shifted by 4g
    const uint32_t mask = kSignPair;
    f32x4 acc[RTW * CT];
#pragma unroll
    for (int i = 0; i < RTW * CT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t* wrow = wl + (16 * wave * RTW + c) * wstride;
    const uint32_t* xcol = xs + c * kw4 * 4;
    const uint32_t* scol = xs + NCOL * kw4 * 4;
    const int sw = c & 7;
    const int sh = 4 * g;
    // the LDS operands of word q + 1 are read before word q's MFMAs (two operand sets, the loop
    // unrolled by two so that each set keeps its registers)
    struct Ops {
        u32x4 bf[CT];
        u32x4 s;
        uint32_t w[RTW];
    };
    auto fetch = [&](int q, Ops& o) {
        const int ch = (4 * q + g) ^ sw;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) o.bf[ct] = *reinterpret_cast<const u32x4*>(xcol + (16 * ct * kw4 + ch) * 4);
        o.s = *reinterpret_cast<const u32x4*>(scol + (4 * q + g) * 4);
#pragma unroll
        for (int rt = 0; rt < RTW; ++rt) o.w[rt] = wrow[16 * rt * wstride + q];
    };
    auto run = [&](const Ops& o) {
#pragma unroll
        for (int rt = 0; rt < RTW; ++rt) {
            const uint32_t w = o.w[rt] << sh;
            const u32x4 av = u32x4{o.s.x ^ (w & mask), o.s.y ^ ((w << 1) & mask), o.s.z ^ ((w << 2) & mask),
                                   o.s.w ^ ((w << 3) & mask)};
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) acc[rt * CT + ct] = mfma16x16x32<T>(av, o.bf[ct], acc[rt * CT + ct]);
        }
    };
    Ops o0, o1;
    fetch(0, o0);
    int q = 0;
    for (; q + 1 < qn; q += 2) {
        fetch(q + 1, o1);
        run(o0);
        if (q + 2 < qn) fetch(q + 2, o0);
        run(o1);
    }
    if (q < qn) run(o0);

    // 3. lane (c, g) holds rows 4g .. 4g+3 of each row tile for batch row 16 ct + c. The block's
    //    [batch row][row] tile goes through LDS (rows padded by 4 floats against bank conflicts), so
    //    that every global store below is a run of consecutive rows of one batch row.
    constexpr int OS = BR + 4;
    float* ot = reinterpret_cast<float*>(smem);
    NQ_STAMP(2);
    __syncthreads();  // every wave is done with the slice
#pragma unroll
    for (int rt = 0; rt < RTW; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
            *reinterpret_cast<f32x4*>(ot + (16 * ct + c) * OS + 16 * (wave * RTW + rt) + 4 * g) = acc[rt * CT + ct];
    __syncthreads();
    // 4. stores: 4 consecutive rows per thread, consecutive threads along a batch row
    const bool split = gridDim.y > 1;
    const int nb = min(NCOL, a.batch - bb);
    constexpr int Q = BR / 4;
    for (int e = t; e < nb * Q; e += NW * 64) {
        const int bl = e / Q;
        const int rl = 4 * (e - bl * Q);
        const int row = i0 + rl;
        if (row >= a.kpad) continue;
        const int b = bb + bl;
        const f32x4 v = *reinterpret_cast<const f32x4*>(ot + bl * OS + rl);
        if (split) {
            *reinterpret_cast<f32x4*>(a.part + (static_cast<size_t>(blockIdx.y) * a.batch + b) * a.kpad + row) = v;
        } else {
            const float vv[4] = {v.x, v.y, v.z, v.w};
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = row + i;
                const float mf = (a.s_mid != nullptr && j < a.M) ? T::to_float(a.s_mid[j]) : 1.0f;
                const float h = j < a.M ? vv[i] * mf : 0.0f;
                hi[i] = bf16_bits(h);
                lo[i] = bf16_bits(h - bf16_value(hi[i]));
            }
            const size_t at = static_cast<size_t>(b) * a.zpitch + row;
            *reinterpret_cast<uint2*>(a.z_hi + at) = uint2{hi[0] | (uint32_t(hi[1]) << 16), hi[2] | (uint32_t(hi[3]) << 16)};
            *reinterpret_cast<uint2*>(a.z_lo + at) = uint2{lo[0] | (uint32_t(lo[1]) << 16), lo[2] | (uint32_t(lo[3]) << 16)};
        }
    }
    if (!split && blockIdx.x == 0 && blockIdx.y == 0) zero_h_pad(a.z_hi, a.z_lo, a.zpitch, a.kpad, bb, NCOL, a.batch);
    NQ_STAMP(3);
}

// The k ranges added in order: h[b][j] = s_mid[j] * sum (0 for j >= r), stored as (hi, lo) for
// j < kpad, zeros in [kpad, zpitch). One thread per 4 columns of one batch row.
template <typename T>
__global__ __launch_bounds__(256) void sb_finish1(const SbArgs a, int ks) {
    const int per_row = a.zpitch / 4;
    const int e = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (e >= a.batch * per_row) return;
    const int b = e / per_row;
    const int j0 = 4 * (e - b * per_row);
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (j0 < a.kpad) {
        // the planes' loads go out kBatch at a time before their adds (one dependent load per plane
        // made this launch wait out a memory round trip per plane); the adds keep the order k = 0, 1, ...
        constexpr int kBatch = 16;
        const f32x4* src = reinterpret_cast<const f32x4*>(a.part + static_cast<size_t>(b) * a.kpad + j0);
        const size_t plane = static_cast<size_t>(a.batch) * a.kpad / 4;  // f32x4 per plane
        for (int k0 = 0; k0 < ks; k0 += kBatch) {
            f32x4 pv[kBatch];
#pragma unroll
            for (int i = 0; i < kBatch; ++i)
                pv[i] = k0 + i < ks ? src[static_cast<size_t>(k0 + i) * plane] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                if (k0 + i < ks) {
                    v[0] += pv[i].x;
                    v[1] += pv[i].y;
                    v[2] += pv[i].z;
                    v[3] += pv[i].w;
                }
            }
        }
    }
    uint16_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int j = j0 + i;
        const float mf = (a.s_mid != nullptr && j < a.M) ? T::to_float(a.s_mid[j]) : 1.0f;
        const float h = j < a.M ? v[i] * mf : 0.0f;
        hi[i] = bf16_bits(h);
        lo[i] = bf16_bits(h - bf16_value(hi[i]));
    }
    const size_t at = static_cast<size_t>(b) * a.zpitch + j0;
    *reinterpret_cast<uint2*>(a.z_hi + at) = uint2{hi[0] | (uint32_t(hi[1]) << 16), hi[2] | (uint32_t(hi[3]) << 16)};
    *reinterpret_cast<uint2*>(a.z_lo + at) = uint2{lo[0] | (uint32_t(lo[1]) << 16), lo[2] | (uint32_t(lo[3]) << 16)};
}

// --------------------------------------------------------------------------- plan and dispatch

constexpr int kS2Waves = 4;
// 9, 13 and 18 fit the ranks 1120, 1632 and 2240 (35, 51 and 70 words) with one or two fewer steps per wave
constexpr int kS2QwChoices[] = {2, 4, 6, 8, 9, 10, 12, 13, 14, 16, 18, 20, 24, 28, 32, 36};
constexpr int kS2MaxWr = kS2Waves * 36;

struct Plan {
    int wr;      // words per row of U
    int kpad;    // 32 * wr
    int s2_qw;   // words per wave of the MFMA stage 2, or 0 for the generic kernel
    int zpitch;  // elements per batch row of each intermediate array
};

inline int64_t kpad_of(int64_t r) { return ceil_div(r, 32) * 32; }

inline Plan plan_of(int64_t r) {
    Plan p;
    p.wr = static_cast<int>(ceil_div(r, 32));
    p.kpad = 32 * p.wr;
    p.s2_qw = 0;
    if (p.wr <= kS2MaxWr) {
        const int need = static_cast<int>(ceil_div(p.wr, kS2Waves));
        for (int q : kS2QwChoices)
            if (q >= need) {
                p.s2_qw = q;
                break;
            }
    }
    // stage 2 reads h up to column 32 * 4 * QW; keep a multiple of 64 columns (128 bytes)
    const int64_t cols = std::max<int64_t>(p.kpad, 32 * kS2Waves * p.s2_qw);
    p.zpitch = static_cast<int>(ceil_div(std::max<int64_t>(cols, 64), 64) * 64);
    return p;
}

inline size_t z_bytes(int64_t batch, const Plan& p) {
    return (static_cast<size_t>(batch) * static_cast<size_t>(p.zpitch) * 2 + 255) / 256 * 256;
}

struct GemvArgs {
    const uint16_t* x;
    const uint16_t* s_in;
    const uint32_t* v_bits;
    const uint16_t* s_mid;
    const uint32_t* u_bits;
    const uint16_t* s_out;
    uint16_t* y;
    int batch, n, r, m, wn;
    Plan plan;
    uint16_t* z_hi;
    uint16_t* z_lo;
    float* part;        // room for the batched passes' per-range sums
    size_t part_bytes;  // (the workspace beyond the intermediate)
    hipStream_t stream;
};

// Launch plan of the batched stage 1 (sb_kernel): RTW row tiles per wave (4 waves), CT batch tiles
// of 16, kw words per k range, ks ranges (grid.y), passes over the batch (grid.z).
struct SbPlan {
    int rtw, ct, kw, ks, passes;
    size_t part_bytes, lds_bytes;
};

// When the batched stage 1 replaces s1m_kernel (measured crossovers, see sb_kernel): on rows of at
// least 256 words, from a batch that falls with the row width (sb_min_batch); at most 128 rows (8
// batch tiles), and an LDS slice of at most 160 KB per block. On narrower rows s1m_kernel with two
// or four row tiles per block is the faster one (n = 4096, r = 1632, 64 / 128 rows: 8.9 / 13.4 us
// against 11.5 / 15.6).
constexpr int kSbWideWords = 256;
// The smallest batch that runs it, by words per row (same-box A/B of the GEMV op against the
// kernels it replaces, us). Over 1024 words: from 1 (no VALU shape covers the row). 513-1024
// words: from 2, where it replaced the MFMA stage 1 (Llama-3-70B down_proj, n = 28672, r = 3520:
// 25.9 / 27.3 / 34.4 / 41.9 -> 22.3 / 22.6 / 24.8 / 28.1 at 2 / 3 / 8 / 12 rows; r = 2912 25.0
// -> 20.8 at 2); one row runs the VALU kernel with four words per lane over four waves (r = 3520:
// 25.7 with the MFMA kernel, 21.9 with this one, 17.5; r = 2912 24.0 / 20.0 / 14.8; n = 20480,
// r = 2048: 18.7 / 14.7 / 11.0), which at two rows holds twice the operands and is slower (30.7).
// 512 words (n = 16384, r = 1632): from 3 (17.0 -> 14.2; the VALU kernel at 1 / 2 rows 8.8 / 10.7
// against 13.5 / 13.9). 320-511 words (n = 11008):
// from 8 (r = 1632: 15.0 -> 13.7 at 8, 17.2 -> 14.2 at 12, 5-6% slower at 3-6; r = 2976: 16.0 /
// 16.0 at 8, 19.4 -> 17.4 at 12). 256-319 words (n = 8192): from 8 when V is under 256 K words
// (Llama-3-70B k/v, r = 512: 11.8 / 13.2 -> 11.1 / 11.2 at 8 / 12 rows; slower at 3-4, where the
// VALU kernel runs), else from 16 (q/o at 8 / 12 rows 14.5 / 17.6 against 14.5 / 16.8, gate 23.4
// / 25.0 against 24.5 / 25.1, both slower at 3-4).
inline int64_t sb_min_batch(int64_t wpr, int64_t rows) {
    if (wpr > 1024) return 1;
    if (wpr > 512) return 2;
    if (wpr == 512) return 3;
    if (wpr >= 320) return 8;
    return rows * wpr < 256 * 1024 ? 8 : 16;
}
constexpr int kSbMaxBatch = 128;
constexpr int kSbLdsBytes = 160 * 1024;
constexpr int kSbMaxBlocks = 256;
// Rounds of blocks the search may take when no plan fits one round (see sb_plan_any).
constexpr int kSbMaxRounds = 4;

// Searches row tiles per wave (1, 2, 4: 64, 128, 256 rows per block) and k ranges for the launch
// with the least estimated time, among those whose grid is one block per CU at most (a second round
// of blocks doubles the time) and whose LDS fits. Estimate, in CU cycles: the MFMAs and their
// operand decode per wave, the DMA of the block's slice at ~32 bytes a cycle, and, with several k
// ranges, the finishing launch (~4000) plus the per-range sums written and read.
//
// Where no plan fits one round (the x slice of 16 * ct + 1 columns crowds the rows' words out of
// LDS: Llama-3-70B down_proj, n = 28672, from 48 batch rows; n = 11008 at r = 2976 at 128 rows), the
// search is repeated with up to kSbMaxRounds rounds of blocks, each plan's estimate multiplied by its
// rounds. The alternative, s1m_kernel, streams all of x through every block of 16 rows of V (n =
// 28672, r = 3520, stage 1 at 48 / 64 / 128 rows: 102.8 / 136.6 / 237.9 us with s1m_kernel).
inline bool sb_plan_any(int64_t batch, int64_t rows, int64_t wpr, int64_t kpad, SbPlan& p);
inline bool sb_plan(int64_t batch, int64_t rows, int64_t wpr, int64_t kpad, SbPlan& p) {
    if (batch > kSbMaxBatch || rows <= 0 || wpr <= 0) return false;
    if (wpr < kSbWideWords || batch < sb_min_batch(wpr, rows)) return false;
    return sb_plan_any(batch, rows, wpr, kpad, p);
}
// The search over grids of up to max_rounds rounds of blocks.
// Up to 32 batch rows a round counts two blocks per CU where their LDS fits (a block's DMA of
// its slice then runs beside the other's MFMAs): interleaved same-box A/B, fp16, bit-identical
// outputs (the plans differ in their row tiles only): down_proj at 8 / 16 / 32 rows 12.91 -> 12.35 /
// 13.72 -> 13.19 / 16.60 -> 16.16 us, Llama-3-70B q/o at 16 / 32 rows 16.27 -> 15.78 / 19.79 ->
// 19.36, gate/up at 16 rows 25.22 -> 23.67, down 29.33 -> 28.89. At 64 rows the plan it picks
// (other k ranges) was slower (21.58 -> 22.62), and four blocks per CU were no better.
inline bool sb_plan_rounds(int64_t batch, int64_t rows, int64_t wpr, int64_t kpad, int max_rounds, SbPlan& p) {
    const int64_t occupancy = batch <= 32 ? 2 : 1;  // blocks per CU a round may count
    const int ct = static_cast<int>(std::min<int64_t>(8, ceil_div(batch, 16)));
    const int passes = static_cast<int>(ceil_div(batch, 16LL * ct));
    const int xcols = 16 * ct + 1;
    double best = -1.0;
    for (int rtw : {1, 2, 4}) {
        const int br = 64 * rtw;
        const int64_t row_blocks = ceil_div(rows, br);
        for (int64_t want = 1; want <= wpr; ++want) {
            const int64_t kw = std::max<int64_t>(2, (ceil_div(wpr, want) + 1) & ~int64_t{1});
            const int64_t ks = ceil_div(wpr, kw);
            const int64_t blocks = row_blocks * ks * passes;
            if (blocks > int64_t{kSbMaxBlocks} * occupancy * max_rounds) break;
            const size_t lds = std::max<size_t>(
                static_cast<size_t>(sb_xs_dwords(xcols, static_cast<int>(kw)) + sb_w_dwords(br, static_cast<int>(kw))) * 4,
                static_cast<size_t>(16 * ct) * (br + 4) * 4);
            if (lds > static_cast<size_t>(kSbLdsBytes)) continue;
            const int64_t per_cu = std::min<int64_t>(occupancy, std::max<int64_t>(1, kSbLdsBytes / static_cast<int64_t>(lds)));
            const double mfma = rtw * ct * kw * 16.0 * 1.25;
            const double dma = (xcols * 64.0 + br * 4.0) * kw / 32.0;
            const double fin = ks > 1 ? 4000.0 + 2.0 * ks * batch * kpad * 4.0 / (256.0 * 16.0) : 0.0;
            const double cost = (mfma + dma) * static_cast<double>(ceil_div(blocks, kSbMaxBlocks * per_cu)) + fin;
            if (best < 0 || cost < best) {
                best = cost;
                p.rtw = rtw;
                p.ct = ct;
                p.kw = static_cast<int>(kw);
                p.ks = static_cast<int>(ks);
                p.passes = passes;
                p.part_bytes = ks > 1 ? static_cast<size_t>(ks) * batch * kpad * 4 : 0;
                p.lds_bytes = lds;
            }
        }
    }
    return best >= 0;
}
// The search itself, for any batch up to kSbMaxBatch: one round of blocks if any plan fits it.
inline bool sb_plan_any(int64_t batch, int64_t rows, int64_t wpr, int64_t kpad, SbPlan& p) {
    if (batch > kSbMaxBatch || rows <= 0 || wpr <= 0) return false;
    return sb_plan_rounds(batch, rows, wpr, kpad, 1, p) || sb_plan_rounds(batch, rows, wpr, kpad, kSbMaxRounds, p);
}

template <typename T, int NB>
void launch_stage1_generic(const GemvArgs& a) {
    // at least one block: with r == 0 it only zeroes the intermediate that stage 2 reads
    const dim3 g1(static_cast<unsigned>(std::max<int64_t>(1, ceil_div(a.plan.kpad, kWaves))),
                  static_cast<unsigned>(ceil_div(a.batch, NB)));
    const bool vec = (a.n % 8 == 0) && aligned(a.x, 16) && aligned(a.s_in, 16);
    if (vec)
        gemv_stage1_kernel<T, NB, true><<<g1, kThreads, 0, a.stream>>>(a.x, a.s_in, a.v_bits, a.s_mid, a.z_hi, a.z_lo,
                                                                        a.batch, a.n, a.r, a.wn, a.plan.kpad,
                                                                        a.plan.zpitch);
    else
        gemv_stage1_kernel<T, NB, false><<<g1, kThreads, 0, a.stream>>>(a.x, a.s_in, a.v_bits, a.s_mid, a.z_hi,
                                                                         a.z_lo, a.batch, a.n, a.r, a.wn, a.plan.kpad,
                                                                         a.plan.zpitch);
}

template <typename T, int NB>
void launch_stage2_generic(const GemvArgs& a) {
    const dim3 g2(static_cast<unsigned>(ceil_div(a.m, kWaves)), static_cast<unsigned>(ceil_div(a.batch, NB)));
    gemv_stage2_kernel<T, NB><<<g2, kThreads, 0, a.stream>>>(a.z_hi, a.z_lo, a.u_bits, a.s_out, a.y, a.batch, a.m,
                                                             a.plan.wr, a.plan.zpitch);
}

// Launch shapes of s1w_kernel, which runs at two batch rows, on rows of 385-1024 words, and on
// rows that are not whole words (s1l_kernel takes one batch row otherwise), measured on MI355X
// (graph-replayed, 64-128 rotating weight copies, stage 1 alone): n = 8192 4.49 us at r = 2240 with
// one word per lane over four waves, four rows; n = 11008 4.64 us with one word per lane over six
// waves, four rows, two groups. WPL words per lane, WR waves per row group, R rows per group, G
// groups per block (G * WR * 64 threads, R * G rows). The lanes of a group cover 64 * WR * WPL >= wn
// words of a row.
struct S1wShape {
    int wpl, wr, r, g;
};

// The instantiated shapes (wpl, wr, r, g).
#ifndef NQ_S1W_SHAPES
#define NQ_S1W_SHAPES(X) X(1, 1, 2, 4) X(2, 1, 2, 4) X(1, 4, 4, 1) X(1, 6, 4, 2) X(2, 4, 4, 1) X(4, 4, 4, 1)
#endif

inline S1wShape s1w_shape(int wn) {
    if (wn <= 64) return {1, 1, 2, 4};
    if (wn <= 128) return {2, 1, 2, 4};
    if (wn <= 256) return {1, 4, 4, 1};
    if (wn <= 384) return {1, 6, 4, 2};
    if (wn <= 512) return {2, 4, 4, 1};
    // up to 1024 words, one batch row (x and s_in staged in LDS instead, 16 rows per block, measured
    // slower: Llama-3-70B down_proj 19.6 against 17.6 us, its mixed-rank draw 18.3 against 14.9)
    return {4, 4, 4, 1};
}

template <typename T, int NB, bool kNorm, bool kOne>
void launch_s1w_cfg(const S1wShape& sh, const S1Table& tab, int blocks, const uint16_t* x, int batch, int n, int wn,
                    float eps, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(ceil_div(batch, NB)),
                    static_cast<unsigned>(tab.count));
#define NQ_S1W_CASE(WPL, WR, R, G)                                                                        \
    if (sh.wpl == WPL && sh.wr == WR && sh.r == R && sh.g == G) {                                         \
        s1w_kernel<T, NB, WPL, WR, R, G, kNorm, kOne><<<grid, G * WR * 64, 0, st>>>(tab, x, batch, n, wn, eps); \
        return;                                                                                           \
    }
    NQ_S1W_SHAPES(NQ_S1W_CASE)
#undef NQ_S1W_CASE
}

template <typename T, int NB>
void launch_s1w_nb(const S1wShape& sh, const S1Table& tab, int blocks, const uint16_t* x, int batch, int n, int wn,
                   bool norm, float eps, hipStream_t st) {
    if (tab.count == 1) {
        if (norm) launch_s1w_cfg<T, NB, true, true>(sh, tab, blocks, x, batch, n, wn, eps, st);
        else launch_s1w_cfg<T, NB, false, true>(sh, tab, blocks, x, batch, n, wn, eps, st);
    } else {
        if (norm) launch_s1w_cfg<T, NB, true, false>(sh, tab, blocks, x, batch, n, wn, eps, st);
        else launch_s1w_cfg<T, NB, false, false>(sh, tab, blocks, x, batch, n, wn, eps, st);
    }
}

// One grid plane per item of a stage-1 table, `rows` rows per block: each item's own block count;
// returns the planes' width (the largest count).
inline int item_planes(S1Table& tab, int rows) {
    int blocks = 0;
    for (int k = 0; k < tab.count; ++k) {
        tab.item[k].blocks = static_cast<int>(ceil_div(tab.item[k].kpad, rows));
        blocks = std::max(blocks, tab.item[k].blocks);
    }
    return blocks;
}

// Launch shapes of s1l_kernel (words per lane, rows per wave, groups, waves per group), the
// fastest of a sweep of 14 on the GEMV shapes of each width (n = 4096 / 8192 / 11008).
struct S1lShape {
    int wpl, r, g, wr;
};
inline S1lShape s1l_shape(int wn) {
    if (wn <= 64) return {1, 2, 4, 1};
    if (wn <= 128) return {2, 2, 4, 1};
    if (wn <= 256) return {1, 2, 2, 4};
    return {2, 2, 4, 3};  // up to kS1lMaxWords
}

template <typename T, bool kNorm, bool kOne>
void launch_s1l_cfg(const S1lShape& sh, const S1Table& tab, int blocks, const uint16_t* x, int n, int wn, float eps,
                    hipStream_t st) {
    const size_t lds = s1l_lds_bytes(wn);
#define NQ_S1L_CASE(WPL, R, G, WR)                                                                           \
    if (sh.wpl == WPL && sh.r == R && sh.g == G && sh.wr == WR) {                                            \
        s1l_kernel<T, WPL, R, G, WR, kNorm, kOne>                                                           \
            <<<dim3(blocks, 1, tab.count), G * WR * 64, lds, st>>>(tab, x, n, wn, eps);                      \
        return;                                                                                              \
    }
    NQ_S1L_CASE(1, 2, 4, 1)
    NQ_S1L_CASE(2, 2, 4, 1)
    NQ_S1L_CASE(1, 2, 2, 4)
    NQ_S1L_CASE(2, 2, 4, 3)
#undef NQ_S1L_CASE
}

// Whether s1l_kernel takes the stage: one batch row, rows of whole words (n % 32 == 0; x and s_in
// are 16-byte aligned), up to kS1lMaxWords words.
inline bool s1l_applies(int batch, int n, int wn) { return batch == 1 && n % 32 == 0 && wn <= kS1lMaxWords; }

inline hipError_t allow_lds_bytes(const void* kernel, int bytes);

// Whether s1b_kernel takes the stage (same-box A/B of the GEMV op against the kernels it replaces,
// 32 rotating weight copies, us): rows of up to 128 words at two to four batch rows (n = 4096, gate
// at 2 / 3 / 4 rows 8.31 / 9.65 / 10.17 -> 7.79 / 8.75 / 9.23, q/k/v/o at 2 / 4 rows 6.76 / 8.57 ->
// 6.45 / 7.59), and rows of 257-384 words at two (down_proj, n = 11008: 9.27 -> 8.03). Elsewhere it
// lost: on 8192-wide rows each block of 4 rows of V stages all of x for its batch rows (Llama-3-70B
// q/o at 4 rows 12.0 -> 15.8 us, k/v 6.7 -> 7.3, gate 19.8 -> 27.2, q/o at 2 rows 10.09 -> 10.24),
// and on 257-384-word rows at 3-4 batch rows the 12-wave shape runs out of its 168 registers and
// spills (11008-wide rows at 3 / 4: 12.6 / 12.8 -> 25.1 / 32.5 us).
// (The kernel's static LDS, its partial sums, takes at most 432 bytes of the 1 KB left aside.)
constexpr int kS1bLdsBytes = kSbLdsBytes - 1024;
inline bool s1b_applies(int batch, int n, int wn) {
    if (batch < 2 || batch > 4 || n % 32 != 0) return false;
    if (!(wn <= 128 || (batch == 2 && wn > 256 && wn <= kS1lMaxWords))) return false;
    return s1b_lds_bytes(wn, batch) <= static_cast<size_t>(kS1bLdsBytes);
}

template <typename T, int NB, bool kNorm, bool kOne>
void launch_s1b_cfg(const S1lShape& sh, const S1Table& tab, int blocks, const uint16_t* x, int n, int wn, float eps,
                    hipStream_t st) {
    const size_t lds = s1b_lds_bytes(wn, NB);
    // (blocks may take more than 64 KB of LDS: the limit is raised once per kernel)
#define NQ_S1B_CASE(WPL, R, G, WR)                                                                               \
    if (sh.wpl == WPL && sh.r == R && sh.g == G && sh.wr == WR) {                                                \
        static const hipError_t attr = allow_lds_bytes(                                                          \
            reinterpret_cast<const void*>(&s1b_kernel<T, WPL, R, G, WR, NB, kNorm, kOne>), kS1bLdsBytes);        \
        (void)attr; /* a refusal surfaces as the launch's error */                                              \
        s1b_kernel<T, WPL, R, G, WR, NB, kNorm, kOne>                                                            \
            <<<dim3(blocks, 1, tab.count), G * WR * 64, lds, st>>>(tab, x, n, wn, eps);                          \
        return;                                                                                                  \
    }
    NQ_S1B_CASE(1, 2, 4, 1)
    NQ_S1B_CASE(2, 2, 4, 1)
    if constexpr (NB == 2) {  // (wider rows take two batch rows only, see s1b_applies)
        NQ_S1B_CASE(2, 2, 4, 3)
    }
#undef NQ_S1B_CASE
}

template <typename T, int NB>
void launch_s1b_table(const S1lShape& sh, const S1Table& tab, int blocks, const uint16_t* x, int n, int wn, bool norm,
                      float eps, hipStream_t st) {
    if (tab.count == 1) {
        if (norm) launch_s1b_cfg<T, NB, true, true>(sh, tab, blocks, x, n, wn, eps, st);
        else launch_s1b_cfg<T, NB, false, true>(sh, tab, blocks, x, n, wn, eps, st);
    } else {
        if (norm) launch_s1b_cfg<T, NB, true, false>(sh, tab, blocks, x, n, wn, eps, st);
        else launch_s1b_cfg<T, NB, false, false>(sh, tab, blocks, x, n, wn, eps, st);
    }
}

// One launch over every item of `tab` (block ranges filled in here). The caller checked that
// the fast stage 1 applies: n >= 8, n % 8 == 0, wn <= 1024, x and each s_in 16-byte aligned,
// every r > 0.
template <typename T>
void launch_s1w_table(S1Table& tab, const uint16_t* x, int batch, int n, int wn, bool norm, float eps,
                      hipStream_t st) {
    if (s1b_applies(batch, n, wn)) {
        const S1lShape sh = s1l_shape(wn);
        const int blocks = item_planes(tab, sh.r * sh.g);
        if (batch == 2) launch_s1b_table<T, 2>(sh, tab, blocks, x, n, wn, norm, eps, st);
        else if (batch == 3) launch_s1b_table<T, 3>(sh, tab, blocks, x, n, wn, norm, eps, st);
        else launch_s1b_table<T, 4>(sh, tab, blocks, x, n, wn, norm, eps, st);
        return;
    }
    if (s1l_applies(batch, n, wn)) {
        const S1lShape sh = s1l_shape(wn);
        const int blocks = item_planes(tab, sh.r * sh.g);
        if (tab.count == 1) {
            if (norm) launch_s1l_cfg<T, true, true>(sh, tab, blocks, x, n, wn, eps, st);
            else launch_s1l_cfg<T, false, true>(sh, tab, blocks, x, n, wn, eps, st);
        } else {
            if (norm) launch_s1l_cfg<T, true, false>(sh, tab, blocks, x, n, wn, eps, st);
            else launch_s1l_cfg<T, false, false>(sh, tab, blocks, x, n, wn, eps, st);
        }
        return;
    }
    const S1wShape sh = s1w_shape(wn);
    const int blocks = item_planes(tab, sh.r * sh.g);
    if (batch <= 1) launch_s1w_nb<T, 1>(sh, tab, blocks, x, batch, n, wn, norm, eps, st);
    else launch_s1w_nb<T, 2>(sh, tab, blocks, x, batch, n, wn, norm, eps, st);
}

inline bool s1m_sin_lds(int n, int wn, int rt = 1) { return 16 * rt * s1m_row_stride(wn, rt) + n / 2 <= kS1mMaxStaged; }
inline size_t s1m_lds_bytes(int n, int wn, int rt = 1) {
    const size_t staged = static_cast<size_t>(16 * rt * s1m_row_stride(wn, rt) + (s1m_sin_lds(n, wn, rt) ? n / 2 : 0)) * 4;
    const size_t reduce = static_cast<size_t>(16) * 64 * (16 * rt + 4);  // the waves' tiles and x^2 sums
    return std::max(staged, reduce);
}
// Whether the MFMA stage 1 takes rows of n columns at all (up to n = 32768).
inline bool s1m_fits(int n, int wn, int rt = 1) {
    (void)n;
    return 16 * rt * s1m_row_stride(wn, rt) <= kS1mMaxStaged;
}

// Raises a kernel's dynamic LDS limit. Each caller runs it once per kernel, on the kernel's first
// launch, which may come inside a caller's stream capture (a graph or torch.compile's CUDA graphs):
// the thread's capture mode is relaxed around the call, which is no stream operation.
inline hipError_t allow_lds_bytes(const void* kernel, int bytes) {
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const hipError_t ex = hipThreadExchangeStreamCaptureMode(&mode);
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (ex == hipSuccess) (void)hipThreadExchangeStreamCaptureMode(&mode);
    return e;
}

// Blocks of s1m_kernel<..., RT> may take more than 64 KB of LDS (the limit is set once per kernel).
template <typename Kernel>
int s1m_allow_lds(Kernel* k) {
    static const hipError_t attr = allow_lds_bytes(reinterpret_cast<const void*>(k), kSbLdsBytes);
    return attr == hipSuccess ? NQ_OK : fail(NQ_ERR_HIP, "nq_gemv stage 1: LDS limit: %s", hipGetErrorString(attr));
}

template <typename T, int NW, int LD, int RT>
void launch_s1m_loads(const S1Table& tab, dim3 grid, const uint16_t* x, int batch, int n, int wn, bool norm, float eps,
                      hipStream_t st) {
    const size_t lds = s1m_lds_bytes(n, wn, RT);
    const bool sl = s1m_sin_lds(n, wn, RT);
    const bool pad = s1m_row_stride(wn, RT) != wn;  // only ever with RT <= 2
#define NQ_S1M_P(NORM, ONE, SL, PAD)                                                                     \
    (s1m_allow_lds(&s1m_kernel<T, NW, NORM, ONE, SL, LD, RT, PAD>),                                      \
     s1m_kernel<T, NW, NORM, ONE, SL, LD, RT, PAD><<<grid, NW * 64, lds, st>>>(tab, x, batch, n, wn, eps))
    // (four row tiles run with s_in in LDS only, see s1m_row_tiles: that variant alone is built)
#define NQ_S1M(NORM, ONE)                                                                                 \
    (sl ? (pad && RT <= 2 ? NQ_S1M_P(NORM, ONE, true, RT <= 2) : NQ_S1M_P(NORM, ONE, true, false))     \
        : (pad && RT <= 2 ? NQ_S1M_P(NORM, ONE, RT == 4, RT <= 2) : NQ_S1M_P(NORM, ONE, RT == 4, false)))
    if (tab.count == 1) {
        if (norm) NQ_S1M(true, true);
        else NQ_S1M(false, true);
    } else {
        if (norm) NQ_S1M(true, false);
        else NQ_S1M(false, false);
    }
#undef NQ_S1M
#undef NQ_S1M_P
}
template <typename T, int NW, int RT>
void launch_s1m_nw(const S1Table& tab, dim3 grid, const uint16_t* x, int batch, int n, int wn, bool norm, float eps,
                   hipStream_t st) {
    const bool sl = s1m_sin_lds(n, wn, RT);
    const int staged = 16 * RT * wn + (sl ? n / 2 : 0);
    const int per_thread = static_cast<int>(ceil_div(staged, NW * 64));
    if (per_thread <= 4) launch_s1m_loads<T, NW, 4, RT>(tab, grid, x, batch, n, wn, norm, eps, st);
    else if (per_thread <= 8) launch_s1m_loads<T, NW, 8, RT>(tab, grid, x, batch, n, wn, norm, eps, st);
    else if (per_thread <= 12) launch_s1m_loads<T, NW, 12, RT>(tab, grid, x, batch, n, wn, norm, eps, st);
    else launch_s1m_loads<T, NW, 16, RT>(tab, grid, x, batch, n, wn, norm, eps, st);
}

// Row tiles per block of s1m_kernel: the fewest of 1, 2 and 4 whose grid is one round of blocks
// (one per CU; a second round costs as much as the first), else 4, the fewest rounds. Measured (us,
// 1 / 2 / 4 row tiles, n = 4096, r = 1632): 16 batch rows 7.2 / 8.7 / 13.2, 64 rows 12.2 / 8.9 / 13.3,
// 128 rows 21.1 / 16.3 / 13.4.
inline int s1m_row_tiles(const S1Table& tab, int batch, int n, int wn) {
    const int64_t passes = ceil_div(batch, 16);
    for (int rt : {1, 2, 4}) {
        // (four row tiles only with s_in in LDS: with s_in from global that variant runs out of registers)
        if (!s1m_fits(n, wn, rt) || (rt == 4 && !s1m_sin_lds(n, wn, rt))) break;
        int64_t blocks = 0;
        for (int k = 0; k < tab.count; ++k) blocks += ceil_div(tab.item[k].kpad, 16 * rt);
        if (blocks * passes <= 256 || rt == 4) return rt;
    }
    return s1m_fits(n, wn, 2) ? 2 : 1;
}

// The MFMA stage 1 over every item of `tab` (16 rt rows per block, 16 batch rows per grid row).
template <typename T>
void launch_s1m_table(S1Table& tab, const uint16_t* x, int batch, int n, int wn, bool norm, float eps,
                      hipStream_t st, int rt = 0) {
    if (rt == 0) rt = s1m_row_tiles(tab, batch, n, wn);
    if (rt == 4 && !s1m_sin_lds(n, wn, 4)) rt = 2;  // the only four-row-tile variant keeps s_in in LDS
    const int blocks = item_planes(tab, 16 * rt);
    // 16 waves per block: a 4096-wide row is one round of loads per wave (latency, not bytes, is
    // what a decode-size stage pays for)
    const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(ceil_div(batch, 16)),
                    static_cast<unsigned>(tab.count));
    if (rt == 4) launch_s1m_nw<T, 16, 4>(tab, grid, x, batch, n, wn, norm, eps, st);
    else if (rt == 2) launch_s1m_nw<T, 16, 2>(tab, grid, x, batch, n, wn, norm, eps, st);
    else launch_s1m_nw<T, 16, 1>(tab, grid, x, batch, n, wn, norm, eps, st);
}

// Stage 1 of a table: the VALU kernel for one or two batch rows of up to 16384 columns (32768 at
// one row), for three or four rows of up to 8192 columns when V holds fewer than 256 K words, two
// rows a pass (4096 x 1632 at 3 / 4 rows 5.7 / 5.8 -> 5.0 / 5.5 us; the Llama-3-70B k/v GEMV, 8192
// x 512, 11.2 / 11.3 -> 7.5 / 7.6 us for the op), and for three rows when the rank is at most 2496
// (same-box A/B of the op: 8192 columns at r = 1792 / 2048 / 2240 / 2400 / 2496 10.5 / 9.6 / 2.8-5
// / 3.1-4.9 / 4.4% faster, 4096 columns at r = 2048 4.6-7.4%; at four rows the gain holds with
// s_mid, 1-2.8%, and turns into a 0.2-0.7% loss without it, so four rows keep the MFMA kernel);
// past that the second pass re-reads too much of V (4096 columns at r = 2560 / 2976: 4.6 / 3.8%
// slower at three rows; 8192 at 3520: 6%) and the MFMA kernel runs, as it does otherwise.
template <typename T>
void launch_stage1_table(S1Table& tab, const uint16_t* x, int batch, int n, int wn, bool norm, float eps,
                         hipStream_t st) {
    int r_max = 0;
    for (int k = 0; k < tab.count; ++k) r_max = std::max(r_max, tab.item[k].r);
    const int64_t v_words = static_cast<int64_t>(r_max) * wn;
    const bool valu_rows = batch <= 2 || (batch <= 4 && wn <= 256 && v_words < 256 * 1024) ||
                           (batch == 3 && wn <= 256 && r_max <= 2496);
    // past 512 words the VALU shape covers one batch row (four words per lane)
    if (!s1b_applies(batch, n, wn) && (!valu_rows || wn > 1024 || (wn > 512 && batch > 1)) && s1m_fits(n, wn))
        launch_s1m_table<T>(tab, x, batch, n, wn, norm, eps, st);
    else
        launch_s1w_table<T>(tab, x, batch, n, wn, norm, eps, st);
}

// The fast stage 1 (s1w up to 16384 columns, 32768 at one batch row; s1m up to 32768; chosen by
// launch_stage1_table) applies.
inline bool s1w_applies(const uint16_t* x, const uint16_t* s_in, int n, int wn, int r) {
    return n >= 8 && n % 8 == 0 && r > 0 && aligned(x, 16) && aligned(s_in, 16) && (wn <= 1024 || s1m_fits(n, wn));
}

inline S1Item s1_item_of(const GemvArgs& a) {
    S1Item it;
    it.v_bits = a.v_bits;
    it.s_in = a.s_in;
    it.s_mid = a.s_mid;
    it.z_hi = a.z_hi;
    it.z_lo = a.z_lo;
    it.r = a.r;
    it.kpad = a.plan.kpad;
    it.zpitch = a.plan.zpitch;
    it.blocks = 0;
    return it;
}

// ---- batched stage 1

template <typename T, int RTW, int CT>
int launch_sb_cfg(const SbArgs& s, const SbPlan& p, hipStream_t st) {
    constexpr int NW = 4;
    // blocks may take more than 64 KB of LDS (once per kernel: the limit is a property of the function)
    static const hipError_t attr = allow_lds_bytes(reinterpret_cast<const void*>(&sb_kernel<T, NW, RTW, CT>),
                                                   kSbLdsBytes);
    if (attr != hipSuccess) return fail(NQ_ERR_HIP, "nq_gemv batched stage 1: LDS limit: %s", hipGetErrorString(attr));
    const dim3 grid(static_cast<unsigned>(ceil_div(s.M, 16 * NW * RTW)), static_cast<unsigned>(p.ks),
                    static_cast<unsigned>(p.passes));
    sb_kernel<T, NW, RTW, CT><<<grid, NW * 64, p.lds_bytes, st>>>(s);
    return NQ_OK;
}

template <typename T, int RTW>
int launch_sb_rtw(const SbArgs& s, const SbPlan& p, hipStream_t st) {
    switch (p.ct) {
        case 1: return launch_sb_cfg<T, RTW, 1>(s, p, st);
        case 2: return launch_sb_cfg<T, RTW, 2>(s, p, st);
        case 3: return launch_sb_cfg<T, RTW, 3>(s, p, st);
        case 4: return launch_sb_cfg<T, RTW, 4>(s, p, st);
        case 5: return launch_sb_cfg<T, RTW, 5>(s, p, st);
        case 6: return launch_sb_cfg<T, RTW, 6>(s, p, st);
        case 7: return launch_sb_cfg<T, RTW, 7>(s, p, st);
        default: return launch_sb_cfg<T, RTW, 8>(s, p, st);
    }
}

// Batched stage 1: rows of whole words (n % 32 == 0), 16-byte aligned x and s_in, and the per-range
// sums fit in the workspace.
inline bool sb1_plan(const GemvArgs& a, SbPlan& p) {
    return a.n % 32 == 0 && a.r > 0 && aligned(a.x, 16) && aligned(a.s_in, 16) &&
           sb_plan(a.batch, a.r, a.wn, a.plan.kpad, p) && p.part_bytes <= a.part_bytes;
}

template <typename T>
int launch_stage1_sb(const GemvArgs& a, const SbPlan& p) {
    SbArgs s{};
    s.words = a.v_bits;
    s.s_in = a.s_in;
    s.x = a.x;
    s.s_mid = a.s_mid;
    s.z_hi = a.z_hi;
    s.z_lo = a.z_lo;
    s.part = a.part;
    s.M = a.r;
    s.wpr = a.wn;
    s.ldx = a.n;
    s.batch = a.batch;
    s.kw = p.kw;
    s.kpad = a.plan.kpad;
    s.zpitch = a.plan.zpitch;
    s.kw4_magic = div_magic(4u * static_cast<uint32_t>(p.kw));
    s.ws_magic = div_magic(static_cast<uint32_t>(p.kw) + 1u);
    const int e = p.rtw == 4 ? launch_sb_rtw<T, 4>(s, p, a.stream)
                             : (p.rtw == 2 ? launch_sb_rtw<T, 2>(s, p, a.stream) : launch_sb_rtw<T, 1>(s, p, a.stream));
    if (e) return e;
    if (p.ks > 1) {
        if (int c = check_launch("nq_gemv stage 1 (batched)")) return c;
        const int64_t threads = static_cast<int64_t>(s.batch) * s.zpitch / 4;
        sb_finish1<T><<<dim3(static_cast<unsigned>(ceil_div(threads, 256))), 256, 0, a.stream>>>(s, p.ks);
    }
    return NQ_OK;
}

template <typename T>
int launch_stage1(const GemvArgs& a) {
    SbPlan sp;
    if (sb1_plan(a, sp)) return launch_stage1_sb<T>(a, sp);
    if (s1w_applies(a.x, a.s_in, a.n, a.wn, a.r)) {
        S1Table tab;
        tab.count = 1;
        tab.item[0] = s1_item_of(a);
        launch_stage1_table<T>(tab, a.x, a.batch, a.n, a.wn, false, 0.0f, a.stream);
        return NQ_OK;
    }
    if (a.batch <= 1) launch_stage1_generic<T, 1>(a);
    else if (a.batch <= 2) launch_stage1_generic<T, 2>(a);
    else if (a.batch <= 4) launch_stage1_generic<T, 4>(a);
    else launch_stage1_generic<T, kMaxNB>(a);
    return NQ_OK;
}

// Batch rows per pass of s2t_kernel over one item (qw words per wave, twice that for a gated pair):
// up to 8, as many as fit the LDS's 128 * QW-column intermediate.
inline int s2t_rows_per_pass(int batch, int qw) {
    const int want = std::min(batch, 8);
    int nb = want <= 1 ? 1 : (want <= 2 ? 2 : (want <= 4 ? 4 : 8));
    while (nb > 1 && nb * qw > 128) nb >>= 1;
    return nb;
}

// Only the batch splits that fit in LDS are instantiated (the host never picks the others).
template <typename T, int QW, int NB, int EPI, int RT>
void launch_s2t_nb(const S2Table& tab, dim3 grid, int batch, hipStream_t st) {
    if constexpr (NB == 1 || (EPI == kEpiGated ? 2 : 1) * NB * QW <= 128)
        s2t_kernel<T, QW, NB, EPI, RT><<<grid, 256, 0, st>>>(tab, batch);
}

// Static LDS of s2t_kernel<QW, NB, one item, RT> (tile, intermediate, partial tiles).
inline int64_t s2t_lds_bytes(int nb, int qw, int rt) {
    return (16LL * rt * kS2Waves * qw + 4) * 4 + 2LL * nb * 32 * kS2Waves * qw * 2 + 16LL * rt * kS2Waves * 64;
}
// Row tiles per block of the MFMA stage 2 for nb batch rows per pass over `tiles` 16-row tiles and
// `passes` passes. One or two batch rows: one tile (measured: two tiles gain nothing). From four:
// the most tiles per block (4, 2, 1) whose grid still has at least 160 blocks and fits one round
// of blocks resident by LDS; if none fits, the fewest rounds, ties to fewer tiles. Measured
// (11008 x 1632, us at batch 4 / 8 / 16, tiles 1 - 2 - 4): 5.55-5.03-4.87, 7.37-6.26-5.49,
// 11.37-8.40-9.74; at 4096 x 1632, batch 8 / 16: 3.89-4.30-5.33, 5.41-4.46-5.45.
inline int s2t_row_tiles(int nb, int qw, int64_t tiles, int64_t passes) {
    if (nb < 4) return 1;
    int best = 1;
    int64_t best_rounds = INT64_MAX;
    for (int rt : {4, 2, 1}) {
        const int64_t blocks = ceil_div(tiles, rt) * passes;
        const int64_t per_cu = std::min<int64_t>(8, (160 * 1024) / s2t_lds_bytes(nb, qw, rt));
        const int64_t rounds = ceil_div(blocks, std::max<int64_t>(1, per_cu) * 256);
        if (rounds == 1 && blocks >= 160) return rt;
        if (rounds <= best_rounds) {  // <= : ties go to the fewer tiles tried later
            best_rounds = rounds;
            best = rt;
        }
    }
    return best;
}

template <typename T, int QW, int NB, int EPI>
void launch_s2t_rt(const S2Table& tab, dim3 grid, int batch, int rt, hipStream_t st) {
    if (rt == 4) launch_s2t_nb<T, QW, NB, EPI, 4>(tab, grid, batch, st);
    else if (rt == 2) launch_s2t_nb<T, QW, NB, EPI, 2>(tab, grid, batch, st);
    else launch_s2t_nb<T, QW, NB, EPI, 1>(tab, grid, batch, st);
}

// NB batch rows of h per block (LDS holds P * 2 * NB * 128 * QW halves: P * NB * QW <= 128
// keeps it within 64 KB); larger batches take several passes over U.
template <typename T, int QW, int EPI>
void launch_s2t_table(S2Table& tab, int batch, hipStream_t st) {
    constexpr int P = EPI == kEpiGated ? 2 : 1;
    const int nb = s2t_rows_per_pass(batch, P * QW);
    // row tiles per block (the gated pair stays at one: it runs two items already)
    int64_t tiles = 0;
    for (int k = 0; k < (EPI == kEpiGated ? 1 : tab.count); ++k) tiles += ceil_div(tab.item[k].m, 16);
    const int rt = EPI == kEpiGated || EPI == kEpiRope ? 1 : s2t_row_tiles(nb, QW, tiles, ceil_div(batch, nb));
    // one grid plane per item (a gated pair runs item 1 inside item 0's blocks)
    const int items = EPI == kEpiGated ? 1 : tab.count;
    int blocks = 0;
    for (int k = 0; k < tab.count; ++k) {
        tab.item[k].blocks = static_cast<int>(ceil_div(tab.item[k].m, 16 * rt));
        blocks = std::max(blocks, tab.item[k].blocks);
    }
    const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(ceil_div(batch, nb)),
                    static_cast<unsigned>(items));
    if (nb == 1) launch_s2t_nb<T, QW, 1, EPI, 1>(tab, grid, batch, st);
    else if constexpr (EPI == kEpiGated) {
        if (nb == 2) launch_s2t_nb<T, QW, 2, EPI, 1>(tab, grid, batch, st);
        else if (nb == 4) launch_s2t_nb<T, QW, 4, EPI, 1>(tab, grid, batch, st);
        else launch_s2t_nb<T, QW, 8, EPI, 1>(tab, grid, batch, st);
    } else {
        if (nb == 2) launch_s2t_rt<T, QW, 2, EPI>(tab, grid, batch, rt, st);
        else if (nb == 4) launch_s2t_rt<T, QW, 4, EPI>(tab, grid, batch, rt, st);
        else launch_s2t_rt<T, QW, 8, EPI>(tab, grid, batch, rt, st);
    }
}

// Launches the MFMA stage 2 for words-per-wave choice qw; false when qw is not one of them.
template <typename T, int EPI>
bool launch_s2t_qw(S2Table& tab, int qw, int batch, hipStream_t st) {
    switch (qw) {
        case 2: launch_s2t_table<T, 2, EPI>(tab, batch, st); return true;
        case 4: launch_s2t_table<T, 4, EPI>(tab, batch, st); return true;
        case 6: launch_s2t_table<T, 6, EPI>(tab, batch, st); return true;
        case 8: launch_s2t_table<T, 8, EPI>(tab, batch, st); return true;
        case 9: launch_s2t_table<T, 9, EPI>(tab, batch, st); return true;
        case 10: launch_s2t_table<T, 10, EPI>(tab, batch, st); return true;
        case 12: launch_s2t_table<T, 12, EPI>(tab, batch, st); return true;
        case 13: launch_s2t_table<T, 13, EPI>(tab, batch, st); return true;
        case 14: launch_s2t_table<T, 14, EPI>(tab, batch, st); return true;
        case 16: launch_s2t_table<T, 16, EPI>(tab, batch, st); return true;
        case 18: launch_s2t_table<T, 18, EPI>(tab, batch, st); return true;
        case 20: launch_s2t_table<T, 20, EPI>(tab, batch, st); return true;
        case 24: launch_s2t_table<T, 24, EPI>(tab, batch, st); return true;
        case 28: launch_s2t_table<T, 28, EPI>(tab, batch, st); return true;
        case 32: launch_s2t_table<T, 32, EPI>(tab, batch, st); return true;
        case 36: launch_s2t_table<T, 36, EPI>(tab, batch, st); return true;
        default: return false;
    }
}

// One s2b_kernel shape over the op's arguments: grid (row blocks, batch passes); the U tile is
// the dynamic LDS. Needs s2t_applies (s2_qw > 0 keeps zpitch >= 32 KC * chunks).
template <typename T, int RT, int WR, int CTW, int KC>
int launch_s2b_cfg(const GemvArgs& a) {
    using S = S2bShape<RT, WR, CTW, KC>;
    constexpr int kStatic = 3 * 16 * S::kSlots;
    S2bArgs s;
    s.u_bits = a.u_bits;
    s.s_out = a.s_out;
    s.y = a.y;
    s.z_hi = a.z_hi;
    s.z_lo = a.z_lo;
    s.m = a.m;
    s.wr = a.plan.wr;
    s.zpitch = a.plan.zpitch;
    s.batch = a.batch;
    s.chunks = static_cast<int>(ceil_div(a.plan.wr, KC));
    s.u_slots = static_cast<int>(ceil_div(static_cast<int64_t>(S::kRows) * a.plan.wr + KC, 64) * 64);
    s.store8 = a.m % 4 == 0 && aligned(a.y, 8);
    const size_t dyn = static_cast<size_t>(s.u_slots) * 4;
    if (32LL * KC * s.chunks > a.plan.zpitch || kStatic + dyn > static_cast<size_t>(kSbLdsBytes))
        return fail(NQ_ERR_UNSUPPORTED, "nq_gemv batched stage 2: shape does not fit");
    static const hipError_t attr = allow_lds_bytes(reinterpret_cast<const void*>(&s2b_kernel<T, RT, WR, CTW, KC>),
                                                   kSbLdsBytes - kStatic);
    if (attr != hipSuccess) return fail(NQ_ERR_HIP, "nq_gemv batched stage 2: LDS limit: %s", hipGetErrorString(attr));
    const dim3 grid(static_cast<unsigned>(ceil_div(a.m, S::kRows)), static_cast<unsigned>(ceil_div(a.batch, S::kBatch)));
    s2b_kernel<T, RT, WR, CTW, KC><<<grid, 256, dyn, a.stream>>>(s);
    return NQ_OK;
}

inline bool s2t_applies(const void* z_hi, const void* z_lo, const uint32_t* u_bits, int m, const Plan& plan) {
    return aligned(z_hi, 16) && aligned(z_lo, 16) && aligned(u_bits, 16) && static_cast<int64_t>(m) * plan.wr >= 4 &&
           plan.s2_qw > 0;
}

// When the batched stage 2 replaces s2t_kernel, and its shape (measured on the Llama-2-7B gate
// and down shapes at r = 1632, batch 16 - 128; us, s2t against s2b): from 16 batch rows when
// m * batch >= 160 K (gate, 11008 rows: 7.7 / 6.4 at 16 rows, 12.3 / 6.8 at 32, 20.8 / 8.9 at 64,
// 38.7 / 13.1 at 128; down, 4096 rows: 4.0 / 5.3 at 16 and 5.0 / 5.5 at 32 stay with s2t, 9.1 / 6.05
// at 64, 16.0 / 7.1 at 128). Every shape gives each wave one row tile against one to four column
// tiles. Over 512 or more row tiles: 64-row blocks (WR = 4) of 16 batch rows up to 64 rows, 32
// beyond, two-word chunks (640-1023 tiles at 16 rows or fewer: as below 512). Below: 32-row blocks (WR = 2) of 16 batch rows and four-word chunks up
// to 64 rows, 32 batch rows and two-word chunks beyond. Smaller chunks leave room in LDS for more
// resident blocks, which is what these latency-bound blocks gain from.
constexpr int64_t kS2bMinWork = 160 * 1024;
constexpr int kS2bMinBatch = 16;
// ... and below 16 rows when U is large (at least 2M words) and s2t_kernel would need two passes or
// more: its LDS holds fewer batch rows per pass at large ranks (two at r = 4224), and every pass
// decodes U again (Llama-3-70B gate, m = 28672: r = 4224 at 4 / 8 rows 26.9 / 50.0 -> 14.3 / 14.3 us;
// r = 3520 at 8 rows 20.6 -> 12.1).
constexpr int64_t kS2bMinWordsFewRows = int64_t{1} << 21;

inline bool s2b_chosen(const GemvArgs& a) {
    if (a.batch >= kS2bMinBatch && static_cast<int64_t>(a.m) * a.batch >= kS2bMinWork) return true;
    return static_cast<int64_t>(a.m) * a.plan.wr >= kS2bMinWordsFewRows &&
           ceil_div(a.batch, s2t_rows_per_pass(a.batch, a.plan.s2_qw)) >= 2;
}

template <typename T>
int launch_stage2_batched(const GemvArgs& a) {
    const int64_t tiles = ceil_div(a.m, 16);
    if (tiles >= 512) {
        // 640-1023 row tiles (the 11008-row gate/up factors) at 16 rows or fewer: 32-row blocks with
        // four-word chunks (same-box, r = 1632 / 2976: 14.52 / 18.67 -> 13.93 / 17.42 us per GEMV; at
        // 1792 tiles, Llama-3-70B gate/up, they lose 12-25%, at 512 they tie, at 24 rows they lose)
        if (tiles >= 640 && tiles < 1024 && a.batch <= 16) return launch_s2b_cfg<T, 2, 2, 1, 4>(a);
        if (a.batch <= 64) return launch_s2b_cfg<T, 4, 4, 2, 2>(a);
        return launch_s2b_cfg<T, 4, 4, 4, 2>(a);
    }
    if (a.batch <= 64) return launch_s2b_cfg<T, 2, 2, 1, 4>(a);
    return launch_s2b_cfg<T, 2, 2, 2, 2>(a);
}

template <typename T>
int launch_stage2(const GemvArgs& a) {
    if (s2t_applies(a.z_hi, a.z_lo, a.u_bits, a.m, a.plan) && s2b_chosen(a)) return launch_stage2_batched<T>(a);
    if (s2t_applies(a.z_hi, a.z_lo, a.u_bits, a.m, a.plan)) {
        S2Table tab;
        tab.count = 1;
        S2Item& it = tab.item[0];
        it.u_bits = a.u_bits;
        it.s_out = a.s_out;
        it.y = a.y;
        it.resid = nullptr;
        it.z_hi = a.z_hi;
        it.z_lo = a.z_lo;
        it.m = a.m;
        it.wr = a.plan.wr;
        it.zpitch = a.plan.zpitch;
        it.ystride = a.m;
        it.blocks = 0;
        if (launch_s2t_qw<T, kEpiStoreOne>(tab, a.plan.s2_qw, a.batch, a.stream)) return NQ_OK;
    }
    if (a.batch <= 1) launch_stage2_generic<T, 1>(a);
    else if (a.batch <= 2) launch_stage2_generic<T, 2>(a);
    else if (a.batch <= 4) launch_stage2_generic<T, 4>(a);
    else launch_stage2_generic<T, kMaxNB>(a);
    return NQ_OK;
}

template <typename T>
int run_gemv(const GemvArgs& a) {
    if (int s = launch_stage1<T>(a)) return s;
    if (int s = check_launch("nq_gemv stage 1")) return s;
    if (int s = launch_stage2<T>(a)) return s;
    return check_launch("nq_gemv stage 2");
}

// The header and the intermediate (what every path needs).
inline size_t gemv_base_bytes(int64_t batch, int64_t r) { return kHeaderBytes + 2 * z_bytes(batch, plan_of(r)); }

// The per-range sums of the batched stage 1 at these sizes. A smaller workspace runs the kernels
// that keep none.
inline size_t gemv_part_bytes(int64_t batch, int64_t n, int64_t r, int64_t m) {
    (void)m;
    const Plan pl = plan_of(r);
    size_t bytes = 0;
    SbPlan p;
    if (n % 32 == 0 && r > 0 && sb_plan(batch, r, ceil_div(n, 32), pl.kpad, p)) bytes = p.part_bytes;
    return (bytes + 255) / 256 * 256;
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" {

size_t nq_gemv_workspace_bytes(int64_t batch, int64_t n, int64_t r, int64_t m) {
    if (batch < 0 || r < 0 || n < 0 || m < 0) return 0;
    return gemv_base_bytes(batch, r) + gemv_part_bytes(batch, n, r, m);
}

}  // extern "C"

namespace nq {
namespace {

enum Stages { kStage1 = 1, kStage2 = 2, kBoth = 3 };

// Validates the arguments one or both stages use and fills `a`; returns NQ_OK, an error
// status, or -1 when there is nothing to do.
int setup_gemv(const char* name, int stages, int dtype, const void* x, const void* s_in, const uint32_t* v_bits,
               const void* s_mid, const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n,
               int64_t r, int64_t m, void* workspace, size_t workspace_bytes, nq_stream_t stream, GemvArgs& a) {
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "%s: unsupported dtype %d", name, dtype);
    if (batch < 0 || n < 0 || r < 0 || m < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: negative size", name);
    if (n > INT32_MAX / 4 || r > INT32_MAX / 4 || m > INT32_MAX / 4 || batch > INT32_MAX / 4 ||
        batch * plan_of(r).zpitch > INT32_MAX / 4 || m * ceil_div(r, 32) > INT32_MAX / 4 ||
        r * ceil_div(n, 32) > INT32_MAX / 4 || batch * n > INT32_MAX / 4)
        return fail(NQ_ERR_UNSUPPORTED, "%s: sizes beyond 2^29 are not supported", name);
    // stage 1 with r == 0 still runs: it zeroes the intermediate stage 2 reads
    if (batch == 0 || (stages != kStage1 && m == 0)) return -1;
    const bool s1 = stages & kStage1, s2 = stages & kStage2;
    if (!workspace || (s1 && (!x || !s_in || !v_bits)) || (s2 && (!u_bits || !s_out || !y)))
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(workspace, 256)) return fail(NQ_ERR_ALIGNMENT, "%s: workspace must be 256-byte aligned", name);
    if ((s1 && (!aligned(x, 2) || !aligned(s_in, 2) || !aligned(v_bits, 4) || (s_mid && !aligned(s_mid, 2)))) ||
        (s2 && (!aligned(s_out, 2) || !aligned(y, 2) || !aligned(u_bits, 4))))
        return fail(NQ_ERR_ALIGNMENT, "%s: misaligned operand", name);
    const size_t need = gemv_base_bytes(batch, r);
    if (workspace_bytes < need)
        return fail(NQ_ERR_WORKSPACE, "%s: workspace has %zu bytes, needs %zu", name, workspace_bytes,
                    nq_gemv_workspace_bytes(batch, n, r, m));
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
    a.plan = plan_of(r);
    char* base = static_cast<char*>(workspace) + kHeaderBytes;
    a.z_hi = reinterpret_cast<uint16_t*>(base);
    a.z_lo = reinterpret_cast<uint16_t*>(base + z_bytes(batch, a.plan));
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + need);
    a.part_bytes = workspace_bytes - need;
    a.stream = as_stream(stream);
    return NQ_OK;
}

template <typename T>
int run_stage1(const GemvArgs& a) {
    if (int s = launch_stage1<T>(a)) return s;
    return check_launch("nq_gemv stage 1");
}

template <typename T>
int run_stage2(const GemvArgs& a) {
    if (int s = launch_stage2<T>(a)) return s;
    return check_launch("nq_gemv stage 2");
}

}  // namespace
}  // namespace nq

extern "C" {

int nq_gemv(int dtype, const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid,
            const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n, int64_t r, int64_t m,
            void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    GemvArgs a;
    const int s = setup_gemv("nq_gemv", kBoth, dtype, x, s_in, v_bits, s_mid, u_bits, s_out, y, batch, n, r, m,
                             workspace, workspace_bytes, stream, a);
    if (s != NQ_OK) return s < 0 ? NQ_OK : s;
    return dtype == NQ_F16 ? run_gemv<F16>(a) : run_gemv<BF16>(a);
}

int nq_gemv_stage1(int dtype, const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid,
                   int64_t batch, int64_t n, int64_t r, int64_t m, void* workspace, size_t workspace_bytes,
                   nq_stream_t stream) {
    GemvArgs a;
    const int s = setup_gemv("nq_gemv_stage1", kStage1, dtype, x, s_in, v_bits, s_mid, nullptr, nullptr, nullptr,
                             batch, n, r, m, workspace, workspace_bytes, stream, a);
    if (s != NQ_OK) return s < 0 ? NQ_OK : s;
    return dtype == NQ_F16 ? run_stage1<F16>(a) : run_stage1<BF16>(a);
}

int nq_gemv_stage2(int dtype, const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n, int64_t r,
                   int64_t m, void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    GemvArgs a;
    const int s = setup_gemv("nq_gemv_stage2", kStage2, dtype, nullptr, nullptr, nullptr, nullptr, u_bits, s_out, y,
                             batch, n, r, m, workspace, workspace_bytes, stream, a);
    if (s != NQ_OK) return s < 0 ? NQ_OK : s;
    return dtype == NQ_F16 ? run_stage2<F16>(a) : run_stage2<BF16>(a);
}

}  // extern "C"

// --------------------------------------------------------------------------- GEMV without allocation
//
// nq_gemv_noalloc runs nq_gemv's two launches with the workspace in `scratch`, a file-scope
// device array each GPU holds for the life of the process. In host code `scratch` names a
// host-side stand-in, not device memory: the device address is fetched once per device with
// hipGetSymbolAddress (with that device current) and only that address is ever passed on.
// Every call on one GPU shares that GPU's array; stage 1 rewrites every element stage 2 reads
// on each call, so nothing is cleared between calls. Calls that overlap on one GPU race.
static __device__ __align__(256) unsigned char scratch[NQ_GEMV_NOALLOC_SCRATCH_BYTES];

namespace nq {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's address of `scratch` (looked up on the first call on that device).
int scratch_of_current_device(const char* name, void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(NQ_ERR_HIP, "%s: hipGetDevice: %s", name, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(NQ_ERR_UNSUPPORTED, "%s: device %d is beyond the %d this build tracks", name, dev,
                    kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        // the first call on a device may come inside a caller's stream capture: the lookup is no
        // stream operation, and the thread's capture mode is relaxed around it
        void* p = nullptr;
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        const hipError_t ex = hipThreadExchangeStreamCaptureMode(&mode);
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (ex == hipSuccess) (void)hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess || p == nullptr)
            return fail(NQ_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", name, dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return NQ_OK;
}

}  // namespace
}  // namespace nq

extern "C" {

int nq_gemv_noalloc(int dtype, const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid,
                    const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n, int64_t r,
                    int64_t m, nq_stream_t stream) {
    const char* name = "nq_gemv_noalloc";
    if (batch < 0 || n < 0 || r < 0 || m < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: negative size", name);
    const size_t need = gemv_base_bytes(batch, r);
    if (need > static_cast<size_t>(NQ_GEMV_NOALLOC_SCRATCH_BYTES))
        return fail(NQ_ERR_WORKSPACE, "%s: batch %lld at rank %lld needs %zu bytes of scratch, the static buffer "
                    "holds %zu", name, (long long)batch, (long long)r, need,
                    static_cast<size_t>(NQ_GEMV_NOALLOC_SCRATCH_BYTES));
    void* ws = nullptr;
    if (int s = scratch_of_current_device(name, &ws)) return s;
    GemvArgs a;
    const int s = setup_gemv(name, kBoth, dtype, x, s_in, v_bits, s_mid, u_bits, s_out, y, batch, n, r, m, ws,
                             NQ_GEMV_NOALLOC_SCRATCH_BYTES, stream, a);
    if (s != NQ_OK) return s < 0 ? NQ_OK : s;
    return dtype == NQ_F16 ? run_gemv<F16>(a) : run_gemv<BF16>(a);
}

}  // extern "C"

// --------------------------------------------------------------------------- grouped calls

namespace nq {
namespace {

// Workspace of a group: the header, then each item's (hi, lo) intermediate in item order.
struct GroupLayout {
    Plan plan[kMaxItems];
    uint16_t* z_hi[kMaxItems];
    uint16_t* z_lo[kMaxItems];
    size_t bytes;
};

int group_layout(const char* name, int64_t count, const nq_gemv_item* items, int64_t batch, void* workspace,
                 GroupLayout& g) {
    if (count < 1 || count > kMaxItems || !items)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: count must be 1..%d with an item array, got %lld", name, kMaxItems,
                    (long long)count);
    size_t off = kHeaderBytes;
    for (int64_t k = 0; k < count; ++k) {
        const int64_t r = items[k].r;
        if (r <= 0 || r > INT32_MAX / 4 || batch * plan_of(r).zpitch > INT32_MAX / 4)
            return fail(NQ_ERR_SHAPE, "%s: item %lld has rank %lld (needs 1 .. 2^29)", name, (long long)k,
                        (long long)r);
        g.plan[k] = plan_of(r);
        const size_t zb = z_bytes(batch, g.plan[k]);
        char* base = static_cast<char*>(workspace);
        g.z_hi[k] = base ? reinterpret_cast<uint16_t*>(base + off) : nullptr;
        g.z_lo[k] = base ? reinterpret_cast<uint16_t*>(base + off + zb) : nullptr;
        off += 2 * zb;
    }
    g.bytes = off;
    return NQ_OK;
}

int check_group_common(const char* name, int dtype, int64_t batch, void* workspace, size_t workspace_bytes,
                       const GroupLayout& g) {
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "%s: unsupported dtype %d", name, dtype);
    if (batch < 0 || batch > INT32_MAX / 4) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: bad batch %lld", name,
                                                        (long long)batch);
    if (!workspace) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null workspace", name);
    if (!aligned(workspace, 256)) return fail(NQ_ERR_ALIGNMENT, "%s: workspace must be 256-byte aligned", name);
    if (workspace_bytes < g.bytes)
        return fail(NQ_ERR_WORKSPACE, "%s: workspace has %zu bytes, needs %zu", name, workspace_bytes, g.bytes);
    return NQ_OK;
}

}  // namespace
}  // namespace nq

extern "C" {

size_t nq_gemv_group_workspace_bytes(int64_t count, const nq_gemv_item* items, int64_t batch) {
    GroupLayout g;
    if (batch < 0 || group_layout("nq_gemv_group_workspace_bytes", count, items, batch, nullptr, g) != NQ_OK) return 0;
    return g.bytes;
}

int nq_gemv_group_stage1(int dtype, int64_t count, const nq_gemv_item* items, const void* x, int64_t batch, int64_t n,
                         float rms_eps, void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    const char* name = "nq_gemv_group_stage1";
    GroupLayout g;
    if (int s = group_layout(name, count, items, batch, workspace, g)) return s;
    if (int s = check_group_common(name, dtype, batch, workspace, workspace_bytes, g)) return s;
    if (n <= 0 || n > INT32_MAX / 4 || batch * n > INT32_MAX / 4)
        return fail(NQ_ERR_SHAPE, "%s: bad n %lld", name, (long long)n);
    if (batch == 0) return NQ_OK;
    const int wn = static_cast<int>(ceil_div(n, 32));
    const auto* xp = static_cast<const uint16_t*>(x);
    if (!x) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null x", name);
    S1Table tab;
    tab.count = static_cast<int>(count);
    for (int64_t k = 0; k < count; ++k) {
        const nq_gemv_item& in = items[k];
        if (!in.v_bits || !in.s_in) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: item %lld: null pointer", name, (long long)k);
        if (in.r * ceil_div(n, 32) > INT32_MAX / 4) return fail(NQ_ERR_UNSUPPORTED, "%s: item too large", name);
        if (!aligned(in.v_bits, 4) || (in.s_mid && !aligned(in.s_mid, 2)))
            return fail(NQ_ERR_ALIGNMENT, "%s: item %lld: misaligned operand", name, (long long)k);
        if (!s1w_applies(xp, static_cast<const uint16_t*>(in.s_in), static_cast<int>(n), wn, static_cast<int>(in.r)))
            return fail(NQ_ERR_UNSUPPORTED,
                        "%s: needs n %% 8 == 0, 8 <= n <= 32768 and 16-byte aligned x and s_in (item %lld)", name,
                        (long long)k);
        S1Item& it = tab.item[k];
        it.v_bits = in.v_bits;
        it.s_in = static_cast<const uint16_t*>(in.s_in);
        it.s_mid = static_cast<const uint16_t*>(in.s_mid);
        it.z_hi = g.z_hi[k];
        it.z_lo = g.z_lo[k];
        it.r = static_cast<int>(in.r);
        it.kpad = g.plan[k].kpad;
        it.zpitch = g.plan[k].zpitch;
        it.blocks = 0;
    }
    const bool norm = rms_eps >= 0.0f;
    if (dtype == NQ_F16)
        launch_stage1_table<F16>(tab, xp, static_cast<int>(batch), static_cast<int>(n), wn, norm, rms_eps,
                                 as_stream(stream));
    else
        launch_stage1_table<BF16>(tab, xp, static_cast<int>(batch), static_cast<int>(n), wn, norm, rms_eps,
                                  as_stream(stream));
    return check_launch(name);
}

}  // extern "C"

namespace nq {
namespace {

// The group stage 2 with any epilogue; `rope` (kEpiRope, kEpiKv) carries the rotary step, the caches
// and what the store does with each of the three items (S2Item::rope).
struct RopeArgs {
    S2Rope rope;
    uint16_t* k_cache;
    uint16_t* v_cache;
    int kind[3];
};

int group_stage2(const char* name, int dtype, int64_t count, const nq_gemv_item* items, int64_t batch, int epilogue,
                 const RopeArgs* rope, void* workspace, size_t workspace_bytes, nq_stream_t stream);

}  // namespace
}  // namespace nq

extern "C" {

int nq_gemv_group_stage2(int dtype, int64_t count, const nq_gemv_item* items, int64_t batch, int epilogue,
                         void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    return group_stage2("nq_gemv_group_stage2", dtype, count, items, batch, epilogue, nullptr, workspace,
                        workspace_bytes, stream);
}

int nq_gemv_group_stage2_rope(int dtype, const nq_gemv_item* items, int64_t batch, void* k_cache, void* v_cache,
                              const void* rope_cos, const void* rope_sin, const int64_t* position, int64_t head_dim,
                              int64_t max_len, void* scores_mask, void* workspace, size_t workspace_bytes,
                              nq_stream_t stream) {
    const char* name = "nq_gemv_group_stage2_rope";
    if (!items) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null items", name);
    if (head_dim < 16 || head_dim % 16 || max_len <= 0 || max_len > INT32_MAX / 2)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: head_dim must be a positive multiple of 16 and max_len positive",
                    name);
    for (int k = 0; k < 3; ++k)
        if (items[k].m % head_dim)
            return fail(NQ_ERR_SHAPE, "%s: item %d: m %lld is not whole heads of %lld", name, k,
                        (long long)items[k].m, (long long)head_dim);
    if (items[1].m != items[2].m) return fail(NQ_ERR_SHAPE, "%s: the key and value items differ in m", name);
    if (batch > 0 && (!k_cache || !v_cache || !rope_cos || !rope_sin || !position))
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(k_cache, 2) || !aligned(v_cache, 2) || !aligned(rope_cos, 2) || !aligned(rope_sin, 2) ||
        !aligned(position, 8))
        return fail(NQ_ERR_ALIGNMENT, "%s: misaligned operand", name);
    if (batch * (items[1].m / head_dim) * max_len * head_dim > ((int64_t)1 << 40))
        return fail(NQ_ERR_UNSUPPORTED, "%s: caches too large", name);
    if (scores_mask && (!aligned(scores_mask, 2) || items[0].m % items[1].m ||
                        batch * (items[0].m / head_dim) * max_len >= ((int64_t)1 << 31)))
        return fail(NQ_ERR_SHAPE, "%s: the scores mask needs whole query groups per kv head, fewer than 2^31 elements "
                                  "and 2-byte alignment", name);
    RopeArgs ra;
    ra.rope.pos = position;
    ra.rope.cos = static_cast<const uint16_t*>(rope_cos);
    ra.rope.sin = static_cast<const uint16_t*>(rope_sin);
    ra.rope.head_dim = static_cast<int>(head_dim);
    ra.rope.max_len = static_cast<int>(max_len);
    ra.rope.mask = static_cast<uint16_t*>(scores_mask);
    ra.rope.mask_total = scores_mask ? static_cast<uint32_t>(batch * (items[0].m / head_dim) * max_len) : 0u;
    ra.rope.mask_groups = scores_mask ? static_cast<int>(items[0].m / items[1].m) : 1;
    ra.k_cache = static_cast<uint16_t*>(k_cache);
    ra.v_cache = static_cast<uint16_t*>(v_cache);
    ra.kind[0] = 1;  // q rotated into its output
    ra.kind[1] = 2;  // k rotated into the key cache
    ra.kind[2] = 3;  // v copied into the value cache
    return group_stage2(name, dtype, 3, items, batch, -1, &ra, workspace, workspace_bytes, stream);
}

int nq_gemv_group_stage2_kv(int dtype, const nq_gemv_item* items, int64_t batch, void* v_cache,
                            const int64_t* position, int64_t head_dim, int64_t max_len, void* workspace,
                            size_t workspace_bytes, nq_stream_t stream) {
    const char* name = "nq_gemv_group_stage2_kv";
    if (!items) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null items", name);
    if (head_dim < 16 || head_dim % 16 || max_len <= 0 || max_len > INT32_MAX / 2)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: head_dim must be a positive multiple of 16 and max_len positive",
                    name);
    for (int k = 0; k < 3; ++k)
        if (items[k].m % head_dim)
            return fail(NQ_ERR_SHAPE, "%s: item %d: m %lld is not whole heads of %lld", name, k,
                        (long long)items[k].m, (long long)head_dim);
    if (batch > 0 && (!v_cache || !position)) return fail(NQ_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
    if (!aligned(v_cache, 2) || !aligned(position, 8)) return fail(NQ_ERR_ALIGNMENT, "%s: misaligned operand", name);
    if (batch * (items[2].m / head_dim) * max_len * head_dim > ((int64_t)1 << 40))
        return fail(NQ_ERR_UNSUPPORTED, "%s: cache too large", name);
    RopeArgs ra;
    ra.rope = S2Rope{position, nullptr, nullptr, static_cast<int>(head_dim), static_cast<int>(max_len), nullptr, 0u, 1};
    ra.k_cache = nullptr;
    ra.v_cache = static_cast<uint16_t*>(v_cache);
    ra.kind[0] = 0;  // q stored into its output
    ra.kind[1] = 0;  // k stored into its output
    ra.kind[2] = 3;  // v copied into the value cache
    return group_stage2(name, dtype, 3, items, batch, -1, &ra, workspace, workspace_bytes, stream);
}

}  // extern "C"

namespace nq {
namespace {

int group_stage2(const char* name, int dtype, int64_t count, const nq_gemv_item* items, int64_t batch, int epilogue,
                 const RopeArgs* rope, void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    GroupLayout g;
    if (int s = group_layout(name, count, items, batch, workspace, g)) return s;
    if (int s = check_group_common(name, dtype, batch, workspace, workspace_bytes, g)) return s;
    if (rope == nullptr && epilogue != NQ_EPI_STORE && epilogue != NQ_EPI_RESIDUAL && epilogue != NQ_EPI_GATED)
        return fail(NQ_ERR_INVALID_ARGUMENT, "%s: unknown epilogue %d", name, epilogue);
    if (epilogue == NQ_EPI_GATED && (count != 2 || items[0].m != items[1].m || items[0].r != items[1].r))
        return fail(NQ_ERR_SHAPE, "%s: the gated epilogue takes two items (gate, up) of equal m and r", name);
    if (batch == 0) return NQ_OK;
    S2Item all[kMaxItems];
    for (int64_t k = 0; k < count; ++k) {
        const nq_gemv_item& in = items[k];
        const int64_t m = in.m;
        if (m <= 0 || m > INT32_MAX / 4 || m * ceil_div(in.r, 32) > INT32_MAX / 4 || in.y_stride < m ||
            batch * in.y_stride > INT32_MAX / 4)
            return fail(NQ_ERR_SHAPE, "%s: item %lld: bad m %lld or y_stride %lld", name, (long long)k, (long long)m,
                        (long long)in.y_stride);
        if (!in.u_bits || !in.s_out || !in.y || (epilogue == NQ_EPI_RESIDUAL && !in.resid))
            return fail(NQ_ERR_INVALID_ARGUMENT, "%s: item %lld: null pointer", name, (long long)k);
        if (!aligned(in.s_out, 2) || !aligned(in.y, 2) || (in.resid && !aligned(in.resid, 2)))
            return fail(NQ_ERR_ALIGNMENT, "%s: item %lld: misaligned operand", name, (long long)k);
        if (!s2t_applies(g.z_hi[k], g.z_lo[k], in.u_bits, static_cast<int>(m), g.plan[k]))
            return fail(NQ_ERR_UNSUPPORTED, "%s: needs 16-byte aligned u_bits, r <= 4608 and m * ceil(r/32) >= 4 "
                        "(item %lld)", name, (long long)k);
        S2Item& it = all[k];
        it.u_bits = in.u_bits;
        it.s_out = static_cast<const uint16_t*>(in.s_out);
        it.y = static_cast<uint16_t*>(in.y);
        it.resid = static_cast<const uint16_t*>(in.resid);
        it.z_hi = g.z_hi[k];
        it.z_lo = g.z_lo[k];
        it.m = static_cast<int>(m);
        it.wr = g.plan[k].wr;
        it.zpitch = g.plan[k].zpitch;
        it.ystride = static_cast<int>(in.y_stride);
        it.blocks = 0;
        it.rope = rope == nullptr ? 0 : rope->kind[k];
        it.cache = rope == nullptr ? nullptr : (it.rope == 2 ? rope->k_cache : it.rope == 3 ? rope->v_cache : nullptr);
    }
    // one launch per class of items that share the stage-2 word split (equal ranks always do)
    const int b = static_cast<int>(batch);
    hipStream_t st = as_stream(stream);
    bool done[kMaxItems] = {false, false, false, false};
    for (int64_t k0 = 0; k0 < count; ++k0) {
        if (done[k0]) continue;
        const int qw = g.plan[k0].s2_qw;
        S2Table tab;
        tab.count = 0;
        tab.rope = rope != nullptr ? rope->rope : S2Rope{nullptr, nullptr, nullptr, 0, 0};
        for (int64_t k = k0; k < count; ++k)
            if (!done[k] && g.plan[k].s2_qw == qw) {
                tab.item[tab.count++] = all[k];
                done[k] = true;
            }
        bool ok;
        if (rope != nullptr && rope->rope.cos == nullptr) {  // nq_gemv_group_stage2_kv
            ok = dtype == NQ_F16 ? launch_s2t_qw<F16, kEpiKv>(tab, qw, b, st)
                                 : launch_s2t_qw<BF16, kEpiKv>(tab, qw, b, st);
        } else if (rope != nullptr) {
            ok = dtype == NQ_F16 ? launch_s2t_qw<F16, kEpiRope>(tab, qw, b, st)
                                 : launch_s2t_qw<BF16, kEpiRope>(tab, qw, b, st);
        } else if (dtype == NQ_F16) {
            ok = epilogue == NQ_EPI_STORE      ? launch_s2t_qw<F16, kEpiStore>(tab, qw, b, st)
                 : epilogue == NQ_EPI_RESIDUAL ? launch_s2t_qw<F16, kEpiResidual>(tab, qw, b, st)
                                               : launch_s2t_qw<F16, kEpiGated>(tab, qw, b, st);
        } else {
            ok = epilogue == NQ_EPI_STORE      ? launch_s2t_qw<BF16, kEpiStore>(tab, qw, b, st)
                 : epilogue == NQ_EPI_RESIDUAL ? launch_s2t_qw<BF16, kEpiResidual>(tab, qw, b, st)
                                               : launch_s2t_qw<BF16, kEpiGated>(tab, qw, b, st);
        }
        if (!ok) return fail(NQ_ERR_UNSUPPORTED, "%s: no stage-2 configuration for this rank", name);
        if (int s = check_launch(name)) return s;
    }
    return NQ_OK;
}

}  // namespace
}  // namespace nq
