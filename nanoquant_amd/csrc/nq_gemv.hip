// Decode GEMV: y = sat(s_out * (U * ((V * (s_in * x)) * s_mid))) with +-1 factors held as
// half2-ordered sign words (element j of a 32-column block at bit 15 - j/2 + 16*(j%2)).
//
// Two launches on the caller's stream:
//   stage 1  h[b, j] = s_mid[j] * sum_k sign(V[j,k]) * s_in[k] * x[b,k]     (fp32, in the workspace)
//   stage 2  y[b, i] = sat(s_out[i] * sum_j sign(U[i,j]) * h[b,j])
// One wave owns one output row and its lanes stride the row's words, so each
// weight word is read once per launch for up to kMaxNB batch rows. Stage 1 flips
// the sign bits of (s_in[k], s_in[k+1]) pairs with the word's bit pair and feeds
// v_dot2 (exact fp16/bf16 products, fp32 sum); stage 2 flips the sign bit of the
// fp32 intermediate and adds. Everything accumulates in fp32.
#include "nq_common.h"

namespace nq {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxNB = 8;
constexpr size_t kHeaderBytes = 256;  // reserved words at the start of the workspace

// Bit of element e (0..31) of a half2 word.
__device__ inline int half2_bit(int e) { return 15 - (e >> 1) + 16 * (e & 1); }

// v with its sign bit xor-ed with bit 31 of `mask`. Takes the float by value: a bit
// cast applied directly to an ext_vector element reads the wrong element with this
// compiler, so vector lanes are always copied to a scalar first.
__device__ inline float flip_sign(float v, uint32_t mask) { return __uint_as_float(__float_as_uint(v) ^ mask); }

template <typename T, int NB, bool kVec>
__global__ __launch_bounds__(kThreads) void gemv_stage1_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ s_in,
                                                               const uint32_t* __restrict__ vbits,
                                                               const uint16_t* __restrict__ s_mid,
                                                               float* __restrict__ h, int batch, int n, int r,
                                                               int wn, int h_stride) {
    const int lane = threadIdx.x & 63;
    const int j = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (j >= r) return;
    const int b0 = blockIdx.y * NB;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    const uint32_t* row = vbits + static_cast<size_t>(j) * wn;
    for (int w = lane; w < wn; w += 64) {
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
    const float mid = s_mid != nullptr ? T::to_float(s_mid[j]) : 1.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float v = wave_sum(acc[b]);
        if (lane == 0 && b0 + b < batch) h[static_cast<size_t>(b0 + b) * h_stride + j] = v * mid;
    }
}

template <typename T, int NB>
__global__ __launch_bounds__(kThreads) void gemv_stage2_kernel(const float* __restrict__ h,
                                                               const uint32_t* __restrict__ ubits,
                                                               const uint16_t* __restrict__ s_out,
                                                               uint16_t* __restrict__ y, int batch, int r, int m,
                                                               int wr, int h_stride) {
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (i >= m) return;
    const int b0 = blockIdx.y * NB;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    const uint32_t* row = ubits + static_cast<size_t>(i) * wr;
    for (int w = lane; w < wr; w += 64) {
        const uint32_t bits = __builtin_nontemporal_load(row + w);
        const int j0 = w * 32;
        if (j0 + 32 <= r) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b0 + b < batch) {
                    const float* hr = h + static_cast<size_t>(b0 + b) * h_stride + j0;
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const f32x4 v = *reinterpret_cast<const f32x4*>(hr + 4 * q);
                        // elements 4q..4q+3 = pairs p = 2q, 2q+1: lo of pair p at bit 15-p, hi at bit 31-p
                        const uint32_t t0 = bits << (2 * q);
                        const uint32_t t1 = bits << (2 * q + 1);
                        acc[b] += flip_sign(v.x, (t0 << 16) & 0x80000000u);
                        acc[b] += flip_sign(v.y, t0 & 0x80000000u);
                        acc[b] += flip_sign(v.z, (t1 << 16) & 0x80000000u);
                        acc[b] += flip_sign(v.w, t1 & 0x80000000u);
                    }
                }
            }
        } else {
            const int valid = r - j0;
            for (int e = 0; e < valid; ++e) {
                const bool neg = (bits >> half2_bit(e)) & 1u;
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    if (b0 + b < batch) {
                        const float hv = h[static_cast<size_t>(b0 + b) * h_stride + j0 + e];
                        acc[b] += neg ? -hv : hv;
                    }
                }
            }
        }
    }
    const float so = T::to_float(s_out[i]);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float v = wave_sum(acc[b]);
        if (lane == 0 && b0 + b < batch) y[static_cast<size_t>(b0 + b) * m + i] = saturate_to<T>(v * so, T::SAT);
    }
}

inline int64_t h_stride_of(int64_t r) { return ceil_div(r, 32) * 32; }

template <typename T, int NB>
int launch_gemv(const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid, const uint32_t* u_bits,
                const void* s_out, void* y, int64_t batch, int64_t n, int64_t r, int64_t m, float* h,
                hipStream_t stream) {
    const int wn = static_cast<int>(ceil_div(n, 32));
    const int wr = static_cast<int>(ceil_div(r, 32));
    const int hs = static_cast<int>(h_stride_of(r));
    const unsigned gy = static_cast<unsigned>(ceil_div(batch, NB));
    const bool vec = (n % 8 == 0) && aligned(x, 16) && aligned(s_in, 16);
    const dim3 g1(static_cast<unsigned>(ceil_div(r, kWaves)), gy);
    if (r == 0) {
        // no rank: h is empty and stage 2 sums nothing
    } else if (vec)
        gemv_stage1_kernel<T, NB, true><<<g1, kThreads, 0, stream>>>(
            static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(s_in), v_bits,
            static_cast<const uint16_t*>(s_mid), h, (int)batch, (int)n, (int)r, wn, hs);
    else
        gemv_stage1_kernel<T, NB, false><<<g1, kThreads, 0, stream>>>(
            static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(s_in), v_bits,
            static_cast<const uint16_t*>(s_mid), h, (int)batch, (int)n, (int)r, wn, hs);
    if (r > 0)
        if (int s = check_launch("nq_gemv stage 1")) return s;
    const dim3 g2(static_cast<unsigned>(ceil_div(m, kWaves)), gy);
    gemv_stage2_kernel<T, NB><<<g2, kThreads, 0, stream>>>(h, u_bits, static_cast<const uint16_t*>(s_out),
                                                           static_cast<uint16_t*>(y), (int)batch, (int)r, (int)m, wr,
                                                           hs);
    return check_launch("nq_gemv stage 2");
}

template <typename T>
int dispatch_nb(const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid, const uint32_t* u_bits,
                const void* s_out, void* y, int64_t batch, int64_t n, int64_t r, int64_t m, float* h,
                hipStream_t stream) {
    if (batch <= 1) return launch_gemv<T, 1>(x, s_in, v_bits, s_mid, u_bits, s_out, y, batch, n, r, m, h, stream);
    if (batch <= 2) return launch_gemv<T, 2>(x, s_in, v_bits, s_mid, u_bits, s_out, y, batch, n, r, m, h, stream);
    if (batch <= 4) return launch_gemv<T, 4>(x, s_in, v_bits, s_mid, u_bits, s_out, y, batch, n, r, m, h, stream);
    return launch_gemv<T, kMaxNB>(x, s_in, v_bits, s_mid, u_bits, s_out, y, batch, n, r, m, h, stream);
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" {

size_t nq_gemv_workspace_bytes(int64_t batch, int64_t n, int64_t r, int64_t m) {
    (void)n;
    (void)m;
    if (batch < 0 || r < 0) return 0;
    const size_t h_bytes = static_cast<size_t>(batch) * static_cast<size_t>(h_stride_of(r)) * sizeof(float);
    return kHeaderBytes + (h_bytes + 255) / 256 * 256;
}

int nq_gemv(int dtype, const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid,
            const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n, int64_t r, int64_t m,
            void* workspace, size_t workspace_bytes, nq_stream_t stream) {
    if (dtype != NQ_F16 && dtype != NQ_BF16) return fail(NQ_ERR_DTYPE, "nq_gemv: unsupported dtype %d", dtype);
    if (batch < 0 || n < 0 || r < 0 || m < 0) return fail(NQ_ERR_INVALID_ARGUMENT, "nq_gemv: negative size");
    if (n > INT32_MAX / 2 || r > INT32_MAX / 2 || m > INT32_MAX / 2 || batch > INT32_MAX / 2)
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
    float* h = reinterpret_cast<float*>(static_cast<char*>(workspace) + kHeaderBytes);
    hipStream_t st = as_stream(stream);
    if (dtype == NQ_F16) return dispatch_nb<F16>(x, s_in, v_bits, s_mid, u_bits, s_out, y, batch, n, r, m, h, st);
    return dispatch_nb<BF16>(x, s_in, v_bits, s_mid, u_bits, s_out, y, batch, n, r, m, h, st);
}

}  // extern "C"
