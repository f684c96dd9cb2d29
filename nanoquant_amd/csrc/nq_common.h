// Shared device and host helpers of the gfx950 NanoQuant kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <string>

#include "../../include/nq_hip.h"

namespace nq {

// ----------------------------------------------------------------------------- host side

// Records the detail of the last failure on this thread; returns `status`.
int fail(int status, const char* fmt, ...);
// Checks the launch that was just enqueued.
int check_launch(const char* what);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline hipStream_t as_stream(nq_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ----------------------------------------------------------------------------- element types

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Storage of both 16-bit float formats is uint16_t; the tag selects the arithmetic.
struct F16 {
    static constexpr uint32_t ONE_PAIR = 0x3C003C00u;  // (+1.0, +1.0)
    static constexpr float SAT = 64504.0f;              // GEMV saturation of the reference (cuda_utils.cuh:84-86)
    static constexpr float SAT_GEMM = 65504.0f;         // GEMM saturation of the reference (gemm_kernel.cu:124-126)
    __device__ static inline float to_float(uint16_t v) {
        return static_cast<float>(__builtin_bit_cast(_Float16, v));
    }
    __device__ static inline uint16_t from_float(float f) {
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
    }
    // a.lo*b.lo + a.hi*b.hi + c, products exact, fp32 sum.
    __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
    }
};

struct BF16 {
    static constexpr uint32_t ONE_PAIR = 0x3F803F80u;
    static constexpr float SAT = 3.3895313892515355e+38f;  // largest finite bf16
    static constexpr float SAT_GEMM = 3.3895313892515355e+38f;
    __device__ static inline float to_float(uint16_t v) {
        return __builtin_bit_cast(float, static_cast<uint32_t>(v) << 16);
    }
    __device__ static inline uint16_t from_float(float f) {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
    }
    __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                               false);
    }
};

// v_mfma_f32_16x16x32_{f16,bf16}: lane l holds A[row l%16][k 8(l/16)..+7], B[k 8(l/16)..+7][col l%16]
// as four dwords of two 16-bit values each, and C[rows 4(l/16)..+3][col l%16].
template <typename T>
__device__ inline f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);

template <>
__device__ inline f32x4 mfma16x16x32<F16>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

template <>
__device__ inline f32x4 mfma16x16x32<BF16>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}

// v_mfma_f32_32x32x16_{f16,bf16}: lane l holds A[row l%32][k 8(l/32)..+7], B[k 8(l/32)..+7][col l%32]
// as four dwords each, and C[row 8(i/4) + 4(l/32) + i%4][col l%32] in register i (i < 16).
template <typename T>
__device__ inline f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c);

template <>
__device__ inline f32x16 mfma32x32x16<F16>(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

template <>
__device__ inline f32x16 mfma32x32x16<BF16>(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}

// (a & mask) | b in one v_and_or_b32; mask and b live in VGPRs (a VOP3 operand cannot take two
// non-inline constants on this target), so the compiler keeps them in registers across a loop.
__device__ inline uint32_t and_or(uint32_t a, uint32_t mask, uint32_t b) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "v"(b));
    return r;
}

// (a & mask) | (b & ~mask) in one v_bfi_b32.
__device__ inline uint32_t bit_select(uint32_t mask, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(a), "v"(b));
    return r;
}

// Buffer resource over `bytes` bytes at `base` (raw, stride 0): a load at or past `bytes` returns
// zero, and offsets are 32-bit (no 64-bit address arithmetic per lane). The last word is the
// gfx9 data-format field for untyped 32-bit access.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ inline rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ inline u32x4 load_b128(rsrc_t rs, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(offset), 0, 0));
}
// Streaming loads (read once: non-temporal)
__device__ inline uint32_t load_b32_stream(rsrc_t rs, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(offset), 0, 2);
}
__device__ inline u32x4 load_b128_stream(rsrc_t rs, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(offset), 0, 2));
}

// DMA of 16 / 4 bytes a lane from global memory into LDS (global_load_lds): a wave's lanes land in
// consecutive slots from `lds` (which must be the same for every lane of the wave).
__device__ inline void dma16(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ inline void dma4(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}

// LDS byte address of a pointer into __shared__ memory.
__device__ inline uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// The same DMAs issued from inline assembly, which the compiler does not track: 16 / 4 bytes a lane
// from base + voff (base wave-uniform, voff a byte offset per lane) into LDS at the wave-uniform
// byte address lds, lane after lane. A DMA issued through the builtin counts, for the compiler's
// wait insertion, as an LDS event whose completion order it cannot know, so wherever a later LDS
// read's data is needed it waits for every outstanding LDS read (lgkmcnt 0): a read issued early
// for the next k tile is drained at the current tile's first use. With the DMAs untracked, LDS reads
// get partial waits. The caller waits for these DMAs itself (wait_vmcnt: the compiler's own vmcnt
// waits count only the loads it knows, so they can only wait longer than needed) and orders them
// against LDS reads with barrier_keep_dma. M0 is written without being declared: on gfx950 the
// compiler uses it only to set up LDS DMAs, and a kernel that calls these calls no builtin DMA.
__device__ inline void dma16_lds(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds) : "memory");
}
__device__ inline void dma4_lds(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds) : "memory");
}

// Waits until at most N of this wave's vector-memory operations (loads, DMAs) are outstanding;
// they complete in issue order.
template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt has 6 bits");
    // gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14; expcnt (6:4) and lgkmcnt (11:8) not waited on
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier for DMA pipelines. __syncthreads() carries workgroup-scope fences, and the
// release fence makes the compiler wait for every outstanding vector-memory operation (vmcnt 0),
// LDS DMAs issued for later steps included, which empties a multi-buffered pipeline at every
// step. Here each wave first waits (wait_vmcnt) for its DMAs that the next step reads; this
// function then waits for the wave's own LDS reads (lgkmcnt 0) and meets the other waves at
// s_barrier. The LDS wait matters: the compiler places the wait for a read's data next to its
// first use, which may come after the barrier, and a wave past the barrier may start a DMA into
// the buffer that a slower wave's reads (still queued behind bank conflicts) have yet to see.
// The empty asm statements with a memory clobber keep the compiler from moving any memory access
// across the barrier.
__device__ inline void barrier_keep_dma() {
    asm volatile("" ::: "memory");
    // gfx9 s_waitcnt: lgkmcnt (11:8) zero; vmcnt (3:0, 15:14) and expcnt (6:4) at their maximum
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <typename T>
__device__ inline uint16_t saturate_to(float v, float sat) {
    v = fminf(fmaxf(v, -sat), sat);  // as the reference's clamp: a NaN input becomes -sat
    return T::from_float(v);
}

// ----------------------------------------------------------------------------- wave helpers

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace nq
