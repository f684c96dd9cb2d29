/*
 * nq_hip.h - C ABI of the MI355X (gfx950) NanoQuant inference kernels.
 *
 * Plain pointers and sizes only: every pointer is device memory on the current
 * HIP device of the calling thread, every call is enqueued on `stream` (a
 * hipStream_t passed as void*, NULL = the null stream) and never synchronises.
 * No entry point allocates: scratch comes from caller buffers whose sizes the
 * *_workspace_bytes queries give, except for nq_gemv_noalloc, whose scratch is a
 * static device array of the library. Calls are thread-safe except that two calls
 * sharing one workspace (or, for nq_gemv_noalloc, one GPU) must not overlap.
 *
 * Every entry point returns an nq_status; nq_status_string() names it and
 * nq_last_error_message() gives the detail of the last failure on this thread.
 *
 * Bit layouts (identical to the reference's packers):
 *   NQ_PACK_LSB_FIRST  element j of a 32-column block -> bit j
 *   NQ_PACK_HALF2      element j of a 32-column block -> bit 15 - j/2 + 16*(j%2)
 *   Marlin             element (o,k) of a [O,K] weight -> word (k/16, 32*(o/64) + 4*(o%8) + (k%8)/2),
 *                      bit 15 - 2*((o%16)/8) - (k%16)/8 + 16*(k%2) - 4*((o%64)/16)
 * A set bit means -1, a clear bit +1.
 */
#ifndef NQ_HIP_H
#define NQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* nq_stream_t;

typedef enum {
    NQ_OK = 0,
    NQ_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative size, unknown enum */
    NQ_ERR_SHAPE = 2,            /* sizes inconsistent with each other or with the layout */
    NQ_ERR_DTYPE = 3,            /* unsupported element type */
    NQ_ERR_ALIGNMENT = 4,        /* a pointer is not aligned as the layout needs */
    NQ_ERR_WORKSPACE = 5,        /* workspace smaller than the matching *_workspace_bytes */
    NQ_ERR_HIP = 6,              /* the HIP runtime reported an error (launch or device) */
    NQ_ERR_UNSUPPORTED = 7       /* valid request this build does not handle */
} nq_status;

typedef enum { NQ_F16 = 0, NQ_BF16 = 1 } nq_dtype;

typedef enum { NQ_PACK_LSB_FIRST = 0, NQ_PACK_HALF2 = 1 } nq_pack_method;

const char* nq_status_string(int status);
const char* nq_last_error_message(void);
/* Library version as 10000*major + 100*minor + patch. */
int nq_version(void);

/* ---------------------------------------------------------------- packing */

/* int8 {-1,+1} [rows, cols] (row-major) -> uint32 [rows, ceil(cols/32)].
 * Columns past `cols` in the last word are packed as +1 (bit 0). A value v is
 * packed as -1 iff v < 0.
 * Replaces pack_binary_gemv (src/nanoquant/kernel/utils.py:51-113). */
int nq_pack_signs(const int8_t* src, uint32_t* dst, int64_t rows, int64_t cols, int method,
                  nq_stream_t stream);

/* uint32 [rows, ceil(cols/32)] -> int8 {-1,+1} [rows, cols]; padding bits are ignored.
 * Replaces unpack_binary_gemv (src/nanoquant/kernel/utils.py:116-183). */
int nq_unpack_signs(const uint32_t* src, int8_t* dst, int64_t rows, int64_t cols, int method,
                    nq_stream_t stream);

/* Re-order the bits of packed words from one method to the other without
 * expanding them (on-disk lsb_first checkpoint words -> half2 kernel words).
 * Padding bits must be clear in `src` (as the packers leave them) and stay clear.
 * No reference counterpart as one call: replaces binary_unpacker (kernel/utils.py:116-183,
 * called at load time by utils/load_utils.py:392) followed by binary_packer(..., "half2")
 * (modules/linear.py:205-206). */
int nq_repack_signs(const uint32_t* src, uint32_t* dst, int64_t rows, int64_t cols, int src_method,
                    int dst_method, nq_stream_t stream);

/* int8 {-1,+1} weight [O, K] -> Marlin words uint32 [K/16, O/2]; O % 64 == 0, K % 16 == 0.
 * Replaces the weight part of pack_binary_marlin (src/nanoquant/kernel/utils.py:191-205). */
int nq_pack_marlin(const int8_t* weight, uint32_t* dst, int64_t O, int64_t K, nq_stream_t stream);

/* Marlin words [K/16, O/2] -> int8 {-1,+1} [O, K] (inverse of nq_pack_marlin; no reference
 * counterpart, used to check and to read packed GEMM weights back). */
int nq_unpack_marlin(const uint32_t* words, int8_t* weight, int64_t O, int64_t K, nq_stream_t stream);

/* Sign words of a {-1,+1} [O, K] matrix (`method` order, ceil(K/32) words a row, as a
 * checkpoint stores V [r, n] and U [m, r]) -> Marlin words uint32 [K_pad/16, O_pad/2] of the
 * matrix padded with +1 to [O_pad, K_pad] (O_pad % 64 == 0, K_pad % 16 == 0); bits past K in
 * `src` are ignored. No reference counterpart as one call: replaces binary_unpacker at load
 * (utils/load_utils.py:392) followed by the sign part of pack_binary_marlin_fused
 * (src/nanoquant/kernel/utils.py:262-277, rank padding included) in _prepare_kernel
 * (modules/linear.py:226-232). */
int nq_repack_marlin(const uint32_t* src, int64_t O, int64_t K, int method, uint32_t* dst, int64_t O_pad,
                     int64_t K_pad, nq_stream_t stream);

/* Scale permutations of pack_binary_marlin (src/nanoquant/kernel/utils.py:206-209), on
 * 16-bit elements: in  [K] -> out [K], natural 16c+8a+2b+d -> 16c+4b+2a+d (K % 16 == 0);
 *                  out [O] -> out [O], natural 32c+8a+2b+d -> 32c+8b+2a+d (O % 32 == 0).
 * Either pair of pointers may be NULL to skip that vector. */
int nq_permute_marlin_scales(const uint16_t* scale_in, uint16_t* scale_in_out, int64_t K,
                             const uint16_t* scale_out, uint16_t* scale_out_out, int64_t O,
                             nq_stream_t stream);

/* ---------------------------------------------------------------- decode GEMV */

/* Bytes of workspace nq_gemv needs: a header, the intermediate as bf16 hi/lo pairs and, for
 * batches whose stage 1 runs the batched k-split kernel, its per-range fp32 sums. That kernel runs
 * on rows of 256 or more words (n >= 8161), n % 32 == 0, up to 128 batch rows, from a batch set by
 * the words per row w = n / 32: w > 1024 from 1 row; 513 <= w <= 1024 from 2; w = 512 from 3;
 * 320 <= w <= 511 from 8; 256 <= w <= 319 from 8 when V holds fewer than 256 K words (r * w),
 * else from 16. This function is the authority: size workspaces from it, not from this list. A
 * workspace that holds the header and intermediate but not those sums is accepted and runs the
 * stage-1 kernels that keep none (results agree to rounding, not bit for bit). */
size_t nq_gemv_workspace_bytes(int64_t batch, int64_t n, int64_t r, int64_t m);

/* y[b, :] = sat(s_out * (U * ((V * (s_in * x[b, :])) * s_mid)))  for b < batch.
 *   x      dtype [batch, n]           s_in  dtype [n]
 *   v_bits uint32 [r, ceil(n/32)]     half2 words of V (+-1 [r, n])
 *   s_mid  dtype [r] or NULL
 *   u_bits uint32 [m, ceil(r/32)]     half2 words of U (+-1 [m, r])
 *   s_out  dtype [m]                  y     dtype [batch, m]
 * Accumulates in fp32; the intermediate is kept as a pair of bf16 values (hi + lo, 16
 * significant bits, fp32 range); fp16 outputs saturate at +-64504 as the reference GEMV does.
 * `workspace` must hold nq_gemv_workspace_bytes(batch, n, r, m) bytes, 256-byte aligned.
 * Replaces nanoquant_dyn_forward (src/nanoquant/kernel/cuda/gemv_kernel.cu:308-429;
 * declared at gemv.h:6-16, registered at pybind.cpp:85-90,110). */
int nq_gemv(int dtype, const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid,
            const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n, int64_t r,
            int64_t m, void* workspace, size_t workspace_bytes, nq_stream_t stream);

/* The two launches nq_gemv makes, one at a time, with the same arguments and workspace:
 * stage 1 writes the intermediate h of x into the workspace, stage 2 turns the workspace's h
 * into y. No counterpart in the reference (both are internal to nanoquant_dyn_forward,
 * gemv_kernel.cu:365-401); they exist to time and profile each launch on its own and for
 * callers that apply several U to one h. */
int nq_gemv_stage1(int dtype, const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid,
                   int64_t batch, int64_t n, int64_t r, int64_t m, void* workspace, size_t workspace_bytes,
                   nq_stream_t stream);
int nq_gemv_stage2(int dtype, const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n,
                   int64_t r, int64_t m, void* workspace, size_t workspace_bytes, nq_stream_t stream);

/* Bytes of the library's static GEMV scratch buffer on each GPU (4 MiB). */
#define NQ_GEMV_NOALLOC_SCRATCH_BYTES (4u << 20)

/* nq_gemv with no workspace argument and no allocation of any kind: the intermediate lives in
 * a static device array of NQ_GEMV_NOALLOC_SCRATCH_BYTES that each GPU holds until the process
 * ends. Same arguments (minus the workspace), kernels and results as nq_gemv, bit for bit,
 * whenever nq_gemv_workspace_bytes(batch, n, r, m) fits in the array; larger batched calls run
 * the stage-1 kernel that keeps no per-range sums (results agree with nq_gemv's to rounding).
 * Returns NQ_ERR_WORKSPACE, launching nothing, when the header and intermediate alone exceed
 * that size (batch > 630 at r = 1632, batch > 227 at r = 4608). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (concurrent streams or threads) race,
 * so order them on one stream. The first call on a device looks up the array's address there.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int nq_gemv_noalloc(int dtype, const void* x, const void* s_in, const uint32_t* v_bits, const void* s_mid,
                    const uint32_t* u_bits, const void* s_out, void* y, int64_t batch, int64_t n, int64_t r,
                    int64_t m, nq_stream_t stream);

/* ---------------------------------------------------------------- grouped decode GEMV
 *
 * Up to four linears in one launch per stage, for the decode step of a transformer layer:
 * q, k and v read the same input, so do gate and up. No counterpart in the reference, whose
 * decode step calls nanoquant_dyn_forward once per linear (modules/linear.py:156-160); the
 * arithmetic of each item is that of nq_gemv. `items` is a host array of `count` items. */
typedef struct nq_gemv_item {
    const uint32_t* v_bits; /* stage 1: half2 words of V, [r, ceil(n/32)] */
    const void* s_in;       /* stage 1: [n], 16-byte aligned */
    const void* s_mid;      /* stage 1: [r] or NULL */
    const uint32_t* u_bits; /* stage 2: half2 words of U, [m, ceil(r/32)], 16-byte aligned */
    const void* s_out;      /* stage 2: [m] */
    void* y;                /* stage 2: output, batch rows of y_stride elements */
    const void* resid;      /* stage 2 with NQ_EPI_RESIDUAL: same layout as y (may be y itself) */
    int64_t r;
    int64_t m;
    int64_t y_stride; /* elements between batch rows of y and resid, >= m */
} nq_gemv_item;

typedef enum {
    NQ_EPI_STORE = 0,    /* y = sat(s_out * acc) */
    NQ_EPI_RESIDUAL = 1, /* y = resid + sat(s_out * acc), each rounded to dtype as two operations */
    NQ_EPI_GATED = 2     /* two items (gate, up) of equal m and r: y of item 0 = silu(gate) * up */
} nq_epilogue;

/* Bytes of workspace the two grouped stages need for these items (0 on bad arguments). */
size_t nq_gemv_group_workspace_bytes(int64_t count, const nq_gemv_item* items, int64_t batch);

/* Stage 1 of every item over the shared input x [batch, n]. With rms_eps >= 0 the input is
 * RMS-normalised first: h is multiplied by rsqrt(mean(x^2) + rms_eps) per batch row; the
 * norm's weight is expected folded into each item's s_in. Needs n % 8 == 0, 8 <= n <= 32768, 16-byte
 * aligned x and s_in; NQ_ERR_UNSUPPORTED otherwise. */
int nq_gemv_group_stage1(int dtype, int64_t count, const nq_gemv_item* items, const void* x, int64_t batch,
                         int64_t n, float rms_eps, void* workspace, size_t workspace_bytes, nq_stream_t stream);

/* Stage 2 of every item from the workspace stage 1 filled, with one of the nq_epilogue
 * stores: one launch per set of items whose ranks share a kernel configuration (equal ranks
 * always do). Needs r <= 4608 and 16-byte aligned u_bits; NQ_ERR_UNSUPPORTED otherwise. */
int nq_gemv_group_stage2(int dtype, int64_t count, const nq_gemv_item* items, int64_t batch, int epilogue,
                         void* workspace, size_t workspace_bytes, nq_stream_t stream);

/* Stage 2 of the q, k and v projections of a decode step (items[0..2], after nq_gemv_group_stage1
 * over the same three items) with the rotary embedding and the KV-cache write folded into the
 * store: each projection output is rounded to dtype as NQ_EPI_STORE rounds it, then q is rotated
 * into items[0].y, k is rotated into k_cache[b, kvh, p, :] and v copied into v_cache[b, kvh, p, :]
 * ([batch, items[1].m / head_dim, max_len, head_dim] each), p = *position (device int64, read when
 * the kernel runs, so a graph replays it). rope_cos/rope_sin [max_len, head_dim]; the rotation is
 * nq_rope_kv_write's, bit for bit (outputs equal nq_gemv_group_stage2 with NQ_EPI_STORE followed by
 * nq_rope_kv_write). head_dim a multiple of 16; every m a multiple of head_dim; items[1].m ==
 * items[2].m. y of items 1 and 2 is not written (any valid pointer). A position outside
 * [0, max_len) zeroes q and writes no cache row. scores_mask (optional, NULL for none): the
 * attention scores buffer [batch * kv_heads, max_len, groups] (groups = items[0].m / items[1].m query
 * heads per kv head) into which the launch writes the step's additive causal mask, 0 for cache
 * positions <= *position and -inf after it, so that the scores product can add into it in place.
 * No counterpart in the reference (its decode step runs Hugging Face's rotary embedding, cache update
 * and mask, kernel/test_decode.py:385-402). */
int nq_gemv_group_stage2_rope(int dtype, const nq_gemv_item* items, int64_t batch, void* k_cache, void* v_cache,
                              const void* rope_cos, const void* rope_sin, const int64_t* position, int64_t head_dim,
                              int64_t max_len, void* scores_mask, void* workspace, size_t workspace_bytes,
                              nq_stream_t stream);

/* Stage 2 of the q, k and v projections of a decode step (items[0..2], after nq_gemv_group_stage1
 * over the same three items) with the value-cache write folded into the store, for a step whose
 * rotary embedding and key-cache write run elsewhere: q and k are stored into items[0].y and
 * items[1].y exactly as NQ_EPI_STORE stores them, v is rounded the same way and copied into
 * v_cache[b, kvh, p, :] ([batch, items[2].m / head_dim, max_len, head_dim]), p = *position (device
 * int64, read when the kernel runs, so a graph replays it); items[2].y is not written (any valid
 * pointer). A position outside [0, max_len) writes no cache row. head_dim a multiple of 16; every m
 * a multiple of head_dim. No counterpart in the reference (its decode step writes the cache in
 * Hugging Face's cache update, kernel/test_decode.py:385-402); it saves the step one launch. */
int nq_gemv_group_stage2_kv(int dtype, const nq_gemv_item* items, int64_t batch, void* v_cache,
                            const int64_t* position, int64_t head_dim, int64_t max_len, void* workspace,
                            size_t workspace_bytes, nq_stream_t stream);

/* ---------------------------------------------------------------- prefill GEMM */

/* C[M, N] = sat((A[M, K] * W) * s_out) with W[k, o] = sign(k, o) * s_in[k]:
 *   A  dtype [M, K] row-major       w_bits uint32 Marlin words [K/16, N/2]
 *   s_in, s_out: permuted as pack_binary_marlin returns them, or NULL (= ones)
 *   C  dtype [M, N]
 * K % 16 == 0, N % 64 == 0. fp32 accumulation; fp16 outputs saturate at +-65504. A must be
 * 16-byte aligned, w_bits 8-byte; a C that is not 16-byte aligned runs the slower 16x16 kernel.
 * workspace: device memory (16-byte aligned) of nq_gemm_onebit_workspace_bytes(M, K, N) bytes
 * lets a small grid split K across blocks (fp32 partial sums, added in a fixed order by a second
 * launch); NULL or a smaller one runs unsplit. Calls that share a workspace must be ordered (one
 * stream). The counterpart of the reference's Marlin workspace, which holds the locks of its
 * cross-block reduction (gemm.cpp:36-56).
 * Replaces marlin_onebit_forward (src/nanoquant/kernel/cuda/gemm.cpp:59-98,
 * registered at pybind.cpp:93-98,113). */
size_t nq_gemm_onebit_workspace_bytes(int64_t M, int64_t K, int64_t N);
int nq_gemm_onebit(int dtype, const void* A, const uint32_t* w_bits, const void* s_in, const void* s_out,
                   void* C, int64_t M, int64_t K, int64_t N, void* workspace, size_t workspace_bytes,
                   nq_stream_t stream);

/* Both stages: imm = A * (V_bits, s_g, s_l) [M, r_pad], then C = imm * (U_bits, s_h) [M, m].
 *   v_bits [n/16, r_pad/2], u_bits [r_pad/16, m/2], s_g [n], s_l [r_pad] or NULL, s_h [m] or NULL
 *   (all permuted as pack_binary_marlin_fused returns them); imm dtype [M, r_pad] is caller memory;
 *   workspace as for nq_gemm_onebit, nq_gemm_nanoquant_workspace_bytes(M, n, r_pad, m) bytes
 *   (the larger need of the two stages, which use it one after the other).
 * Replaces marlin_nanoquant_forward (src/nanoquant/kernel/cuda/gemm.cpp:112-122,
 * registered at pybind.cpp:99-104,114). */
size_t nq_gemm_nanoquant_workspace_bytes(int64_t M, int64_t n, int64_t r_pad, int64_t m);
int nq_gemm_nanoquant(int dtype, const void* A, const uint32_t* v_bits, const uint32_t* u_bits,
                      const void* s_g, const void* s_l, const void* s_h, void* imm, void* C, int64_t M,
                      int64_t n, int64_t r_pad, int64_t m, void* workspace, size_t workspace_bytes,
                      nq_stream_t stream);

/* ---------------------------------------------------------------- decode attention */

/* Bytes of workspace nq_attention_decode needs (0 on bad arguments): the partial results of
 * every (sequence, kv head, 64-position chunk). */
size_t nq_attention_decode_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads, int64_t head_dim,
                                           int64_t max_len);

/* Attention of one new token per sequence at the position *position (device int64, equal for
 * every sequence), with the rotary embedding and the KV-cache write:
 *   q, k, v   rows of qkv_stride elements (>= heads * head_dim), e.g. slices of one
 *             [batch, (heads + 2 kv_heads) * head_dim] projection output; q holds heads
 *             heads, k and v kv_heads heads, each head_dim wide
 *   k_cache, v_cache  [batch, kv_heads, max_len, head_dim], 16-byte aligned; row *position
 *             receives the rotated key and the value
 *   rope_cos, rope_sin  [max_len, head_dim] (the rotate-half convention)
 *   out       [batch, heads * head_dim] = softmax(q k^T * scaling) v over positions <= *position
 *   workspace nq_attention_decode_workspace_bytes(...) bytes, 256-byte aligned (no initial
 *             contents needed); calls sharing a workspace must not overlap.
 * Query head h uses kv head h / (heads / kv_heads). Two launches: one block per 64-position
 * chunk writes a partial result, then one block per (sequence, kv head) combines the chunks.
 * Rounding: rotary products and sum in dtype as the unfused torch path does, scores rounded to
 * dtype then scaled in fp32, softmax and the value product in fp32, output rounded to dtype
 * (the unfused path also rounds the probabilities to dtype). A position outside [0, max_len)
 * writes zeros to out and nothing to the caches. head_dim must be 128 and heads / kv_heads one
 * of 1, 2, 4, 8; NQ_ERR_UNSUPPORTED otherwise. No counterpart in the reference, whose decode
 * step runs Hugging Face's attention (kernel/test_decode.py:385-402); this is the part of a
 * decode step between the q/k/v and o projections. */
int nq_attention_decode(int dtype, const void* q, const void* k, const void* v, int64_t qkv_stride,
                        void* k_cache, void* v_cache, const void* rope_cos, const void* rope_sin,
                        const int64_t* position, void* out, int64_t batch, int64_t heads, int64_t kv_heads,
                        int64_t head_dim, int64_t max_len, float scaling, void* workspace, size_t workspace_bytes,
                        nq_stream_t stream);

/* Rotary embedding and KV-cache write of one new token per sequence, with the attention products
 * left to the caller: the first part of nq_attention_decode on its own. qkv [batch, qkv_stride]
 * holds heads query heads, kv_heads key heads and kv_heads value heads of head_dim (even) each;
 * the query heads are rotated into q_out [batch, q_stride] (q_out may be qkv), the key heads
 * rotated into k_cache[b, kvh, p, :] and the value heads copied into v_cache[b, kvh, p, :]
 * ([batch, kv_heads, max_len, head_dim] each), p = *position (device int64). rope_cos/rope_sin
 * [max_len, head_dim]. Rounded as the unfused path: T(x cos) + T(rotate_half(x) sin), summed in
 * T. A position outside [0, max_len) zeroes q_out and writes no cache row. No counterpart in the
 * reference, whose decode step runs Hugging Face's rotary embedding and cache update
 * (kernel/test_decode.py:385-402). */
int nq_rope_kv_write(int dtype, const void* qkv, int64_t qkv_stride, void* k_cache, void* v_cache,
                     const void* rope_cos, const void* rope_sin, const int64_t* position, void* q_out,
                     int64_t q_stride, int64_t batch, int64_t heads, int64_t kv_heads, int64_t head_dim,
                     int64_t max_len, nq_stream_t stream);

/* ---------------------------------------------------------------- dense GEMV */

/* y[b, j] = dtype(sum_k w[j, k] xn[b, k]) for b < batch, j < m: a dense linear of a few rows, the
 * lm_head of a decode step. w dtype [m, n] row-major, x dtype [batch, n] contiguous (16-byte aligned
 * both). xn is x, or with norm_weight (dtype [n], 16-byte aligned; NULL for none) x's RMS norm as a
 * Llama decoder rounds it: dtype(g[k] * dtype(x[k] * rsqrt(mean_k x^2 + eps))), mean and products in
 * fp32. fp32 sum, rounded once to dtype (overflow to +-inf as a torch linear does); with y_float32
 * the rounded values are stored widened to float32 (y then float [batch, ldy]), else y is dtype
 * rows of ldy >= m elements. n a multiple of 8, at most 32256; batch at most 65535. Each wave
 * streams rows of w with the next 8 KB of loads in flight during the current row's arithmetic,
 * which is what reading a large w from HBM takes. No counterpart in the reference, whose decode step runs the final norm and the lm_head as
 * torch ops (kernel/test_decode.py:387-394). */
int nq_dense_gemv(int dtype, const void* w, const void* x, const void* norm_weight, float eps, void* y,
                  int y_float32, int64_t batch, int64_t n, int64_t m, int64_t ldy, nq_stream_t stream);

/* Greedy token choice of the decode step: out[b] = the index of the largest of the n float32
 * logits in row b (x + b * ldx), the first one of equal values, the first NaN if there is one
 * (torch.argmax's order). One launch of one block per row; rows <= 2097120, n < 2^30; x 4-byte and
 * out 8-byte aligned. Replaces the argmax of the reference's decode harness
 * (src/nanoquant/kernel/test_decode.py:350-353, greedy here in place of its top-k sampling),
 * which torch runs as its own reduction launches. */
int nq_argmax_rows(const float* x, int64_t rows, int64_t n, int64_t ldx, int64_t* out, nq_stream_t stream);

/* ---------------------------------------------------------------- measurement aid */

/* Enqueue a one-thread kernel that writes the GPU's constant-rate wall clock to *dst (device
 * memory) when it runs: stream-ordered timestamps that can sit inside a HIP graph, around steps
 * of the graph itself. No counterpart in the reference (a benchmarking aid). */
int nq_timestamp(uint64_t* dst, nq_stream_t stream);
/* Ticks per second of that clock on the current device (0 on error). */
int64_t nq_wall_clock_hz(void);

/* Latency-floor probes (no counterpart in the reference; benchmarking aids). nq_probe_empty
 * enqueues a kernel of `blocks` x `threads` that does nothing: the fixed cost of one launch.
 * nq_probe_read streams `bytes` (a multiple of 16, 16-byte aligned, below 2 GiB) from `src` in
 * `blocks` (1 .. 2^20) equal contiguous runs of at most 64 KB, 16 bytes a lane, every load of a
 * lane issued before the first use: the cost of one cold read of that size with nothing else to
 * do. `sink` (device, `blocks` words) receives one word per block (the xor of the first wave's
 * data) when `store` is nonzero; otherwise it is written only when a block's xor of its data
 * equals a fixed constant, so the launch pays for no store. */
int nq_probe_empty(int64_t blocks, int64_t threads, nq_stream_t stream);
int nq_probe_read(const void* src, int64_t bytes, int64_t blocks, uint32_t* sink, int store, nq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NQ_HIP_H */
