"""CPU restatement of the NanoQuant inference path (test infrastructure only).

Every public function cites the reference file:line it restates. Integer/bit work
is numpy; the float truth is float64 numpy; the timed CPU baseline is the
reference's own torch-CPU dense path.

Pins (``tests/test_oracle.py``):

* ``pack_binary_gemv`` / ``unpack_binary_gemv``: known-answer words for both bit
  orders, the round trip on the partial-word shapes of the reference test
  ``tests/test_shaman_transfer.py:239-260``, the word-count rules of
  ``tests/test_reconstruction_efficiency.py:161-172`` and
  ``checkpoint_audit.py:33-35``, and an independent decode of the ``half2`` words
  by the sign extraction the reference GEMV kernel itself performs
  (``gemv_kernel.cu:93-96,114`` with ``cuda_utils.cuh:94-101``).
* ``pack_binary_marlin`` / ``pack_binary_marlin_fused`` / ``pack_marlin_torch``: golden
  vectors written by the reference's own packer (``tests/golden/make_marlin_vectors.py``).
* ``nanoquant_forward_f64``: closed forms (all-+1 signs, one-hot inputs) and a
  brute-force triple loop on tiny shapes.
* ``marlin_nanoquant_f64``: equal to ``nanoquant_forward_f64`` with the identity rounding;
  a closed form whose intermediate is not representable in fp16 or bf16 (it must come out
  rounded to the nearest value of the type); the clamp of the fp16 intermediate.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "HALF2_BIT", "LSB_BIT", "bit_position", "pack_binary_gemv", "unpack_binary_gemv",
    "gemv_kernel_sign", "marlin_bit_map", "marlin_perm_in", "marlin_perm_out",
    "pack_binary_marlin", "unpack_binary_marlin", "pack_binary_marlin_fused",
    "MARLIN_MIN_MAX_PAR", "nanoquant_forward_f64", "marlin_nanoquant_f64", "compute_forward_torch",
    "gemv_output_shape", "check_gemv_tuning", "GEMV_TUNING_CHOICES",
    "marlin_onebit_output_shape", "round_rank", "random_case", "pack_signs_torch", "unpack_signs_torch",
    "pack_marlin_torch",
]

MARLIN_MIN_MAX_PAR = 32  # kernel/utils.py:21, gemm.cpp:33

# Bit that holds element j (0..31) of a 32-column block.
# lsb_first: bit j (kernel/utils.py:99-100).
# half2: the powers list [15, 31, 14, 30, ..., 0, 16] (kernel/utils.py:101-104),
# i.e. bit 15 - j//2 + 16*(j%2).
LSB_BIT = np.arange(32, dtype=np.int64)
HALF2_BIT = np.array([15 - j // 2 + 16 * (j % 2) for j in range(32)], dtype=np.int64)


def bit_position(method: str) -> np.ndarray:
    """Bit index of each column of a 32-column block (kernel/utils.py:99-106)."""
    if method == "lsb_first":
        return LSB_BIT
    if method == "half2":
        return HALF2_BIT
    raise ValueError(f"Unsupported method: '{method}'. Supported methods are 'lsb_first', 'half2'.")


def pack_binary_gemv(signs: np.ndarray, method: str = "lsb_first") -> np.ndarray:
    """Pack an int8 {-1,+1} matrix [R, C] into uint32 words [R, ceil(C/32)].

    Restates ``pack_binary_gemv`` (kernel/utils.py:51-113): int8 only (TypeError,
    :79-80); columns padded to a multiple of 32 with +1 (:87-93); bit = (1 - v)//2
    so +1 -> 0 and -1 -> 1 (:96); bit placement by ``method`` (:99-106); the words
    are summed in int32 with wraparound (:109-112), which is the uint32 pattern
    returned here.
    """
    signs = np.asarray(signs)
    if signs.dtype != np.int8:
        raise TypeError("Input tensor must be int8.")
    powers = bit_position(method)
    rows, cols = signs.shape
    words = (cols + 31) // 32
    padded = np.ones((rows, words * 32), dtype=np.int64)
    padded[:, :cols] = signs
    bits = (1 - padded) // 2
    blocks = bits.reshape(rows, words, 32)
    packed = (blocks << powers[None, None, :]).sum(axis=2)
    return (packed & 0xFFFFFFFF).astype(np.uint32)


def unpack_binary_gemv(packed: np.ndarray, shape, method: str = "lsb_first") -> np.ndarray:
    """Inverse of :func:`pack_binary_gemv` (kernel/utils.py:116-183).

    ValueError for a non-2D input (:146-147) or a shape that does not match
    ``(rows, ceil(cols/32))`` (:152-154); trims the padding (:178); 0 -> +1 and
    1 -> -1 (:183).
    """
    packed = np.asarray(packed)
    if packed.ndim != 2:
        raise ValueError(f"Unsupported packed tensor format. Expected 2D tensor, got {packed.ndim} dimensions.")
    rows, cols = (int(s) for s in shape)
    words = (cols + 31) // 32
    if packed.shape != (rows, words):
        raise ValueError(
            f"Unsupported packed tensor shape. Expected ({rows}, {words}), got {tuple(packed.shape)}.")
    powers = bit_position(method)
    u = packed.astype(np.uint32).astype(np.int64)
    bits = (u[:, :, None] >> powers[None, None, :]) & 1
    flat = bits.reshape(rows, words * 32)[:, :cols]
    return (1 - 2 * flat).astype(np.int8)


def gemv_kernel_sign(word: int, j: int) -> int:
    """Sign (+1/-1) of element ``j`` of a ``half2`` word as the reference GEMV reads it.

    The reference kernel gives each of 4 lanes 8 consecutive elements of a word;
    lane q (= j // 8) shifts the word left by 4*q (``shift_base``,
    gemv_kernel.cu:114) and component p of its uint4 (elements 8q+2p, 8q+2p+1)
    takes sign bits 15 and 31 of ``word << (4q + p)`` (cuda_utils.cuh:94-101). This is
    an independent statement of the half2 bit order, written from the consumer side.
    """
    q, rem = divmod(j, 8)
    p, hi = divmod(rem, 2)
    shifted = (int(word) << (4 * q + p)) & 0xFFFFFFFF
    bit = (shifted >> (31 if hi else 15)) & 1
    return -1 if bit else 1


# ---------------------------------------------------------------------------
# Marlin layout (kernel/utils.py:186-284)
# ---------------------------------------------------------------------------

def marlin_bit_map(O: int, K: int):
    """Word row, word column and bit of element (o, k) of a [O, K] weight.

    Restates the reshape/permute/shift of ``pack_binary_marlin``
    (kernel/utils.py:192-205) as closed-form index arithmetic:
    o = 64*tile_out + 16*o16 + 8*o8 + o1 and k = 16*tile_red + 8*r8 + 2*r2 + r1;
    the word is (row=tile_red, col=32*tile_out + 4*o1 + r2) of a [K/16, O/2] array
    and the bit is 15 - (2*o8 + r8) + 16*r1 - 4*o16.
    """
    o = np.arange(O, dtype=np.int64)[:, None]
    k = np.arange(K, dtype=np.int64)[None, :]
    row = np.broadcast_to(k // 16, (O, K))
    col = (o // 64) * 32 + (o % 8) * 4 + (k % 8) // 2
    bit = 15 - 2 * ((o % 16) // 8) - ((k % 16) // 8) + 16 * (k % 2) - 4 * ((o % 64) // 16)
    return row, np.broadcast_to(col, (O, K)), np.broadcast_to(bit, (O, K))


def marlin_perm_in(K: int) -> np.ndarray:
    """Position of natural input-scale index i in the packed scale vector.

    kernel/utils.py:206-207: a [K/16, 2, 4, 2] view permuted (0, 2, 1, 3), so natural
    16c + 8a + 2b + d lands at 16c + 4b + 2a + d.
    """
    i = np.arange(K, dtype=np.int64)
    c, a, b, d = i // 16, (i % 16) // 8, (i % 8) // 2, i % 2
    return 16 * c + 4 * b + 2 * a + d


def marlin_perm_out(O: int) -> np.ndarray:
    """Position of natural output-scale index i in the packed scale vector.

    kernel/utils.py:208-209: a [O/32, 4, 4, 2] view permuted (0, 2, 1, 3), so natural
    32c + 8a + 2b + d lands at 32c + 8b + 2a + d.
    """
    i = np.arange(O, dtype=np.int64)
    c, a, b, d = i // 32, (i % 32) // 8, (i % 8) // 2, i % 2
    return 32 * c + 8 * b + 2 * a + d


def pack_binary_marlin(weight: np.ndarray, scale_in: np.ndarray, scale_out: np.ndarray):
    """Pack a {-1,+1} weight [O, K] for the binary GEMM (kernel/utils.py:186-214).

    Returns (words uint32 [K/16, O/2], scale_in permuted, scale_out permuted,
    workspace_size = (O // 128) * 32). Requires O % 64 == 0 and K % 16 == 0 (the
    reference's reshape fails otherwise); the scale vectors need len % 16 == 0 and
    len % 32 == 0 respectively (:206-209).
    """
    weight = np.asarray(weight)
    O, K = weight.shape
    if O % 64 or K % 16:
        raise ValueError(f"pack_binary_marlin needs O % 64 == 0 and K % 16 == 0, got {weight.shape}")
    scale_in = np.asarray(scale_in).reshape(-1)
    scale_out = np.asarray(scale_out).reshape(-1)
    if scale_in.size % 16 or scale_out.size % 32:
        raise ValueError("scale_in length must be a multiple of 16 and scale_out a multiple of 32")
    row, col, bit = marlin_bit_map(O, K)
    neg = (1 - weight.astype(np.int64)) // 2
    words = np.zeros((K // 16, O // 2), dtype=np.int64)
    np.add.at(words, (row.ravel(), col.ravel()), (neg << bit).ravel())
    words = (words & 0xFFFFFFFF).astype(np.uint32)
    s_in = np.empty_like(scale_in)
    s_in[marlin_perm_in(scale_in.size)] = scale_in
    s_out = np.empty_like(scale_out)
    s_out[marlin_perm_out(scale_out.size)] = scale_out
    workspace_size = s_out.size // 128 * MARLIN_MIN_MAX_PAR
    return words, s_in, s_out, workspace_size


def unpack_binary_marlin(words: np.ndarray, O: int, K: int) -> np.ndarray:
    """Signs [O, K] held by Marlin words [K/16, O/2] (inverse of the bit map above)."""
    row, col, bit = marlin_bit_map(O, K)
    u = np.asarray(words).astype(np.uint32).astype(np.int64)
    b = (u[row, col] >> bit) & 1
    return (1 - 2 * b).astype(np.int8)


def pack_binary_marlin_fused(V_sign: np.ndarray, U_sign: np.ndarray, scale_g, scale_l, scale_h):
    """Pack both factors for ``marlin_nanoquant_forward`` (kernel/utils.py:217-284).

    V_sign [N, R] and U_sign [R, M] ({-1,+1}); R is padded up to a multiple of 256
    with +1 signs and zero ``scale_l`` (:262-271); the first stage packs V_sign.T
    with (scale_g, scale_l) and the second U_sign.T with (scale_l, scale_h), whose
    returned input scale is discarded (:274-277). Returns
    (V_bits, U_bits, scale_g', scale_l', scale_h', workspace) with an int32 zero
    workspace of max(ws_v, ws_u) entries (:280-284). A missing ``scale_l`` makes
    the reference fail; here that is a ValueError.
    """
    if scale_l is None:
        raise ValueError("pack_binary_marlin_fused needs scale_l (use ones when the layer has none)")
    V_sign = np.asarray(V_sign)
    U_sign = np.asarray(U_sign)
    scale_l = np.asarray(scale_l).reshape(-1)
    N = np.asarray(scale_g).reshape(-1).shape[0]
    R = scale_l.shape[0]
    M = np.asarray(scale_h).reshape(-1).shape[0]
    if R % 32:
        R = (R // 32 + 1) * 32
    rank_marlin = (R + 255) // 256 * 256
    if rank_marlin > R:
        pad = rank_marlin - R
        V_sign = np.concatenate([V_sign, np.ones((N, pad), dtype=np.int8)], axis=1)
        U_sign = np.concatenate([U_sign, np.ones((pad, M), dtype=np.int8)], axis=0)
        scale_l = np.concatenate([scale_l, np.zeros(pad, dtype=scale_l.dtype)])
    V_bits, s_g, s_l, ws_v = pack_binary_marlin(V_sign.T, scale_g, scale_l)
    U_bits, _, s_h, ws_u = pack_binary_marlin(U_sign.T, scale_l, scale_h)
    workspace = np.zeros(max(ws_v, ws_u), dtype=np.int32)
    return V_bits, U_bits, s_g, s_l, s_h, workspace


# ---------------------------------------------------------------------------
# Dense forward (modules/linear.py:282-291)
# ---------------------------------------------------------------------------

def nanoquant_forward_f64(x, s_in, V, s_mid, U, s_out):
    """y = s_out * (U @ ((V @ (s_in * x)) * s_mid)) in float64, row-batched.

    x [B, n], s_in [n], V [r, n] (+-1), s_mid [r] or None, U [m, r] (+-1),
    s_out [m]. Restates ``_compute_forward`` (linear.py:282-291): F.linear(x*s_pre, V),
    times scale_mid, F.linear(., U), times scale_post.
    """
    x = np.asarray(x, dtype=np.float64)
    h = (x * np.asarray(s_in, dtype=np.float64)) @ np.asarray(V, dtype=np.float64).T
    if s_mid is not None:
        h = h * np.asarray(s_mid, dtype=np.float64)
    y = h @ np.asarray(U, dtype=np.float64).T
    return y * np.asarray(s_out, dtype=np.float64)


def marlin_nanoquant_f64(x, s_in, V, s_mid, U, s_out, round_imm, sat_imm=None):
    """The prefill GEMM's algorithm in float64 with its intermediate rounding point.

    ``marlin_nanoquant_cuda`` (gemm.cpp:112-122) is two ``marlin_onebit`` products whose
    intermediate ``imm`` is a tensor of the activation dtype: h = (s_in * x) @ V^T * s_mid is
    clamped to +-``sat_imm`` (gemm_kernel.cu:124-126, fp16 only) and rounded by ``round_imm``
    (a float64 -> float64 function that rounds to that dtype), then y = s_out * (h @ U^T).
    With ``round_imm`` the identity and no clamp this is ``nanoquant_forward_f64``.
    """
    x = np.asarray(x, dtype=np.float64)
    h = (x * np.asarray(s_in, dtype=np.float64)) @ np.asarray(V, dtype=np.float64).T
    if s_mid is not None:
        h = h * np.asarray(s_mid, dtype=np.float64)
    if sat_imm is not None:
        h = np.clip(h, -sat_imm, sat_imm)
    h = round_imm(h)
    y = h @ np.asarray(U, dtype=np.float64).T
    return y * np.asarray(s_out, dtype=np.float64)


def compute_forward_torch(x, V, U, scale_pre, scale_mid, scale_post):
    """The reference's dense dequantize-and-matmul path, in torch on the CPU.

    Same four steps as linear.py:282-291 in the tensors' dtype; the inputs are the
    dense +-1 factors the reference loader materialises (load_utils.py:392). This is
    the CPU baseline that is timed, not a parity truth.
    """
    import torch.nn.functional as F

    y = F.linear(x * scale_pre, V)
    if scale_mid is not None:
        y = y * scale_mid
    y = F.linear(y, U)
    return y * scale_post


def pack_signs_torch(signs, method: str = "lsb_first"):
    """The packer of kernel/utils.py:51-113 as eager torch ops on the CPU (the timed CPU baseline
    of packing; the reference decorates it with torch.compile, whose compile time the baseline
    leaves out). Pad to 32 columns with +1 (:87-93), bits (1 - v) // 2 (:96), int32 weights 2^bit
    in ``method`` order (:99-109), int32 sum with wraparound (:112). Checked against
    :func:`pack_binary_gemv` in tests/test_oracle.py."""
    import torch

    rows, cols = signs.shape
    words = (cols + 31) // 32
    if words * 32 != cols:
        signs = torch.cat([signs, torch.ones(rows, words * 32 - cols, dtype=signs.dtype)], dim=1)
    bits = ((1 - signs) // 2).int().view(rows, words, 32)
    weights = torch.from_numpy((np.uint64(1) << bit_position(method).astype(np.uint64)).astype(np.uint32)
                               .view(np.int32).copy())
    return (bits * weights).sum(dim=2, dtype=torch.int32).contiguous()


def pack_marlin_torch(weight):
    """The Marlin packer of kernel/utils.py:186-205 as eager torch ops on the CPU (the timed CPU
    baseline of Marlin packing). The [O, K] weight is viewed as (O/64, 4, 2, 8, K/16, 2, 4, 2) =
    (tile_out, o16, o8, o1, tile_red, r8, r2, r1) and permuted to (tile_red, tile_out, o1, r2, o16,
    r1, o8, r8), so that each run of 32 values is one word's elements (:192-196); element
    (o16, r1, o8, r8) takes bit 15 - (2 o8 + r8) + 16 r1 - 4 o16 (:198-202); bits (1 - v) // 2
    weighted by 2^bit are summed in int32 (:204) into words [K/16, O/2] (:205). Checked against the
    reference-written vectors in tests/test_oracle.py."""
    import torch

    O_, K_ = weight.shape
    v = weight.reshape(O_ // 64, 4, 2, 8, K_ // 16, 2, 4, 2).permute(4, 0, 3, 6, 1, 7, 2, 5).reshape(-1, 32).int()
    o16, r1, o8, r8 = np.meshgrid(np.arange(4), np.arange(2), np.arange(2), np.arange(2), indexing="ij")
    bit = (15 - (2 * o8 + r8) + 16 * r1 - 4 * o16).reshape(-1).astype(np.uint64)
    weights = torch.from_numpy((np.uint64(1) << bit).astype(np.uint32).view(np.int32).copy())
    return (((1 - v) // 2) * weights).sum(dim=1, dtype=torch.int32).reshape(K_ // 16, O_ // 2).contiguous()


def unpack_signs_torch(packed, shape, method: str = "lsb_first"):
    """The unpacker of kernel/utils.py:116-183 as eager torch ops on the CPU (timed CPU baseline):
    every bit extracted with a shift by its position and ``& 1`` (:172), trimmed to the original
    columns (:178), 0 -> +1 and 1 -> -1 (:183). Checked against :func:`unpack_binary_gemv`."""
    import torch

    rows, cols = (int(v) for v in shape)
    words = (cols + 31) // 32
    shifts = torch.from_numpy(bit_position(method).astype(np.int32))
    bits = (packed.unsqueeze(2) >> shifts) & 1
    flat = bits.view(rows, words * 32).to(torch.int8)[:, :cols]
    return (1 - 2 * flat).to(torch.int8)


# ---------------------------------------------------------------------------
# Op-level rules
# ---------------------------------------------------------------------------

# parameter_sweep instances of nanoquant_dyn_forward (gemv_kernel.cu:351-354).
GEMV_TUNING_CHOICES = {
    "n_th": (64, 128, 256),
    "n_rpw": (1, 2, 4, 8),
    "n_acc": (1, 2),
    "n_pipe": (1, 2, 4, 8, 16),
}


def check_gemv_tuning(th1, th2, rpw1, rpw2, acc1, acc2, pipe1, pipe2):
    """First tuning-int error the reference raises, as (name, message), or None.

    The reference validates stage 1's four ints in nesting order, launches stage 1,
    then validates stage 2's (gemv_kernel.cu:405-425); the message format is
    meta_utils.h:36.
    """
    order = [("n_th1", th1, "n_th"), ("n_rpw1", rpw1, "n_rpw"), ("n_acc1", acc1, "n_acc"),
             ("n_pipe1", pipe1, "n_pipe"), ("n_th2", th2, "n_th"), ("n_rpw2", rpw2, "n_rpw"),
             ("n_acc2", acc2, "n_acc"), ("n_pipe2", pipe2, "n_pipe")]
    for name, value, key in order:
        choices = GEMV_TUNING_CHOICES[key]
        if value not in choices:
            return name, f"{name} should be one of [{', '.join(str(c) for c in choices)}], but {value} was given"
    return None


def gemv_output_shape(x_shape, m: int):
    """Output shape of nanoquant_dyn_forward: x's shape with the last dim -> m.

    The Meta impl (pybind.cpp:26-31); the device impl returns [B, m] for 2-D x and
    [m] for 1-D x (gemv_kernel.cu:340,345-346,427).
    """
    out = list(x_shape)
    out[-1] = m
    return tuple(out)


def marlin_onebit_output_shape(a_shape, b_shape):
    """[A.size(0), 2 * B.size(1)] (gemm.cpp:44-55)."""
    return (a_shape[0], 2 * b_shape[1])


# ---------------------------------------------------------------------------
# Synthetic inputs
# ---------------------------------------------------------------------------

def round_rank(bpw: float, m: int, n: int) -> int:
    """Rank rule of the benchmark configs: round32(bpw * m * n / (m + n))."""
    return int(round(bpw * m * n / (m + n) / 32.0)) * 32


def random_case(seed: int, m: int, n: int, r: int, B: int, with_mid: bool = False):
    """Seeded inputs in a fixed draw order: U signs [m, r], V signs [r, n], s_in [n],
    s_out [m], x [B, n] (then s_mid [r] when asked). Signs are Bernoulli(0.5);
    scales are fp16 |N(1, 0.2)|; x is fp16 N(0, 1)."""
    rng = np.random.default_rng(seed)
    U = np.where(rng.random((m, r)) < 0.5, -1, 1).astype(np.int8)
    V = np.where(rng.random((r, n)) < 0.5, -1, 1).astype(np.int8)
    s_in = np.abs(rng.normal(1.0, 0.2, n)).astype(np.float16)
    s_out = np.abs(rng.normal(1.0, 0.2, m)).astype(np.float16)
    x = rng.normal(0.0, 1.0, (B, n)).astype(np.float16)
    s_mid = np.abs(rng.normal(1.0, 0.2, r)).astype(np.float16) if with_mid else None
    return dict(U=U, V=V, s_in=s_in, s_out=s_out, x=x, s_mid=s_mid)
