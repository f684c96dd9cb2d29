"""Packers and op lookup with the signatures of the reference's ``kernel/utils.py``.

Each function keeps the reference's name, arguments, return values, layouts and
errors (``src/nanoquant/kernel/utils.py:33-284,503-507``). Like the reference's
device-agnostic torch packers, each packs a tensor where it lives: CUDA tensors with
the gfx950 HIP library, CPU tensors on the host (``_host.py``, the same words bit for
bit), so a packed state dict can be written and read on a machine without a GPU. A
CUDA tensor never takes the host path, and a CPU tensor never the GPU one.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .. import _lib
from . import _host

MARLIN_MIN_MAX_PAR = 32

_METHODS = {"lsb_first": _lib.NQ_PACK_LSB_FIRST, "half2": _lib.NQ_PACK_HALF2}


def get_kernel_function(namespace: str, dtype: torch.dtype, kernel_type: str):
    """Resolve ``torch.ops.binary_kernels.<namespace>[_dyn]_forward`` (kernel/utils.py:33-48)."""
    try:
        from .. import binary_kernels
        binary_kernels.ensure_loaded()
    except Exception as exc:
        raise ImportError("Could not import `binary_kernels`. Did you build the extension?\n"
                          f"Original error: {exc}") from exc

    mid = "_dyn" if kernel_type != "fixed" else ""
    op_name = f"{namespace}{mid}_forward"

    try:
        return getattr(torch.ops.binary_kernels, op_name)
    except AttributeError as exc:
        have = dir(torch.ops.binary_kernels) if hasattr(torch.ops, "binary_kernels") else []
        raise AttributeError(f"Dispatcher op `{namespace}::{op_name}` not found. "
                             f"Available in torch.ops.binary_kernels: {have}") from exc


def _method_code(method: str) -> int:
    try:
        return _METHODS[method]
    except KeyError:
        raise ValueError(f"Unsupported method: '{method}'. Supported methods are 'lsb_first', 'half2'.") from None


def _on_host(*tensors: torch.Tensor) -> bool:
    """True for CPU tensors (packed on the host); CUDA tensors go to the HIP kernels; anything
    else, or a mix, is refused."""
    kinds = {t.device.type for t in tensors if t is not None}
    if kinds == {"cpu"}:
        return True
    if kinds == {"cuda"}:
        return False
    raise RuntimeError(f"nanoquant_amd packs CPU or CUDA tensors, all on one device; got {sorted(kinds)}")


def pack_binary_gemv(tensor: torch.Tensor, method: str = "lsb_first") -> torch.Tensor:
    """Pack a {-1,+1} int8 matrix [R, C] into int32 words [R, ceil(C/32)] (kernel/utils.py:51-113).

    TypeError for a non-int8 input; ValueError for an unknown ``method``. Columns are
    padded with +1 (bit 0); a set bit means -1. ``method`` 'lsb_first' puts column j of a
    32-column block at bit j, 'half2' at bit 15 - j//2 + 16*(j%2).
    """
    if tensor.dtype != torch.int8:
        raise TypeError("Input tensor must be int8.")
    n_rows, n_cols = tensor.shape
    code = _method_code(method)
    words = (n_cols + 31) // 32
    if _on_host(tensor):
        return _host.pack_signs(tensor, code)
    src = tensor.contiguous()
    out = torch.empty((n_rows, words), dtype=torch.int32, device=src.device)
    if out.numel():
        lib = _lib.load()
        with torch.cuda.device(src.device):
            status = lib.nq_pack_signs(src.data_ptr(), out.data_ptr(), n_rows, n_cols, code,
                                       _lib.stream_of(src.device))
        _lib.check(status, "pack_binary_gemv")
    return out


def unpack_binary_gemv(packed_tensor: torch.Tensor, original_shape: Tuple[int, int],
                       method: str = "lsb_first") -> torch.Tensor:
    """Inverse of :func:`pack_binary_gemv` (kernel/utils.py:116-183): int8 {-1,+1} of
    ``original_shape``. ValueError for a non-2D input, a shape that is not
    (rows, ceil(cols/32)), or an unknown ``method``."""
    if packed_tensor.dim() != 2:
        raise ValueError(f"Unsupported packed tensor format. Expected 2D tensor, got {packed_tensor.dim()} dimensions.")
    n_rows, n_cols = (int(s) for s in original_shape)
    words_per_row = (n_cols + 31) // 32
    if tuple(packed_tensor.shape) != (n_rows, words_per_row):
        raise ValueError(
            f"Unsupported packed tensor shape. Expected ({n_rows}, {words_per_row}), got {packed_tensor.shape}.")
    code = _method_code(method)
    if packed_tensor.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"packed words must be int32, got {packed_tensor.dtype}")
    if _on_host(packed_tensor):
        return _host.unpack_signs(packed_tensor, n_rows, n_cols, code)
    src = packed_tensor.contiguous()
    out = torch.empty((n_rows, n_cols), dtype=torch.int8, device=src.device)
    if out.numel():
        lib = _lib.load()
        with torch.cuda.device(src.device):
            status = lib.nq_unpack_signs(src.data_ptr(), out.data_ptr(), n_rows, n_cols, code,
                                         _lib.stream_of(src.device))
        _lib.check(status, "unpack_binary_gemv")
    return out


def repack_binary_gemv(packed_tensor: torch.Tensor, original_shape: Tuple[int, int], src_method: str = "lsb_first",
                       dst_method: str = "half2") -> torch.Tensor:
    """Re-order packed words between bit orders without expanding them.

    Equivalent to ``pack_binary_gemv(unpack_binary_gemv(p, shape, src), dst)``, the
    route a checkpoint's lsb_first words take to the GEMV's half2 words
    (load_utils.py:392 then linear.py:205-206), in one pass over the words.
    """
    if packed_tensor.dim() != 2:
        raise ValueError(f"Unsupported packed tensor format. Expected 2D tensor, got {packed_tensor.dim()} dimensions.")
    n_rows, n_cols = (int(s) for s in original_shape)
    if tuple(packed_tensor.shape) != (n_rows, (n_cols + 31) // 32):
        raise ValueError(f"Unsupported packed tensor shape. Expected ({n_rows}, {(n_cols + 31) // 32}), "
                         f"got {packed_tensor.shape}.")
    if packed_tensor.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"packed words must be int32, got {packed_tensor.dtype}")
    s_code, d_code = _method_code(src_method), _method_code(dst_method)
    if _on_host(packed_tensor):
        return _host.repack_signs(packed_tensor, n_rows, n_cols, s_code, d_code)
    src = packed_tensor.contiguous()
    out = torch.empty(src.shape, dtype=torch.int32, device=src.device)
    if out.numel():
        lib = _lib.load()
        with torch.cuda.device(src.device):
            status = lib.nq_repack_signs(src.data_ptr(), out.data_ptr(), n_rows, n_cols, s_code, d_code,
                                         _lib.stream_of(src.device))
        _lib.check(status, "repack_binary_gemv")
    return out


def _permute_scales(scale_in, scale_out):
    s_in = scale_in.reshape(-1).contiguous()
    s_out = scale_out.reshape(-1).contiguous()
    for name, s in (("scale_in", s_in), ("scale_out", s_out)):
        if s.element_size() != 2:
            raise TypeError(f"{name} must be a 16-bit float tensor, got {s.dtype}")
    if s_in.numel() % 16:
        raise RuntimeError(f"shape '[{s_in.numel() // 16}, 2, 4, 2]' is invalid for input of size {s_in.numel()}")
    if s_out.numel() % 32:
        raise RuntimeError(f"shape '[{s_out.numel() // 32}, 4, 4, 2]' is invalid for input of size {s_out.numel()}")
    if _on_host(s_in, s_out):
        return _host.permute_marlin_scales(s_in, s_out)
    p_in = torch.empty_like(s_in)
    p_out = torch.empty_like(s_out)
    lib = _lib.load()
    with torch.cuda.device(s_in.device):
        status = lib.nq_permute_marlin_scales(s_in.data_ptr(), p_in.data_ptr(), s_in.numel(), s_out.data_ptr(),
                                              p_out.data_ptr(), s_out.numel(), _lib.stream_of(s_in.device))
    _lib.check(status, "pack_binary_marlin scales")
    return p_in, p_out


def pack_binary_marlin(weight: torch.Tensor, scale_in: torch.Tensor,
                       scale_out: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]:
    """Pack a {-1,+1} weight [O, K] for the binary GEMM (kernel/utils.py:186-214).

    Returns (int32 words [K/16, O/2], permuted scale_in, permuted scale_out,
    workspace_size). O must be a multiple of 64 and K of 16 (RuntimeError otherwise,
    as the reference's reshape raises).
    """
    O, K = weight.shape
    if O % 64 or K % 16:
        raise RuntimeError(f"shape '[{O // 64}, 4, 2, 8, {K // 16}, 2, 4, 2]' is invalid for input of size {O * K}")
    w = (weight if weight.dtype == torch.int8 else weight.to(torch.int8)).contiguous()
    if _on_host(w, scale_in, scale_out):
        words = _host.pack_marlin(w)
    else:
        words = torch.empty((K // 16, O // 2), dtype=torch.int32, device=w.device)
        if words.numel():
            lib = _lib.load()
            with torch.cuda.device(w.device):
                status = lib.nq_pack_marlin(w.data_ptr(), words.data_ptr(), O, K, _lib.stream_of(w.device))
            _lib.check(status, "pack_binary_marlin")
    s_in, s_out = _permute_scales(scale_in, scale_out)
    workspace_size = s_out.numel() // 128 * MARLIN_MIN_MAX_PAR
    return words, s_in, s_out, workspace_size


def pack_binary_marlin_fused(V_sign: torch.Tensor, U_sign: torch.Tensor, scale_g: torch.Tensor,
                             scale_l: torch.Tensor, scale_h: torch.Tensor):
    """Pack both binary factors for ``marlin_nanoquant_forward`` (kernel/utils.py:217-284).

    V_sign [N, R] and U_sign [R, M] in {-1,+1}; R is padded to a multiple of 256 with +1
    signs and zero ``scale_l``. Returns (V_bits, U_bits, scale_g', scale_l', scale_h',
    workspace) with an int32 zero workspace. ``scale_l`` is required (the reference
    fails without it; NanoQuantLinear passes ones when the layer has no mid scale).
    """
    if scale_l is None:
        raise ValueError("pack_binary_marlin_fused needs scale_l (use ones when the layer has none)")
    dev = V_sign.device
    N = scale_g.shape[0]
    R = scale_l.shape[0]
    M = scale_h.shape[0]
    p = 32
    if R % p != 0:
        R = ((R // p) + 1) * p
    rank_p = 256
    rank_marlin = (R + rank_p - 1) // rank_p * rank_p
    if rank_marlin > R:
        pad_amount = rank_marlin - R
        V_sign = torch.cat([V_sign, torch.ones(N, pad_amount, device=dev, dtype=torch.int8)], dim=1)
        U_sign = torch.cat([U_sign, torch.ones(pad_amount, M, device=dev, dtype=torch.int8)], dim=0)
        scale_l = torch.cat([scale_l, torch.zeros(pad_amount, device=scale_l.device, dtype=scale_l.dtype)], dim=0)

    V_bits, scale_g_marlin, scale_l_marlin, workspace_size_v = pack_binary_marlin(V_sign.T, scale_g, scale_l)
    U_bits, _, scale_h_marlin, workspace_size_u = pack_binary_marlin(U_sign.T, scale_l, scale_h)
    workspace_size = max(workspace_size_v, workspace_size_u)
    workspace = torch.zeros(workspace_size, device=dev, dtype=torch.int32)
    return V_bits.contiguous(), U_bits.contiguous(), scale_g_marlin, scale_l_marlin, scale_h_marlin, workspace


def repack_binary_marlin(packed_tensor: torch.Tensor, original_shape: Tuple[int, int],
                         padded_shape: Tuple[int, int] | None = None, src_method: str = "lsb_first") -> torch.Tensor:
    """Marlin words of a {-1,+1} [O, K] matrix given as its packed sign words.

    ``packed_tensor`` holds ``original_shape`` = (O, K) in ``src_method`` order, (O, ceil(K/32))
    words, as a checkpoint stores V [r, n] and U [m, r] (linear.py:359-376). The matrix is padded
    with +1 to ``padded_shape`` (default: unpadded; O_pad % 64 == 0, K_pad % 16 == 0) and returned
    as int32 words [K_pad/16, O_pad/2], the words ``pack_binary_marlin`` makes from the dense
    padded matrix, in one pass on the GPU.
    """
    if packed_tensor.dim() != 2:
        raise ValueError(f"Unsupported packed tensor format. Expected 2D tensor, got {packed_tensor.dim()} dimensions.")
    O, K = (int(s) for s in original_shape)
    O_pad, K_pad = (O, K) if padded_shape is None else (int(s) for s in padded_shape)
    if tuple(packed_tensor.shape) != (O, (K + 31) // 32):
        raise ValueError(f"Unsupported packed tensor shape. Expected ({O}, {(K + 31) // 32}), "
                         f"got {packed_tensor.shape}.")
    if packed_tensor.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"packed words must be int32, got {packed_tensor.dtype}")
    if O_pad < O or K_pad < K or O_pad % 64 or K_pad % 16:
        raise RuntimeError(f"padded shape ({O_pad}, {K_pad}) must cover ({O}, {K}) with O % 64 == 0 and K % 16 == 0")
    code = _method_code(src_method)
    if _on_host(packed_tensor):
        return _host.repack_marlin(packed_tensor, O, K, O_pad, K_pad, code)
    src = packed_tensor.contiguous()
    words = torch.empty((K_pad // 16, O_pad // 2), dtype=torch.int32, device=src.device)
    if words.numel():
        lib = _lib.load()
        with torch.cuda.device(src.device):
            status = lib.nq_repack_marlin(src.data_ptr(), O, K, code, words.data_ptr(), O_pad, K_pad,
                                          _lib.stream_of(src.device))
        _lib.check(status, "repack_binary_marlin")
    return words


def marlin_rank(rank: int) -> int:
    """The rank the fused Marlin packer pads to: a multiple of 32, then of 256 (kernel/utils.py:251-271)."""
    rank = (rank + 31) // 32 * 32
    return (rank + 255) // 256 * 256


def pack_binary_marlin_fused_from_packed(V_packed: torch.Tensor, V_shape: Tuple[int, int], U_packed: torch.Tensor,
                                         U_shape: Tuple[int, int], scale_g: torch.Tensor, scale_l: torch.Tensor,
                                         scale_h: torch.Tensor, src_method: str = "lsb_first"):
    """``pack_binary_marlin_fused(V.T, U.T, ...)`` from a checkpoint's sign words of V [r, n] and U [m, r].

    Returns the same (V_bits, U_bits, scale_g', scale_l', scale_h', workspace) as the fused
    packer given the dense factors (kernel/utils.py:217-284, as ``_prepare_kernel`` calls it,
    linear.py:226-232), without expanding either factor: the words are repacked on the GPU
    with the rank padding (+1 signs, zero ``scale_l``) folded in.
    """
    if scale_l is None:
        raise ValueError("pack_binary_marlin_fused needs scale_l (use ones when the layer has none)")
    r, n = (int(s) for s in V_shape)
    m, r_u = (int(s) for s in U_shape)
    if r_u != r or scale_l.shape[0] != r or scale_g.shape[0] != n or scale_h.shape[0] != m:
        raise ValueError(f"factor shapes disagree: V {tuple(V_shape)}, U {tuple(U_shape)}, scales "
                         f"{scale_g.shape[0]}, {scale_l.shape[0]}, {scale_h.shape[0]}")
    r_pad = marlin_rank(r)
    V_bits = repack_binary_marlin(V_packed, (r, n), (r_pad, n), src_method)
    U_bits = repack_binary_marlin(U_packed, (m, r), (m, r_pad), src_method)
    if r_pad > r:
        scale_l = torch.cat([scale_l, torch.zeros(r_pad - r, device=scale_l.device, dtype=scale_l.dtype)], dim=0)
    scale_g_marlin, scale_l_marlin = _permute_scales(scale_g, scale_l)
    _, scale_h_marlin = _permute_scales(scale_l, scale_h)
    workspace_size = max(scale_l_marlin.numel(), scale_h_marlin.numel()) // 128 * MARLIN_MIN_MAX_PAR
    workspace = torch.zeros(workspace_size, device=V_bits.device, dtype=torch.int32)
    return V_bits, U_bits, scale_g_marlin, scale_l_marlin, scale_h_marlin, workspace


# Aliases of the reference (kernel/utils.py:503-506)
binary_packer = pack_binary_gemv
binary_unpacker = unpack_binary_gemv
marlin_onebit_packer = pack_binary_marlin
marlin_nanoquant_packer = pack_binary_marlin_fused
