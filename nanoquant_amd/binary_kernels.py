"""The ``torch.ops.binary_kernels`` operators, backed by the gfx950 HIP library.

Importing this module registers, under the namespace ``binary_kernels``, the three
schemas of the reference extension (``src/nanoquant/kernel/pybind.cpp:85-104``)
with a CUDA (= HIP on ROCm) implementation that calls the C ABI and a fake
(Meta) implementation that only computes shapes (``pybind.cpp:11-48,117-124``,
``gemm.cpp:100-110,124-134``). There is no CPU implementation: a CPU tensor fails
in the dispatcher as it does with the reference.

Argument checks and their messages follow the reference: RuntimeError for
device/contiguity/dtype/size problems (``cuda_utils.cuh:13-50``,
``gemv_kernel.cu:316-338``, ``gemm.cpp:44-52,90``) and ValueError for tuning ints
outside the instantiated sets (``gemv_kernel.cu:351-354``, ``meta_utils.h:36``).
The tuning ints are validated and otherwise ignored: the HIP GEMV picks its own
launch shape. Shapes the reference kernels mishandle silently (sizes that are not
multiples of their tiles, >2-D inputs) are computed correctly here, and the
packed operand shapes are checked, which the reference does not do.
"""
from __future__ import annotations

import torch

from . import _lib

_NS = "binary_kernels"
MARLIN_MIN_MAX_PAR = 32

GEMV_SCHEMA = (
    "nanoquant_dyn_forward("
    "Tensor x, Tensor scale_g, Tensor Ubits, Tensor? scale_l, Tensor Vbits, Tensor scale_h, "
    "int num_thread_stage1=128, int num_thread_stage2=128, int num_row_per_warp_stage1=2, "
    "int num_row_per_warp_stage2=2, int num_acc_stage1=4, int num_acc_stage2=4, "
    "int num_pipeline_stage1=2, int num_pipeline_stage2=2) -> Tensor")
ONEBIT_SCHEMA = (
    "marlin_onebit_forward("
    "Tensor x, Tensor weight, Tensor? scale_g, Tensor? scale_h, Tensor(a!) workspace) -> Tensor")
NANOQUANT_SCHEMA = (
    "marlin_nanoquant_forward("
    "Tensor x, Tensor weight_u, Tensor weight_v, Tensor? scale_g, Tensor? scale_l, Tensor? scale_h, "
    "Tensor(a!) workspace) -> Tensor")

TUNING_CHOICES = {
    "n_th": (64, 128, 256),
    "n_rpw": (1, 2, 4, 8),
    "n_acc": (1, 2),
    "n_pipe": (1, 2, 4, 8, 16),
}

_DTYPE_WORD = {torch.float16: "float16", torch.bfloat16: "bfloat16"}


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_cuda_cont(name: str, t: torch.Tensor, dtype=None, dtype_word=None) -> None:
    """CHECK_CUDA_CONT_* of cuda_utils.cuh:13-50 (same messages)."""
    _check(t.is_cuda, f"{name} must be a CUDA tensor")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    if dtype is torch.int32:
        _check(t.dtype == torch.int32, f"{name} tensor dtype must be int32")
    elif dtype is not None:
        _check(t.dtype == dtype, f"{name} must be {dtype_word} tensor")


def _check_tuning(th1, th2, rpw1, rpw2, acc1, acc2, pipe1, pipe2) -> None:
    """parameter_sweep validation in the reference's order (gemv_kernel.cu:405-425)."""
    order = [("n_th1", th1, "n_th"), ("n_rpw1", rpw1, "n_rpw"), ("n_acc1", acc1, "n_acc"),
             ("n_pipe1", pipe1, "n_pipe"), ("n_th2", th2, "n_th"), ("n_rpw2", rpw2, "n_rpw"),
             ("n_acc2", acc2, "n_acc"), ("n_pipe2", pipe2, "n_pipe")]
    for name, value, key in order:
        choices = TUNING_CHOICES[key]
        if value not in choices:
            raise ValueError(f"{name} should be one of [{', '.join(str(c) for c in choices)}], but {value} was given")


# --------------------------------------------------------------------------- GEMV workspace
# The GEMV workspace is a 256-byte reserved header followed by the intermediate h as two
# bf16 arrays (hi, then lo), each [batch][zpitch]; stage 1 rewrites every element of both
# on each call, so the buffer needs no initial contents. It is taken from torch's caching
# allocator per call, as the reference allocates its intermediate per call
# (gemv_kernel.cu:345-346): the allocator orders reuse by stream, and under graph capture
# the block comes from the graph's private pool and stays reserved for its replays, so no
# captured graph can be left pointing at memory that was handed to another tensor.


def gemv_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


# --------------------------------------------------------------------------- nanoquant_dyn_forward

def _gemv_args(x, scale_g, Ubits, scale_l, Vbits, scale_h):
    st = x.dtype
    _check(st in (torch.float16, torch.bfloat16), "Support only Half or BFloat16")
    word = _DTYPE_WORD[st]
    _check_cuda_cont("x", x, st, word)
    _check_cuda_cont("scale_g", scale_g, st, word)
    _check_cuda_cont("scale_h", scale_h, st, word)
    _check_cuda_cont("Ubits", Ubits, torch.int32)
    _check_cuda_cont("Vbits", Vbits, torch.int32)
    if scale_l is not None:
        _check_cuda_cont("(*scale_l)", scale_l, st, word)
        _check(scale_l.size(0) == Ubits.size(0), "scale_l size mismatch")
    _check(x.dim() >= 1, "x must have at least one dimension")
    n = x.size(-1)
    r = Ubits.size(0)
    m = scale_h.size(0)
    # checks the reference leaves to out-of-bounds reads
    _check(Ubits.dim() == 2 and Ubits.size(1) == (n + 31) // 32,
           f"Ubits must be [r, ceil(n/32)] = [{r}, {(n + 31) // 32}], got {list(Ubits.shape)}")
    _check(Vbits.dim() == 2 and Vbits.size(0) == m and Vbits.size(1) == (r + 31) // 32,
           f"Vbits must be [m, ceil(r/32)] = [{m}, {(r + 31) // 32}], got {list(Vbits.shape)}")
    _check(scale_g.numel() == n, f"scale_g must have {n} elements, got {scale_g.numel()}")
    _check(scale_h.dim() == 1, "scale_h must be 1-D")
    _check(scale_l is None or scale_l.dim() == 1, "scale_l must be 1-D")
    return n, r, m


def nanoquant_dyn_forward_cuda(x, scale_g, Ubits, scale_l, Vbits, scale_h, num_thread_stage1=128,
                               num_thread_stage2=128, num_row_per_warp_stage1=2, num_row_per_warp_stage2=2,
                               num_acc_stage1=4, num_acc_stage2=4, num_pipeline_stage1=2,
                               num_pipeline_stage2=2):
    """Device implementation of ``nanoquant_dyn_forward`` (gemv_kernel.cu:308-429)."""
    n, r, m = _gemv_args(x, scale_g, Ubits, scale_l, Vbits, scale_h)
    _check_tuning(num_thread_stage1, num_thread_stage2, num_row_per_warp_stage1, num_row_per_warp_stage2,
                  num_acc_stage1, num_acc_stage2, num_pipeline_stage1, num_pipeline_stage2)
    lead = tuple(x.shape[:-1])
    batch = 1
    for d in lead:
        batch *= d
    y = torch.empty(lead + (m,), dtype=x.dtype, device=x.device)
    if batch == 0 or m == 0:
        return y
    lib = _lib.load()
    with torch.cuda.device(x.device):
        stream = _lib.stream_of(x.device)
        ws = gemv_workspace(x.device, lib.nq_gemv_workspace_bytes(batch, n, r, m))
        status = lib.nq_gemv(_lib.dtype_code(x.dtype), x.data_ptr(), scale_g.data_ptr(), Ubits.data_ptr(),
                             _lib.ptr(scale_l), Vbits.data_ptr(), scale_h.data_ptr(), y.data_ptr(), batch, n, r, m,
                             ws.data_ptr(), ws.numel(), stream)
    _lib.check(status, "nanoquant_dyn_forward")
    return y


def nanoquant_dyn_forward_fake(x, scale_g, Ubits, scale_l, Vbits, scale_h, num_thread_stage1=128,
                               num_thread_stage2=128, num_row_per_warp_stage1=2, num_row_per_warp_stage2=2,
                               num_acc_stage1=4, num_acc_stage2=4, num_pipeline_stage1=2,
                               num_pipeline_stage2=2):
    """Shape-only implementation (pybind.cpp:11-32): x's shape with the last dim -> m."""
    return x.new_empty(tuple(x.shape[:-1]) + (scale_h.size(0),))


# --------------------------------------------------------------------------- Marlin GEMM

def _onebit_check_and_shape(x, weight, scale_g, scale_h, workspace, max_par=MARLIN_MIN_MAX_PAR):
    """marlin_onebit_check_and_alloc (gemm.cpp:36-56), without the allocation."""
    _check(x.dim() == 2, f"x must be 2-D, got {x.dim()}-D")
    _check(weight.dim() == 2, f"weight must be 2-D, got {weight.dim()}-D")
    prob_m = x.size(0)
    prob_n = weight.size(1) * 2
    prob_k = x.size(1)
    _check(prob_k == weight.size(0) * 16, "k dimension mismatch")
    _check(scale_g is None or scale_g.size(0) == prob_k, "s_in size mismatch")
    _check(scale_h is None or scale_h.size(0) == prob_n, "s_out size mismatch")
    _check(max_par >= MARLIN_MIN_MAX_PAR, f"max_par must be at least {MARLIN_MIN_MAX_PAR}")
    _check(workspace.numel() >= prob_n // 128 * max_par, "workspace too small")
    return prob_m, prob_n, prob_k


def _onebit_device_checks(x, weight, scale_g, scale_h):
    _check(x.dtype in (torch.float16, torch.bfloat16), "Unsupported dtype: Marlin only supports Half and BFloat16")
    _check(x.is_cuda and weight.is_cuda, "x and weight must be CUDA tensors")
    _check(x.is_contiguous() and weight.is_contiguous(), "x and weight must be contiguous")
    _check(weight.dtype == torch.int32, "weight tensor dtype must be int32")
    _check(weight.size(1) % 32 == 0, "weight must have a multiple of 32 columns (out_features % 64 == 0)")
    for name, s in (("scale_g", scale_g), ("scale_h", scale_h)):
        if s is not None:
            _check(s.is_cuda and s.is_contiguous(), f"{name} must be a contiguous CUDA tensor")
            _check(s.dtype == x.dtype, f"{name} must have the dtype of x ({x.dtype})")
            _check(s.dim() == 1, f"{name} must be 1-D")


def _split_workspace(device, nbytes):
    """Scratch for the GEMM's split-K partial sums (None when the shape does not split)."""
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def marlin_onebit_forward_cuda(x, weight, scale_g, scale_h, workspace):
    """Device implementation of ``marlin_onebit_forward`` (gemm.cpp:59-98)."""
    prob_m, prob_n, prob_k = _onebit_check_and_shape(x, weight, scale_g, scale_h, workspace)
    _onebit_device_checks(x, weight, scale_g, scale_h)
    C = torch.empty((prob_m, prob_n), dtype=x.dtype, device=x.device)
    if prob_m == 0 or prob_n == 0:
        return C
    lib = _lib.load()
    # fp32 partial sums when the library splits K across blocks (small grids); the caching
    # allocator makes this stream-ordered scratch
    split = _split_workspace(x.device, lib.nq_gemm_onebit_workspace_bytes(prob_m, prob_k, prob_n))
    with torch.cuda.device(x.device):
        status = lib.nq_gemm_onebit(_lib.dtype_code(x.dtype), x.data_ptr(), weight.data_ptr(), _lib.ptr(scale_g),
                                    _lib.ptr(scale_h), C.data_ptr(), prob_m, prob_k, prob_n, _lib.ptr(split),
                                    0 if split is None else split.numel(), _lib.stream_of(x.device))
    _lib.check(status, "marlin_onebit_forward")
    return C


def marlin_onebit_forward_fake(x, weight, scale_g, scale_h, workspace):
    prob_m, prob_n, _ = _onebit_check_and_shape(x, weight, scale_g, scale_h, workspace)
    return x.new_empty((prob_m, prob_n))


def marlin_nanoquant_forward_cuda(x, weight_u, weight_v, scale_g, scale_l, scale_h, workspace):
    """Device implementation of ``marlin_nanoquant_forward`` (gemm.cpp:112-122): the first
    stage maps x [B, n] through ``weight_u`` (V's bits) to imm [B, r'], the second maps imm
    through ``weight_v`` (U's bits) to y [B, m]."""
    prob_m, r_pad, n = _onebit_check_and_shape(x, weight_u, scale_g, scale_l, workspace)
    _onebit_device_checks(x, weight_u, scale_g, scale_l)
    _check(weight_v.dim() == 2, f"weight must be 2-D, got {weight_v.dim()}-D")
    _check(r_pad == weight_v.size(0) * 16, "k dimension mismatch")
    m = weight_v.size(1) * 2
    _check(scale_h is None or scale_h.size(0) == m, "s_out size mismatch")
    _check(workspace.numel() >= m // 128 * MARLIN_MIN_MAX_PAR, "workspace too small")
    _onebit_device_checks(x, weight_v, None, scale_h)
    imm = torch.empty((prob_m, r_pad), dtype=x.dtype, device=x.device)
    y = torch.empty((prob_m, m), dtype=x.dtype, device=x.device)
    if prob_m == 0 or m == 0:
        return y
    lib = _lib.load()
    split = _split_workspace(x.device, lib.nq_gemm_nanoquant_workspace_bytes(prob_m, n, r_pad, m))
    with torch.cuda.device(x.device):
        status = lib.nq_gemm_nanoquant(_lib.dtype_code(x.dtype), x.data_ptr(), weight_u.data_ptr(),
                                       weight_v.data_ptr(), _lib.ptr(scale_g), _lib.ptr(scale_l),
                                       _lib.ptr(scale_h), imm.data_ptr(), y.data_ptr(), prob_m, n, r_pad, m,
                                       _lib.ptr(split), 0 if split is None else split.numel(),
                                       _lib.stream_of(x.device))
    _lib.check(status, "marlin_nanoquant_forward")
    return y


def marlin_nanoquant_forward_fake(x, weight_u, weight_v, scale_g, scale_l, scale_h, workspace):
    """marlin_nanoquant_meta (gemm.cpp:124-134): both stages' checks, the final shape."""
    prob_m, r_pad, _ = _onebit_check_and_shape(x, weight_u, scale_g, scale_l, workspace)
    imm = x.new_empty((prob_m, r_pad))
    prob_m, m, _ = _onebit_check_and_shape(imm, weight_v, None, scale_h, workspace)
    return x.new_empty((prob_m, m))


# --------------------------------------------------------------------------- registration

def _register():
    lib = torch.library.Library(_NS, "DEF")
    lib.define(GEMV_SCHEMA)
    lib.define(ONEBIT_SCHEMA)
    lib.define(NANOQUANT_SCHEMA)
    lib.impl("nanoquant_dyn_forward", nanoquant_dyn_forward_cuda, "CUDA")
    lib.impl("marlin_onebit_forward", marlin_onebit_forward_cuda, "CUDA")
    lib.impl("marlin_nanoquant_forward", marlin_nanoquant_forward_cuda, "CUDA")
    torch.library.register_fake(f"{_NS}::nanoquant_dyn_forward", nanoquant_dyn_forward_fake, lib=lib)
    torch.library.register_fake(f"{_NS}::marlin_onebit_forward", marlin_onebit_forward_fake, lib=lib)
    torch.library.register_fake(f"{_NS}::marlin_nanoquant_forward", marlin_nanoquant_forward_fake, lib=lib)
    return lib


_LIBRARY = _register()


def ensure_loaded() -> None:
    """Raise ImportError unless the HIP library is present and loadable."""
    _lib.load()
