"""ctypes binding of the C ABI in ``include/nq_hip.h`` (``libnq_hip.so``).

torch is imported first so that the library binds to the HIP runtime torch has
already loaded (both carry the soname ``libamdhip64.so.7``): device pointers and
``hipStream_t`` handles from torch are then valid in the library.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_NAME = "libnq_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

NQ_OK = 0
NQ_ERR_INVALID_ARGUMENT = 1
NQ_ERR_SHAPE = 2
NQ_ERR_DTYPE = 3
NQ_ERR_ALIGNMENT = 4
NQ_ERR_WORKSPACE = 5
NQ_ERR_HIP = 6
NQ_ERR_UNSUPPORTED = 7

NQ_F16 = 0
NQ_BF16 = 1
NQ_PACK_LSB_FIRST = 0
NQ_PACK_HALF2 = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_size = ctypes.c_size_t

NQ_EPI_STORE = 0
NQ_EPI_RESIDUAL = 1
NQ_EPI_GATED = 2


class GemvItem(ctypes.Structure):
    """``nq_gemv_item`` of include/nq_hip.h."""

    _fields_ = [
        ("v_bits", _vp), ("s_in", _vp), ("s_mid", _vp), ("u_bits", _vp), ("s_out", _vp), ("y", _vp),
        ("resid", _vp), ("r", _i64), ("m", _i64), ("y_stride", _i64),
    ]


_items_p = ctypes.POINTER(GemvItem)

# name -> (restype, argtypes); every function declared in include/nq_hip.h
SIGNATURES = {
    "nq_status_string": (ctypes.c_char_p, [_int]),
    "nq_last_error_message": (ctypes.c_char_p, []),
    "nq_version": (_int, []),
    "nq_pack_signs": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "nq_unpack_signs": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "nq_repack_signs": (_int, [_vp, _vp, _i64, _i64, _int, _int, _vp]),
    "nq_pack_marlin": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "nq_unpack_marlin": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "nq_repack_marlin": (_int, [_vp, _i64, _i64, _int, _vp, _i64, _i64, _vp]),
    "nq_permute_marlin_scales": (_int, [_vp, _vp, _i64, _vp, _vp, _i64, _vp]),
    "nq_gemv_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "nq_gemv": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _size, _vp]),
    "nq_gemv_stage1": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _size, _vp]),
    "nq_gemv_stage2": (_int, [_int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _size, _vp]),
    "nq_gemv_noalloc": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "nq_gemv_group_workspace_bytes": (_size, [_i64, _items_p, _i64]),
    "nq_gemv_group_stage1": (_int, [_int, _i64, _items_p, _vp, _i64, _i64, ctypes.c_float, _vp, _size, _vp]),
    "nq_gemv_group_stage2": (_int, [_int, _i64, _items_p, _i64, _int, _vp, _size, _vp]),
    "nq_gemv_group_stage2_rope": (_int, [_int, _items_p, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp,
                                         _size, _vp]),
    "nq_gemv_group_stage2_kv": (_int, [_int, _items_p, _i64, _vp, _vp, _i64, _i64, _vp, _size, _vp]),
    "nq_attention_decode_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "nq_attention_decode": (_int, [_int, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                   _i64, ctypes.c_float, _vp, _size, _vp]),
    "nq_rope_kv_write": (_int, [_int, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _vp]),
    "nq_dense_gemv": (_int, [_int, _vp, _vp, _vp, ctypes.c_float, _vp, _int, _i64, _i64, _i64, _i64, _vp]),
    "nq_argmax_rows": (_int, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "nq_gemm_onebit_workspace_bytes": (_size, [_i64, _i64, _i64]),
    "nq_gemm_onebit": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _size, _vp]),
    "nq_gemm_nanoquant_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "nq_gemm_nanoquant": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _size,
                                 _vp]),
    "nq_timestamp": (_int, [_vp, _vp]),
    "nq_wall_clock_hz": (_i64, []),
    "nq_probe_empty": (_int, [_i64, _i64, _vp]),
    "nq_probe_read": (_int, [_vp, _i64, _i64, _vp, _int, _vp]),
}


_lock = threading.Lock()
_lib = None


class NQError(RuntimeError):
    """A failure status returned by the HIP library."""

    def __init__(self, status: int, what: str, detail: str):
        super().__init__(f"{what}: {detail or 'error'} [{status}]")
        self.status = status


def load() -> ctypes.CDLL:
    """Load the library once; ImportError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(f"the nanoquant_amd HIP library is not built ({LIB_PATH} is missing); "
                                  "run `python -m nanoquant_amd.build`")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != NQ_OK:
        detail = load().nq_last_error_message().decode(errors="replace")
        raise NQError(status, what, detail)


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(device) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype) -> int:
    if dtype == torch.float16:
        return NQ_F16
    if dtype == torch.bfloat16:
        return NQ_BF16
    raise TypeError(f"unsupported dtype {dtype}")
