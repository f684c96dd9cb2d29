"""MI355X-native (gfx950) NanoQuant inference path: sign packing, decode GEMV and
prefill GEMM as HIP kernels behind ``torch.ops.binary_kernels``.

Importing the package registers the operators; the HIP library
(``libnq_hip.so``, built by ``python -m nanoquant_amd.build``) is loaded on first use.
"""
from . import binary_kernels  # noqa: F401  (registers torch.ops.binary_kernels.*)
from .kernel.utils import (binary_packer, binary_unpacker, get_kernel_function, marlin_nanoquant_packer,  # noqa: F401
                           marlin_onebit_packer, pack_binary_gemv, pack_binary_marlin, pack_binary_marlin_fused,
                           pack_binary_marlin_fused_from_packed, repack_binary_gemv, repack_binary_marlin,
                           unpack_binary_gemv)
from .modules.linear import NanoQuantLinear, load_packed_for_kernels  # noqa: F401

__all__ = [
    "NanoQuantLinear", "pack_binary_gemv", "unpack_binary_gemv", "repack_binary_gemv", "pack_binary_marlin",
    "pack_binary_marlin_fused", "get_kernel_function", "binary_packer", "binary_unpacker", "marlin_onebit_packer",
    "marlin_nanoquant_packer", "repack_binary_marlin", "pack_binary_marlin_fused_from_packed",
    "load_packed_for_kernels",
]
