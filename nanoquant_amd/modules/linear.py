"""``NanoQuantLinear``: the quantized linear of the reference, inference side.

Mirrors the inference surface of ``src/nanoquant/modules/linear.py``: conversion of
an ``nn.Linear`` by ``module.__class__ = NanoQuantLinear`` plus
``init_for_inference`` (:116-129), the dense forward (:177-184, :282-291), the
kernel forward (:136-175) with ``_prepare_kernel`` for the ``gemv`` and ``gemm``
kernels (:186-238), and the packed ``state_dict`` round trip (:359-433). The
packers and ops it calls are this package's HIP-backed ones.

As in the reference, the kernel forwards do not add ``bias`` (linear.py:155-166;
only the dense path adds it, :182-183). Quantization-time training, knowledge
distillation and the gemlite kernel are not part of this package.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernel.utils import (binary_packer, binary_unpacker, get_kernel_function, marlin_nanoquant_packer,
                            pack_binary_marlin_fused_from_packed, repack_binary_gemv)

# Rows up to which kernel_type "auto" runs the GEMV; more rows run the GEMM. Measured on the
# Llama-2-7B gate and down shapes at 0.55 bpw (bench.py --batch-sweep): at 64 rows the GEMV takes
# 34.4 and 37.5 us against the GEMM's 35.3 and 38.5 us, at 128 rows 63 and 69 us against 41 and 45 us.
AUTO_GEMV_MAX_ROWS = 64

# The GEMV tuning ints _prepare_kernel fixes (linear.py:210-219); the kernels here accept and
# validate them but pick their own launch shapes.
_GEMV_KWARGS = {
    "num_thread_stage1": 128,
    "num_thread_stage2": 128,
    "num_row_per_warp_stage1": 2,
    "num_row_per_warp_stage2": 2,
    "num_acc_stage1": 1,
    "num_acc_stage2": 1,
    "num_pipeline_stage1": 8,
    "num_pipeline_stage2": 8,
}


class _BinarySignSTE(torch.autograd.Function):
    """sign() with 0 -> +1 and an identity backward (linear.py:15-23)."""

    @staticmethod
    def forward(ctx, value):
        signs = value.sign()
        return signs.masked_fill_(signs == 0, 1)

    @staticmethod
    def backward(ctx, grad_output):
        return grad_output


class NanoQuantLinear(nn.Module):
    """Binary low-rank linear y = s_post * (U (s_mid * (V (s_pre * x)))) (+ bias on the dense path).

    V [rank, in_features] and U [out_features, rank] hold +-1; scale_pre [1, in],
    scale_mid [1, rank] (optional) and scale_post [1, out] are the scales.
    """

    def init_for_inference(self, rank, has_scale_mid=False):
        """Turn a converted ``nn.Linear`` into an empty NanoQuant layer (linear.py:116-129)."""
        self.rank = rank
        self.do_train = False
        self._binarized = True
        self.dtype = torch.bfloat16

        if "weight" in self._parameters:
            del self._parameters["weight"]
        self.register_parameter("weight", None)

        self._setup_path(factors=None)

        if not has_scale_mid and hasattr(self, "scale_mid"):
            delattr(self, "scale_mid")

    def _setup_path(self, factors):
        """Create the factor and scale parameters (linear.py:74-114, inference branch)."""
        if factors is not None:
            vals = {
                "scale_pre": factors.scale_pre.float(),
                "scale_post": factors.scale_post.float(),
                "V": self.binary_ste(factors.B.float()),
                "U": self.binary_ste(factors.A.float().mT),
            }
            if getattr(factors, "scale_mid", None) is not None:
                vals["scale_mid"] = factors.scale_mid.float()
        else:
            device = None
            if getattr(self, "bias", None) is not None:
                device = self.bias.device
            if device is None:
                device = torch.device("cpu")
            vals = {
                "scale_pre": torch.empty(1, self.in_features, device=device),
                "scale_post": torch.empty(1, self.out_features, device=device),
                "V": torch.empty(self.rank, self.in_features, device=device),
                "U": torch.empty(self.out_features, self.rank, device=device),
                "scale_mid": torch.empty(1, self.rank, device=device),
            }
        for name, tensor in vals.items():
            setattr(self, name, nn.Parameter(tensor.to(self.dtype), requires_grad=False))

    def binary_ste(self, x):
        return _BinarySignSTE.apply(x)

    def quantize(self, x):
        if self._binarized:
            return x
        return self.binary_ste(x)

    # ------------------------------------------------------------------ forward

    def forward(self, x):
        if getattr(self, "do_kernel_inference", False):
            orig_dtype = x.dtype
            if x.dtype != self.dtype:
                x = x.to(self.dtype)

            original_shape = None
            if x.ndim == 3:
                original_shape = x.shape
                x = x.contiguous().view(-1, x.size(-1))
            elif x.ndim == 2:
                x = x.contiguous()
            else:
                raise ValueError(f"Expected 2D or 3D input tensor, got {x.ndim}D")

            if self.kernel_type == "gemv" or (self.kernel_type == "auto" and x.size(0) <= AUTO_GEMV_MAX_ROWS):
                y = self.kernel_forward(x, self.scale_pre, self.V_int8, self.scale_mid, self.U_int8,
                                        self.scale_post, **self.kernel_kwargs)
            elif self.kernel_type == "gemm":
                y = self.kernel_forward(x, self.V_int8, self.U_int8, self.s1, self.s2, self.s3, self.workspace)
            elif self.kernel_type == "auto":
                y = self.gemm_forward(x, self.V_marlin, self.U_marlin, self.s1, self.s2, self.s3, self.workspace)
            else:
                raise ValueError(f"Unknown kernel_type: {self.kernel_type}")

            if original_shape is not None:
                y = y.view(original_shape[0], original_shape[1], -1)

            return y.to(orig_dtype) if y.dtype != orig_dtype else y

        s_mid_m = getattr(self, "scale_mid", None)
        y = self._compute_forward(x, self.V, self.U, self.scale_pre, s_mid_m, self.scale_post)
        if self.bias is not None:
            y += self.bias
        return y

    def _compute_forward(self, x, V, U, scale_pre, scale_mid, scale_post):
        """Dense dequantize-and-matmul path (linear.py:282-291)."""
        Vq = self.quantize(V)
        Uq = self.quantize(U)
        y = F.linear(x * scale_pre, Vq)
        if scale_mid is not None:
            y = y * scale_mid
        y = F.linear(y, Uq)
        return y * scale_post

    def _prepare_kernel(self, kernel_type="gemv", dtype=torch.float16):
        """Pack the factors for a kernel and switch the forward to it (linear.py:186-238).

        Besides the reference's "gemv" and "gemm", "auto" keeps both layouts (V_int8/U_int8 in
        half2 order for the GEMV, V_marlin/U_marlin with s1..s3 and the workspace for the GEMM)
        and runs each call on the GEMV up to AUTO_GEMV_MAX_ROWS rows, on the GEMM beyond.
        """
        self.do_kernel_inference = True
        self.kernel_type = kernel_type
        self.dtype = dtype

        if kernel_type == "gemlite":
            raise NotImplementedError("the gemlite kernel is not part of nanoquant_amd; use 'gemv' or 'gemm'")

        self.scale_pre = nn.Parameter(self.scale_pre.to(dtype).squeeze(0), requires_grad=False)
        self.scale_post = nn.Parameter(self.scale_post.to(dtype).squeeze(0), requires_grad=False)
        self.scale_mid = getattr(self, "scale_mid", None)
        if self.scale_mid is not None:
            self.scale_mid = nn.Parameter(self.scale_mid.to(dtype).squeeze(0), requires_grad=False)

        if kernel_type == "gemv":
            self.U_int8 = binary_packer(self.U.to(torch.int8), method="half2")
            self.V_int8 = binary_packer(self.V.to(torch.int8), method="half2")
            delattr(self, "U")
            delattr(self, "V")
            self.kernel_forward = get_kernel_function("nanoquant", dtype, kernel_type="dynamic")
            self.kernel_kwargs = dict(_GEMV_KWARGS)
        elif kernel_type == "gemm":
            if self.scale_mid is None:
                self.scale_mid = nn.Parameter(
                    torch.ones(self.rank, device=self.scale_pre.device, dtype=dtype), requires_grad=False)
            (self.V_int8, self.U_int8, self.s1, self.s2, self.s3, self.workspace) = marlin_nanoquant_packer(
                self.V.to(torch.int8).T,
                self.U.to(torch.int8).T,
                self.scale_pre,
                self.scale_mid,
                self.scale_post,
            )
            for key in ["U", "V", "scale_pre", "scale_mid", "scale_post"]:
                delattr(self, key)
            self.kernel_forward = get_kernel_function("marlin_nanoquant", dtype, kernel_type="fixed")
        elif kernel_type == "auto":
            U8, V8 = self.U.to(torch.int8), self.V.to(torch.int8)
            self.U_int8 = binary_packer(U8, method="half2")
            self.V_int8 = binary_packer(V8, method="half2")
            s_mid = self.scale_mid
            if s_mid is None:
                s_mid = torch.ones(self.rank, device=self.scale_pre.device, dtype=dtype)
            (self.V_marlin, self.U_marlin, self.s1, self.s2, self.s3, self.workspace) = marlin_nanoquant_packer(
                V8.T, U8.T, self.scale_pre, s_mid, self.scale_post)
            delattr(self, "U")
            delattr(self, "V")
            self._set_auto_forwards(dtype)
        else:
            raise ValueError("kernel_type must be one of ['gemv', 'gemm', 'gemlite', 'auto'].")

    def _set_auto_forwards(self, dtype):
        self.kernel_forward = get_kernel_function("nanoquant", dtype, kernel_type="dynamic")
        self.kernel_kwargs = dict(_GEMV_KWARGS)
        self.gemm_forward = get_kernel_function("marlin_nanoquant", dtype, kernel_type="fixed")

    def _prepare_kernel_from_packed(self, V_packed, V_shape, U_packed, U_shape, kernel_type="gemv",
                                    dtype=torch.float16, method="lsb_first"):
        """``_prepare_kernel`` from the factors' packed sign words instead of dense V/U.

        ``V_packed``/``U_packed`` are the words of V [rank, in] and U [out, rank] in ``method``
        order (a checkpoint's ``{name}_packed`` entries, lsb_first, linear.py:359-376). The kernel
        words are made from them on the GPU (half2 for gemv; Marlin, rank padding included, for
        gemm) and are bit-identical to what ``_prepare_kernel`` makes from the dense factors;
        the dense factors are never built (the reference unpacks them at load,
        load_utils.py:392, and packs them again here, linear.py:205-206,226-232).
        """
        if kernel_type == "gemlite":
            raise NotImplementedError("the gemlite kernel is not part of nanoquant_amd; use 'gemv' or 'gemm'")
        if kernel_type not in ("gemv", "gemm", "auto"):
            raise ValueError("kernel_type must be one of ['gemv', 'gemm', 'gemlite', 'auto'].")
        V_shape = tuple(int(s) for s in V_shape)
        U_shape = tuple(int(s) for s in U_shape)
        if V_shape != (self.rank, self.in_features) or U_shape != (self.out_features, self.rank):
            raise ValueError(f"packed factor shapes {V_shape}, {U_shape} do not match rank {self.rank}, "
                             f"in {self.in_features}, out {self.out_features}")
        device = self.scale_pre.device
        V_packed = V_packed.to(device)
        U_packed = U_packed.to(device)
        for name in ("U", "V"):
            if name in self._parameters:
                del self._parameters[name]
        self.do_kernel_inference = True
        self.kernel_type = kernel_type
        self.dtype = dtype
        self.scale_pre = nn.Parameter(self.scale_pre.to(dtype).squeeze(0), requires_grad=False)
        self.scale_post = nn.Parameter(self.scale_post.to(dtype).squeeze(0), requires_grad=False)
        self.scale_mid = getattr(self, "scale_mid", None)
        if self.scale_mid is not None:
            self.scale_mid = nn.Parameter(self.scale_mid.to(dtype).squeeze(0), requires_grad=False)

        if kernel_type in ("gemv", "auto"):
            self.U_int8 = repack_binary_gemv(U_packed, U_shape, method, "half2")
            self.V_int8 = repack_binary_gemv(V_packed, V_shape, method, "half2")
            self.kernel_forward = get_kernel_function("nanoquant", dtype, kernel_type="dynamic")
            self.kernel_kwargs = dict(_GEMV_KWARGS)
        if kernel_type == "auto":
            s_mid = self.scale_mid
            if s_mid is None:
                s_mid = torch.ones(self.rank, device=device, dtype=dtype)
            (self.V_marlin, self.U_marlin, self.s1, self.s2, self.s3, self.workspace) = \
                pack_binary_marlin_fused_from_packed(V_packed, V_shape, U_packed, U_shape, self.scale_pre, s_mid,
                                                     self.scale_post, method)
            self._set_auto_forwards(dtype)
        elif kernel_type == "gemm":
            if self.scale_mid is None:
                self.scale_mid = nn.Parameter(torch.ones(self.rank, device=device, dtype=dtype), requires_grad=False)
            (self.V_int8, self.U_int8, self.s1, self.s2, self.s3, self.workspace) = \
                pack_binary_marlin_fused_from_packed(V_packed, V_shape, U_packed, U_shape, self.scale_pre,
                                                     self.scale_mid, self.scale_post, method)
            for key in ["scale_pre", "scale_mid", "scale_post"]:
                delattr(self, key)
            self.kernel_forward = get_kernel_function("marlin_nanoquant", dtype, kernel_type="fixed")

    # ------------------------------------------------------------------ packed state dict

    def pack_weights(self):
        """``{name}_packed`` lsb_first int32 words and ``{name}_shape`` for V and U (linear.py:359-376)."""
        packed_data = {}

        def pack_param(param_name):
            if not hasattr(self, param_name):
                return
            param = getattr(self, param_name)
            if param is None:
                return
            param_bin = param.data
            if not torch.all((param_bin == 1) | (param_bin == -1)):
                raise ValueError(f"Cannot pack {param_name}: factors must contain only -1 and +1")
            packed_data[f"{param_name}_packed"] = binary_packer(param_bin.to(torch.int8))
            packed_data[f"{param_name}_shape"] = torch.tensor(param.shape, dtype=torch.long)

        pack_param("V")
        pack_param("U")
        return packed_data

    def state_dict(self, *args, **kwargs):
        """State dict with V/U replaced by their packed words (linear.py:378-394)."""
        state = super().state_dict(*args, **kwargs)
        prefix = kwargs.get("prefix", "")
        for name in ("U", "V"):
            state.pop(prefix + name, None)
        for k, v in self.pack_weights().items():
            state[prefix + k] = v
        return state

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        """Unpack ``*_packed``/``*_shape`` into V/U before the default load (linear.py:396-433)."""
        has_mid = (prefix + "scale_mid") in state_dict
        if not has_mid and hasattr(self, "scale_mid"):
            delattr(self, "scale_mid")

        def unpack_param(param_name):
            packed_key = prefix + f"{param_name}_packed"
            shape_key = prefix + f"{param_name}_shape"
            if packed_key in state_dict and shape_key in state_dict:
                packed_val = state_dict.pop(packed_key)
                shape = state_dict.pop(shape_key)
                state_dict[prefix + param_name] = binary_unpacker(packed_val, tuple(shape.tolist())).to(self.dtype)

        unpack_param("V")
        unpack_param("U")
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)


def load_packed_for_kernels(model: nn.Module, state_dict: dict, kernel_type: str = "gemv",
                            dtype: torch.dtype = torch.float16, method: str = "lsb_first"):
    """Load a packed NanoQuant state dict with every ``NanoQuantLinear`` made ready for a kernel.

    ``state_dict`` is what ``model.state_dict()`` saves: ``{name}_packed`` sign words and
    ``{name}_shape`` for V and U (linear.py:359-394), scales and every other parameter as is.
    The other entries load as usual; each NanoQuantLinear then takes the kernel words straight
    from its packed entries (``_prepare_kernel_from_packed``), so no dense +-1 factor is ever
    built, on the host or the GPU. The reference's route is ``load_state_dict`` (unpacking the
    words to dense factors, load_utils.py:392, linear.py:396-433) then ``_prepare_kernel``.
    Returns ``load_state_dict``'s result for the remaining entries; a missing packed entry raises
    KeyError.
    """
    state = dict(state_dict)
    layers = []
    for name, mod in model.named_modules():
        if not isinstance(mod, NanoQuantLinear):
            continue
        prefix = f"{name}." if name else ""
        words = {}
        for p in ("V", "U"):
            pk, sk = f"{prefix}{p}_packed", f"{prefix}{p}_shape"
            if pk not in state or sk not in state:
                raise KeyError(f"missing {pk} or {sk} in the packed state dict")
            words[p] = (state.pop(pk), tuple(int(s) for s in state.pop(sk).tolist()))
        for p in ("V", "U"):  # never loaded densely
            if p in mod._parameters:
                del mod._parameters[p]
        layers.append((mod, words))
    result = model.load_state_dict(state, strict=False)
    for mod, words in layers:
        mod._prepare_kernel_from_packed(*words["V"], *words["U"], kernel_type=kernel_type, dtype=dtype, method=method)
    return result
