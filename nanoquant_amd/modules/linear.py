"""``NanoQuantLinear``: the binary low-rank linear layer, inference side.

The layer computes ``y = s_post * (U (s_mid * (V (s_pre * x))))`` with ``V`` [rank, in] and
``U`` [out, rank] holding +-1. What callers and checkpoints of the reference
(``src/nanoquant/modules/linear.py``) rely on, and what this class therefore keeps:

* conversion of an ``nn.Linear`` by ``lin.__class__ = NanoQuantLinear`` followed by
  ``init_for_inference(rank, has_scale_mid)`` (:116-129): frozen parameters ``scale_pre``
  [1, in], ``scale_post`` [1, out], ``V``, ``U`` and optionally ``scale_mid`` [1, rank], all in
  ``self.dtype`` (bf16), ``weight`` set to None, ``bias`` kept;
* the dense forward (:177-184 with :282-291), in the reference's operation order so that it
  rounds the same way, plus ``bias``;
* ``_prepare_kernel(kernel_type, dtype)`` (:186-238) leaving the attributes the reference
  leaves (``V_int8``/``U_int8``, scales squeezed to 1-D in ``dtype``, ``kernel_forward``,
  ``kernel_kwargs``; for "gemm" the Marlin words with ``s1``..``s3`` and ``workspace`` instead of
  the scales), after which ``forward`` casts x to ``dtype``, flattens a 3-D input, runs the
  kernel and restores shape and dtype (:136-175). The kernel paths add no ``bias``
  (:155-166), as in the reference;
* a state dict in which ``V``/``U`` appear as ``{name}_packed`` lsb_first sign words plus
  ``{name}_shape`` (:359-394), expanded back on load (:396-433).

Additions of this package: kernel type "auto" (GEMV up to ``auto_gemv_max_rows`` rows, GEMM
beyond), ``_prepare_kernel_from_packed`` and ``load_packed_for_kernels`` (kernel words made
straight from checkpoint words). Quantization-time training, knowledge distillation and the
gemlite kernel are not part of this package.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernel.utils import (binary_packer, binary_unpacker, get_kernel_function, marlin_nanoquant_packer,
                            pack_binary_marlin_fused_from_packed, repack_binary_gemv)

# Kernel type "auto" runs the GEMV while rows * rank * (in + out) stays within a work bound, and
# at most AUTO_GEMV_MAX_ROWS rows (at least AUTO_GEMV_MIN_ROWS); the GEMM otherwise. The bound
# depends on the layer's orientation: the GEMV's cost grows with the rows faster on a tall U (its
# stage 2) than on a wide V (its k-split stage 1), and the GEMM runs slower on a long K. Fitted on
# both kernels at 16-256 rows on every Llama-2-7B (1.0 and 0.55 bpw) and Llama-3-70B (0.55 bpw)
# linear shape (bench.py --batch-sweep --batch-sweep-shapes configs): the sum of the picked times
# over the 80 cells is 0.4% above always picking the faster op (worst cell 10.7%: Llama-3-70B q/o
# at 64 rows), against 10.3% above (worst 73%, Llama-3-70B down_proj at 128 rows) for a fixed
# switch at 128 rows. The GEMV won or tied at 16 rows on every shape.
AUTO_GEMV_WORK_TALL = 2.3e9  # out_features >= in_features
AUTO_GEMV_WORK_WIDE = 3.5e9  # in_features > out_features
AUTO_GEMV_MIN_ROWS = 16
AUTO_GEMV_MAX_ROWS = 256


def auto_gemv_max_rows(in_features: int, out_features: int, rank: int) -> int:
    """Rows up to which kernel type "auto" runs the GEMV on a layer of these sizes."""
    work = AUTO_GEMV_WORK_WIDE if in_features > out_features else AUTO_GEMV_WORK_TALL
    rows = int(work // max(1, rank * (in_features + out_features)))
    return max(AUTO_GEMV_MIN_ROWS, min(AUTO_GEMV_MAX_ROWS, rows))

# The GEMV tuning ints the reference fixes when it prepares the layer (linear.py:210-219). The
# HIP kernels validate them and choose their own launch shapes.
GEMV_TUNING = (("num_thread_stage1", 128), ("num_thread_stage2", 128), ("num_row_per_warp_stage1", 2),
               ("num_row_per_warp_stage2", 2), ("num_acc_stage1", 1), ("num_acc_stage2", 1),
               ("num_pipeline_stage1", 8), ("num_pipeline_stage2", 8))

KERNEL_TYPES = ("gemv", "gemm", "auto")
SIGN_FACTORS = ("V", "U")  # the +-1 factors, in the order the state dict packs them


class _SignPassThrough(torch.autograd.Function):
    """Exact +-1 signs (a zero counts as +1) whose gradient passes through unchanged (linear.py:15-23)."""

    @staticmethod
    def forward(ctx, value):
        return torch.where(value == 0, torch.ones_like(value), torch.sign(value))

    @staticmethod
    def backward(ctx, grad):
        return grad


def _frozen(t: torch.Tensor) -> nn.Parameter:
    return nn.Parameter(t, requires_grad=False)


class NanoQuantLinear(nn.Module):
    """Binary low-rank linear y = s_post * (U (s_mid * (V (s_pre * x)))) (+ bias on the dense path)."""

    # ------------------------------------------------------------------ construction

    def _parameter_shapes(self, with_mid: bool):
        shapes = {"scale_pre": (1, self.in_features), "scale_post": (1, self.out_features),
                  "V": (self.rank, self.in_features), "U": (self.out_features, self.rank)}
        if with_mid:
            shapes["scale_mid"] = (1, self.rank)
        return shapes

    def _home_device(self) -> torch.device:
        bias = getattr(self, "bias", None)
        return bias.device if bias is not None else torch.device("cpu")

    def init_for_inference(self, rank, has_scale_mid=False):
        """Give a converted ``nn.Linear`` the empty factors and scales of a NanoQuant layer
        (linear.py:116-129): bf16, frozen, on the bias's device (else the CPU)."""
        self.rank = rank
        self.do_train = False
        self._binarized = True
        self.dtype = torch.bfloat16
        self._parameters.pop("weight", None)
        self.register_parameter("weight", None)
        self._setup_path(None, with_mid=has_scale_mid)
        if not has_scale_mid and hasattr(self, "scale_mid"):
            delattr(self, "scale_mid")

    def _setup_path(self, factors, with_mid: bool = True):
        """Create the parameters: empty ones of the layer's shapes (``factors`` None), or the signs
        of solved factors (``B`` [rank, in] gives V, the transpose of ``A`` [rank, out] gives U)
        with their scales (the inference branch of linear.py:74-114)."""
        if factors is None:
            home = self._home_device()
            values = {name: torch.empty(shape, device=home)
                      for name, shape in self._parameter_shapes(with_mid).items()}
        else:
            values = {"scale_pre": factors.scale_pre.float(), "scale_post": factors.scale_post.float(),
                      "V": self.binary_ste(factors.B.float()), "U": self.binary_ste(factors.A.float().mT)}
            if getattr(factors, "scale_mid", None) is not None:
                values["scale_mid"] = factors.scale_mid.float()
        for name, value in values.items():
            setattr(self, name, _frozen(value.to(self.dtype)))

    def binary_ste(self, x):
        return _SignPassThrough.apply(x)

    def quantize(self, x):
        return x if self._binarized else self.binary_ste(x)

    # ------------------------------------------------------------------ forward

    def forward(self, x):
        if getattr(self, "do_kernel_inference", False):
            return self._kernel_forward(x)
        y = self._compute_forward(x, self.V, self.U, self.scale_pre, getattr(self, "scale_mid", None),
                                  self.scale_post)
        return y if self.bias is None else y + self.bias

    def _compute_forward(self, x, V, U, scale_pre, scale_mid, scale_post):
        """The dense dequantize-and-matmul path (linear.py:282-291): scale, V, mid scale, U, scale,
        each rounded in the tensors' dtype in that order."""
        hidden = F.linear(x * scale_pre, self.quantize(V))
        if scale_mid is not None:
            hidden = hidden * scale_mid
        return F.linear(hidden, self.quantize(U)) * scale_post

    def _kernel_forward(self, x):
        if x.ndim not in (2, 3):
            raise ValueError(f"Expected 2D or 3D input tensor, got {x.ndim}D")
        caller_dtype = x.dtype
        lead = x.shape[:-1]
        rows = x.to(self.dtype).contiguous().reshape(-1, x.shape[-1])
        y = self._run_kernel(rows).reshape(*lead, -1)
        return y if y.dtype == caller_dtype else y.to(caller_dtype)

    def _run_kernel(self, rows):
        kind = self.kernel_type
        if kind == "gemv" or (kind == "auto" and rows.size(0) <= self.auto_gemv_rows):
            return self.kernel_forward(rows, self.scale_pre, self.V_int8, self.scale_mid, self.U_int8,
                                       self.scale_post, **self.kernel_kwargs)
        if kind == "gemm":
            return self.kernel_forward(rows, self.V_int8, self.U_int8, self.s1, self.s2, self.s3, self.workspace)
        if kind == "auto":
            return self.gemm_forward(rows, self.V_marlin, self.U_marlin, self.s1, self.s2, self.s3, self.workspace)
        raise ValueError(f"Unknown kernel_type: {kind}")

    # ------------------------------------------------------------------ kernel preparation

    @staticmethod
    def _check_kernel_type(kernel_type):
        if kernel_type == "gemlite":
            raise NotImplementedError("the gemlite kernel is not part of nanoquant_amd; use 'gemv' or 'gemm'")
        if kernel_type not in KERNEL_TYPES:
            raise ValueError("kernel_type must be one of ['gemv', 'gemm', 'gemlite', 'auto'].")

    def _enter_kernel_mode(self, kernel_type, dtype):
        """Common part of both preparations: the flags, and the scales as 1-D ``dtype`` parameters
        (``scale_mid`` becomes a plain None when the layer has none, linear.py:198-203)."""
        self.do_kernel_inference = True
        self.kernel_type = kernel_type
        self.dtype = dtype
        self.auto_gemv_rows = auto_gemv_max_rows(self.in_features, self.out_features, self.rank)
        for name in ("scale_pre", "scale_post", "scale_mid"):
            value = getattr(self, name, None)
            setattr(self, name, None if value is None else _frozen(value.to(dtype).squeeze(0)))

    def _mid_or_ones(self, dtype):
        if self.scale_mid is not None:
            return self.scale_mid
        return torch.ones(self.rank, device=self.scale_pre.device, dtype=dtype)

    def _use_gemv_words(self, U_words, V_words, dtype):
        self.U_int8, self.V_int8 = U_words, V_words
        self.kernel_forward = get_kernel_function("nanoquant", dtype, kernel_type="dynamic")
        self.kernel_kwargs = dict(GEMV_TUNING)

    def _use_gemm_words(self, marlin, dtype, keep_gemv: bool):
        """``marlin`` is the packer's (V words, U words, s1, s2, s3, workspace). With
        ``keep_gemv`` (kernel type "auto") the GEMV words stay in V_int8/U_int8 and the GEMM
        gets V_marlin/U_marlin; otherwise the Marlin words take V_int8/U_int8 and the scales go."""
        words_v, words_u, self.s1, self.s2, self.s3, self.workspace = marlin
        gemm = get_kernel_function("marlin_nanoquant", dtype, kernel_type="fixed")
        if keep_gemv:
            self.V_marlin, self.U_marlin, self.gemm_forward = words_v, words_u, gemm
            return
        self.V_int8, self.U_int8, self.kernel_forward = words_v, words_u, gemm
        for name in ("scale_pre", "scale_mid", "scale_post"):
            delattr(self, name)

    def _drop_dense_factors(self):
        for name in SIGN_FACTORS:
            if hasattr(self, name):
                delattr(self, name)

    def _prepare_kernel(self, kernel_type="gemv", dtype=torch.float16):
        """Pack the dense factors for a kernel and route ``forward`` through it (linear.py:186-238).

        "gemv": half2 sign words. "gemm": the Marlin layout (a missing ``scale_mid`` becomes ones,
        linear.py:221-225). "auto" (this package): both, the GEMV taking up to
        ``auto_gemv_max_rows(in, out, rank)`` rows and the GEMM more.
        """
        self._check_kernel_type(kernel_type)
        self._enter_kernel_mode(kernel_type, dtype)
        U8, V8 = self.U.to(torch.int8), self.V.to(torch.int8)
        if kernel_type != "gemm":
            self._use_gemv_words(binary_packer(U8, method="half2"), binary_packer(V8, method="half2"), dtype)
        if kernel_type != "gemv":
            if kernel_type == "gemm" and self.scale_mid is None:
                self.scale_mid = _frozen(self._mid_or_ones(dtype))
            marlin = marlin_nanoquant_packer(V8.T, U8.T, self.scale_pre, self._mid_or_ones(dtype), self.scale_post)
            self._use_gemm_words(marlin, dtype, keep_gemv=kernel_type == "auto")
        self._drop_dense_factors()

    def _prepare_kernel_from_packed(self, V_packed, V_shape, U_packed, U_shape, kernel_type="gemv",
                                    dtype=torch.float16, method="lsb_first"):
        """``_prepare_kernel`` from the factors' packed sign words instead of dense V/U.

        ``V_packed``/``U_packed`` are the words of V [rank, in] and U [out, rank] in ``method``
        order (a checkpoint's ``{name}_packed`` entries, lsb_first, linear.py:359-376). The kernel
        words are made from them on the GPU (half2 for gemv; Marlin, rank padding included, for
        gemm) and are bit-identical to what ``_prepare_kernel`` makes from the dense factors;
        the dense factors are never built (the reference unpacks them at load,
        load_utils.py:392, and packs them again, linear.py:205-206,226-232).
        """
        self._check_kernel_type(kernel_type)
        V_shape = tuple(int(s) for s in V_shape)
        U_shape = tuple(int(s) for s in U_shape)
        if V_shape != (self.rank, self.in_features) or U_shape != (self.out_features, self.rank):
            raise ValueError(f"packed factor shapes {V_shape}, {U_shape} do not match rank {self.rank}, "
                             f"in {self.in_features}, out {self.out_features}")
        self._drop_dense_factors()
        self._enter_kernel_mode(kernel_type, dtype)
        home = self.scale_pre.device
        V_packed, U_packed = V_packed.to(home), U_packed.to(home)
        if kernel_type != "gemm":
            self._use_gemv_words(repack_binary_gemv(U_packed, U_shape, method, "half2"),
                                 repack_binary_gemv(V_packed, V_shape, method, "half2"), dtype)
        if kernel_type != "gemv":
            if kernel_type == "gemm" and self.scale_mid is None:
                self.scale_mid = _frozen(self._mid_or_ones(dtype))
            marlin = pack_binary_marlin_fused_from_packed(V_packed, V_shape, U_packed, U_shape, self.scale_pre,
                                                          self._mid_or_ones(dtype), self.scale_post, method)
            self._use_gemm_words(marlin, dtype, keep_gemv=kernel_type == "auto")

    # ------------------------------------------------------------------ packed state dict

    def pack_weights(self):
        """``{name}_packed`` (lsb_first int32 words) and ``{name}_shape`` (int64) of each sign
        factor the layer still holds (linear.py:359-376); ValueError when one is not all +-1."""
        out = {}
        for name in SIGN_FACTORS:
            factor = getattr(self, name, None)
            if factor is None:
                continue
            signs = factor.data
            if not bool(((signs == 1) | (signs == -1)).all()):
                raise ValueError(f"Cannot pack {name}: factors must contain only -1 and +1")
            out[f"{name}_packed"] = binary_packer(signs.to(torch.int8))
            out[f"{name}_shape"] = torch.tensor(tuple(factor.shape), dtype=torch.long)
        return out

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        """Save as nn.Module does, with each dense sign factor replaced by its packed words
        (linear.py:378-394)."""
        super()._save_to_state_dict(destination, prefix, keep_vars)
        if getattr(self, "do_train", False):
            return
        for name in SIGN_FACTORS:
            destination.pop(prefix + name, None)
        for key, value in self.pack_weights().items():
            destination[prefix + key] = value

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        """Expand ``{name}_packed``/``{name}_shape`` into dense factors in ``self.dtype``, then load
        as usual; a state without ``scale_mid`` removes the layer's (linear.py:396-433)."""
        if prefix + "scale_mid" not in state_dict and hasattr(self, "scale_mid"):
            delattr(self, "scale_mid")
        for name in SIGN_FACTORS:
            words_key, shape_key = f"{prefix}{name}_packed", f"{prefix}{name}_shape"
            if words_key in state_dict and shape_key in state_dict:
                words = state_dict.pop(words_key)
                shape = tuple(state_dict.pop(shape_key).tolist())
                state_dict[prefix + name] = binary_unpacker(words, shape).to(self.dtype)
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
    pending = []
    for name, mod in model.named_modules():
        if not isinstance(mod, NanoQuantLinear):
            continue
        prefix = f"{name}." if name else ""
        words = []
        for factor in SIGN_FACTORS:
            wk, sk = f"{prefix}{factor}_packed", f"{prefix}{factor}_shape"
            if wk not in state or sk not in state:
                raise KeyError(f"missing {wk} or {sk} in the packed state dict")
            words += [state.pop(wk), tuple(int(s) for s in state.pop(sk).tolist())]
        for factor in SIGN_FACTORS:  # never loaded densely
            mod._parameters.pop(factor, None)
        pending.append((mod, words))
    result = model.load_state_dict(state, strict=False)
    for mod, words in pending:
        mod._prepare_kernel_from_packed(*words, kernel_type=kernel_type, dtype=dtype, method=method)
    return result
