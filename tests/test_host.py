"""Host-side checks that need no GPU: the C ABI library, op schemas, fake shapes,
argument validation and the module's dense path."""
import os
import re

import numpy as np
import pytest
import torch
import torch.nn as nn

import nanoquant_amd
import oracle as O
from nanoquant_amd import _lib, binary_kernels as bk
from nanoquant_amd.kernel import utils as ku
from nanoquant_amd.modules.linear import NanoQuantLinear

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nq_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(nq_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert "nq_gemv" in names and "nq_gemm_nanoquant" in names and "nq_pack_signs" in names
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.nq_version() >= 100
    assert lib.nq_status_string(0) == b"ok"
    assert lib.nq_status_string(_lib.NQ_ERR_WORKSPACE) == b"workspace too small"


def test_c_abi_argument_errors_need_no_gpu():
    lib = _lib.load()
    # rejected before any launch: unknown bit order, bad shapes, bad dtype
    assert lib.nq_pack_signs(None, None, 4, 32, 7, None) == _lib.NQ_ERR_INVALID_ARGUMENT
    assert lib.nq_pack_marlin(None, None, 63, 16, None) == _lib.NQ_ERR_SHAPE
    assert lib.nq_gemm_onebit(9, None, None, None, None, None, 1, 16, 64, None, 0, None) == _lib.NQ_ERR_DTYPE
    assert lib.nq_gemm_onebit(0, None, None, None, None, None, 1, 24, 64, None, 0, None) == _lib.NQ_ERR_SHAPE
    assert lib.nq_gemv(0, None, None, None, None, None, None, None, 1, 64, 32, 64, None, 0, None) == \
        _lib.NQ_ERR_INVALID_ARGUMENT
    assert b"null pointer" in lib.nq_last_error_message()
    # empty problems are no-ops
    assert lib.nq_pack_signs(None, None, 0, 32, 0, None) == 0
    assert lib.nq_gemv_workspace_bytes(1, 4096, 1632, 11008) >= 1632 * 4
    # grouped GEMV and decode attention
    items = (_lib.GemvItem * 2)()
    for it in items:
        it.r, it.m, it.y_stride = 1632, 11008, 11008
    assert lib.nq_gemv_group_workspace_bytes(2, items, 1) >= 2 * lib.nq_gemv_workspace_bytes(1, 4096, 1632, 11008) - 256
    assert lib.nq_gemv_group_workspace_bytes(0, items, 1) == 0
    assert lib.nq_gemv_group_workspace_bytes(5, items, 1) == 0
    assert lib.nq_gemv_group_stage2(0, 2, items, 1, 7, None, 0, None) == _lib.NQ_ERR_INVALID_ARGUMENT
    attn = lambda dtype, hd, heads, kv, L: lib.nq_attention_decode(  # noqa: E731
        dtype, None, None, None, heads * hd, None, None, None, None, None, None, 1, heads, kv, hd, L, 1.0, None, 0,
        None)
    assert attn(9, 128, 32, 32, 384) == _lib.NQ_ERR_DTYPE
    assert attn(0, 64, 32, 32, 384) == _lib.NQ_ERR_UNSUPPORTED
    assert attn(0, 128, 24, 8, 384) == _lib.NQ_ERR_UNSUPPORTED  # 3 query heads per kv head
    assert attn(0, 128, 30, 8, 64) == _lib.NQ_ERR_SHAPE
    assert attn(0, 128, 32, 32, 384) == _lib.NQ_ERR_INVALID_ARGUMENT  # null pointers
    # (2 + 128) floats per query head per 64-position chunk
    assert lib.nq_attention_decode_workspace_bytes(1, 32, 32, 128, 384) == 32 * 6 * 130 * 4
    assert lib.nq_attention_decode_workspace_bytes(1, 32, 32, 64, 384) == 0
    # the rotary store of the q/k/v stage 2 and the standalone rotary kernel
    qkv_items = (_lib.GemvItem * 3)()
    for it, m in zip(qkv_items, (4096, 4096, 4096)):
        it.r, it.m, it.y_stride = 1120, m, 12288
    rope2 = lambda hd, L: lib.nq_gemv_group_stage2_rope(  # noqa: E731
        0, qkv_items, 1, None, None, None, None, None, hd, L, None, None, 0, None)
    assert rope2(120, 384) == _lib.NQ_ERR_INVALID_ARGUMENT  # head_dim not a multiple of 16
    assert rope2(128, 0) == _lib.NQ_ERR_INVALID_ARGUMENT
    assert rope2(128, 384) == _lib.NQ_ERR_INVALID_ARGUMENT  # null caches
    qkv_items[2].m = 2048
    assert rope2(128, 384) == _lib.NQ_ERR_SHAPE  # k and v differ
    qkv_items[0].m = 4000
    assert rope2(128, 384) == _lib.NQ_ERR_SHAPE  # q is not whole heads
    rope = lambda dt, hd, stride: lib.nq_rope_kv_write(  # noqa: E731
        dt, None, stride, None, None, None, None, None, None, 32 * hd, 1, 32, 32, hd, 384, None)
    assert rope(9, 128, 96 * 128) == _lib.NQ_ERR_DTYPE
    assert rope(0, 127, 96 * 127) == _lib.NQ_ERR_INVALID_ARGUMENT  # odd head_dim
    assert rope(0, 128, 95 * 128) == _lib.NQ_ERR_SHAPE  # row too short for q, k and v
    assert rope(0, 128, 96 * 128) == _lib.NQ_ERR_INVALID_ARGUMENT  # null pointers
    # the decode step's argmax
    assert lib.nq_argmax_rows(None, 2, 0, 64, None, None) == _lib.NQ_ERR_INVALID_ARGUMENT  # no logits
    assert lib.nq_argmax_rows(None, 2, 64, 64, None, None) == _lib.NQ_ERR_INVALID_ARGUMENT  # null pointers
    assert lib.nq_argmax_rows(None, 0, 64, 64, None, None) == 0  # no rows


# The schema strings of the reference extension (kernel/pybind.cpp:85-104), written out here as
# the concatenation of its C string literals, independently of the package's own constants.
REFERENCE_SCHEMAS = {
    "nanoquant_dyn_forward":
        "nanoquant_dyn_forward(Tensor x, Tensor scale_g, Tensor Ubits, Tensor? scale_l, Tensor Vbits, "
        "Tensor scale_h, int num_thread_stage1=128, int num_thread_stage2=128, int num_row_per_warp_stage1=2, "
        "int num_row_per_warp_stage2=2, int num_acc_stage1=4, int num_acc_stage2=4, int num_pipeline_stage1=2, "
        "int num_pipeline_stage2=2) -> Tensor",
    "marlin_onebit_forward":
        "marlin_onebit_forward(Tensor x, Tensor weight, Tensor? scale_g, Tensor? scale_h, Tensor(a!) workspace) "
        "-> Tensor",
    "marlin_nanoquant_forward":
        "marlin_nanoquant_forward(Tensor x, Tensor weight_u, Tensor weight_v, Tensor? scale_g, Tensor? scale_l, "
        "Tensor? scale_h, Tensor(a!) workspace) -> Tensor",
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_schemas_are_the_reference_schemas(name):
    registered = str(getattr(torch.ops.binary_kernels, name).default._schema)
    want = str(torch._C.parse_schema("binary_kernels::" + REFERENCE_SCHEMAS[name]))
    assert registered == want
    # and the package's constants are those strings
    const = {"nanoquant_dyn_forward": bk.GEMV_SCHEMA, "marlin_onebit_forward": bk.ONEBIT_SCHEMA,
             "marlin_nanoquant_forward": bk.NANOQUANT_SCHEMA}[name]
    assert const == REFERENCE_SCHEMAS[name]


def meta(*shape, dtype=torch.float16):
    return torch.empty(*shape, device="meta", dtype=dtype)


def test_fake_shapes():
    op = torch.ops.binary_kernels
    y = op.nanoquant_dyn_forward(meta(4096), meta(4096), meta(1024, 128, dtype=torch.int32), None,
                                 meta(4096, 32, dtype=torch.int32), meta(4096))
    assert tuple(y.shape) == O.gemv_output_shape((4096,), 4096)
    y = op.nanoquant_dyn_forward(meta(2, 3, 64), meta(64), meta(32, 2, dtype=torch.int32), None,
                                 meta(128, 1, dtype=torch.int32), meta(128))
    assert tuple(y.shape) == (2, 3, 128)
    ws = meta(8 * 32, dtype=torch.int32)
    y = op.marlin_onebit_forward(meta(5, 64), meta(4, 128, dtype=torch.int32), meta(64), meta(256), ws)
    assert tuple(y.shape) == O.marlin_onebit_output_shape((5, 64), (4, 128))
    y = op.marlin_nanoquant_forward(meta(7, 4096), meta(256, 128, dtype=torch.int32), meta(16, 2048, dtype=torch.int32),
                                    meta(4096), meta(256), meta(4096), meta(4096 // 128 * 32, dtype=torch.int32))
    assert tuple(y.shape) == (7, 4096)


def test_fake_checks_follow_the_reference():
    op = torch.ops.binary_kernels
    ws = meta(64, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="k dimension mismatch"):
        op.marlin_onebit_forward(meta(5, 48), meta(4, 128, dtype=torch.int32), None, None, ws)
    with pytest.raises(RuntimeError, match="s_in size mismatch"):
        op.marlin_onebit_forward(meta(5, 64), meta(4, 128, dtype=torch.int32), meta(32), None, ws)
    with pytest.raises(RuntimeError, match="s_out size mismatch"):
        op.marlin_onebit_forward(meta(5, 64), meta(4, 128, dtype=torch.int32), None, meta(128), ws)
    with pytest.raises(RuntimeError, match="workspace too small"):
        op.marlin_onebit_forward(meta(5, 64), meta(4, 128, dtype=torch.int32), None, None, meta(1, dtype=torch.int32))


def test_cpu_tensors_have_no_kernel():
    x = torch.zeros(1, 64, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        torch.ops.binary_kernels.nanoquant_dyn_forward(x, torch.zeros(64, dtype=torch.float16),
                                                       torch.zeros(32, 2, dtype=torch.int32), None,
                                                       torch.zeros(64, 1, dtype=torch.int32),
                                                       torch.zeros(64, dtype=torch.float16))


def test_device_impl_messages_without_a_gpu():
    h = torch.float16
    args = (torch.zeros(1, 64, dtype=h), torch.zeros(64, dtype=h), torch.zeros(32, 2, dtype=torch.int32), None,
            torch.zeros(64, 1, dtype=torch.int32), torch.zeros(64, dtype=h))
    with pytest.raises(RuntimeError, match="^x must be a CUDA tensor$"):
        bk.nanoquant_dyn_forward_cuda(*args)
    with pytest.raises(RuntimeError, match="^Support only Half or BFloat16$"):
        bk.nanoquant_dyn_forward_cuda(torch.zeros(1, 64), *args[1:])


@pytest.mark.parametrize("ints", [(128, 128, 2, 2, 1, 1, 8, 8), (128, 128, 2, 2, 4, 4, 2, 2), (32, 128, 2, 2, 1, 1, 8, 8),
                                  (256, 64, 8, 1, 2, 1, 16, 1), (128, 128, 2, 3, 1, 1, 8, 8), (64, 64, 1, 1, 1, 1, 1, 3)])
def test_tuning_validation_matches_oracle(ints):
    expect = O.check_gemv_tuning(*ints)
    if expect is None:
        bk._check_tuning(*ints)
    else:
        with pytest.raises(ValueError, match=re.escape(expect[1])):
            bk._check_tuning(*ints)


def test_get_kernel_function():
    assert ku.get_kernel_function("nanoquant", torch.float16, "dynamic") is torch.ops.binary_kernels.nanoquant_dyn_forward
    assert ku.get_kernel_function("marlin_nanoquant", torch.float16, "fixed") is \
        torch.ops.binary_kernels.marlin_nanoquant_forward
    with pytest.raises(AttributeError, match="not found"):
        ku.get_kernel_function("nosuch", torch.float16, "fixed")


def test_packer_errors_before_device_work():
    with pytest.raises(TypeError, match="int8"):
        ku.pack_binary_gemv(torch.ones(2, 2, dtype=torch.int32))
    with pytest.raises(ValueError, match="Unsupported method"):
        ku.pack_binary_gemv(torch.ones(2, 2, dtype=torch.int8), method="msb")
    with pytest.raises(ValueError, match="Expected 2D"):
        ku.unpack_binary_gemv(torch.zeros(3, dtype=torch.int32), (1, 3))
    with pytest.raises(ValueError, match="Expected \\(2, 1\\)"):
        ku.unpack_binary_gemv(torch.zeros(2, 2, dtype=torch.int32), (2, 3))
    with pytest.raises(RuntimeError, match="is invalid for input of size"):
        ku.pack_binary_marlin(torch.ones(65, 16, dtype=torch.int8), torch.ones(16), torch.ones(65))
    with pytest.raises(ValueError, match="scale_l"):
        ku.pack_binary_marlin_fused(torch.ones(64, 32, dtype=torch.int8), torch.ones(32, 64, dtype=torch.int8),
                                    torch.ones(64), None, torch.ones(64))


def test_packers_refuse_mixed_devices():
    meta = torch.ones(64, dtype=torch.float16, device="meta")
    with pytest.raises(RuntimeError, match="CPU or CUDA tensors"):
        ku.pack_binary_marlin(torch.ones(64, 64, dtype=torch.int8), meta, torch.ones(64, dtype=torch.float16))


def make_layer(in_f, out_f, rank, seed=0, with_mid=False, bias=False, dtype=torch.float32, device="cpu"):
    torch.manual_seed(seed)
    lin = nn.Linear(in_f, out_f, bias=bias, device=device)
    lin.__class__ = NanoQuantLinear
    lin.init_for_inference(rank, has_scale_mid=with_mid)
    c = O.random_case(seed, out_f, in_f, rank, 1, with_mid=with_mid)
    with torch.no_grad():
        lin.V.copy_(torch.from_numpy(c["V"].astype(np.float32)))
        lin.U.copy_(torch.from_numpy(c["U"].astype(np.float32)))
        lin.scale_pre.copy_(torch.from_numpy(c["s_in"].astype(np.float32))[None])
        lin.scale_post.copy_(torch.from_numpy(c["s_out"].astype(np.float32))[None])
        if with_mid:
            lin.scale_mid.copy_(torch.from_numpy(c["s_mid"].astype(np.float32))[None])
    return lin.to(device=device, dtype=dtype), c


def test_module_dense_path_matches_oracle():
    lin, c = make_layer(64, 96, 32, seed=3, with_mid=True)
    x = torch.from_numpy(np.random.default_rng(0).normal(size=(4, 64)).astype(np.float32))
    lin.dtype = torch.float32
    y = lin(x)
    # the parameters were created in the reference's default bf16, so take the stored values
    f = lambda t: t.detach().double().numpy().reshape(-1)  # noqa: E731
    y64 = O.nanoquant_forward_f64(x.numpy(), f(lin.scale_pre), c["V"], f(lin.scale_mid), c["U"], f(lin.scale_post))
    np.testing.assert_allclose(y.detach().numpy(), y64, rtol=1e-4, atol=1e-3)


def test_module_inference_init_and_gemlite_refusal():
    lin, _ = make_layer(32, 64, 16)
    assert lin.weight is None and tuple(lin.V.shape) == (16, 32) and tuple(lin.U.shape) == (64, 16)
    assert not hasattr(lin, "scale_mid")
    with pytest.raises(NotImplementedError):
        lin._prepare_kernel("gemlite")


def test_package_exports():
    assert nanoquant_amd.binary_packer is ku.pack_binary_gemv
    assert nanoquant_amd.marlin_nanoquant_packer is ku.pack_binary_marlin_fused


def test_gemm_split_workspace_sizes():
    """The GEMM asks for split-K scratch only where its grid is small, and then for one fp32
    plane of the output per k range, each range at least 8 of the 64-k steps."""
    lib = _lib.load()
    # large grids and K % 64 != 0 never split
    assert lib.nq_gemm_onebit_workspace_bytes(2048, 1792, 11008) == 0
    assert lib.nq_gemm_onebit_workspace_bytes(2048, 4096, 1792) == 0
    assert lib.nq_gemm_onebit_workspace_bytes(256, 4096 + 16, 1280) == 0
    assert lib.nq_gemm_onebit_workspace_bytes(0, 4096, 1280) == 0
    # B=256, K=4096 (64 steps, not long), N=1280: 20 tiles of 64 x 256, so the split runs 40 tiles of
    # 32 x 256 -> 256 // 40 = 6 ranges of ceil(64 / 6) = 11 steps, and 6 ranges cover the steps
    assert lib.nq_gemm_onebit_workspace_bytes(256, 4096, 1280) == 6 * 256 * 1280 * 4
    # B=256, K=1792 (28 even steps), N=4096: 64 tiles, 128 of 32 rows -> K over two wave groups, no split
    assert lib.nq_gemm_onebit_workspace_bytes(256, 1792, 4096) == 0
    # B=256, K=11008 (172 steps: long), N=1792: 56 tiles of 32 rows -> 256 // 56 = 4 ranges of
    # ceil(172 / 4) = 43 steps (at most 96: each over four wave groups), and 4 ranges cover the steps
    assert lib.nq_gemm_onebit_workspace_bytes(256, 11008, 1792) == 4 * 256 * 1792 * 4
    # B=256, K=28672 (448 steps), N=3584: 112 tiles of 32 rows -> 2 ranges of 224 steps, too long for
    # the 32-row wave groups; 56 tiles of 64 rows -> 256 // 56 = 4 ranges of 112 steps over four groups
    assert lib.nq_gemm_onebit_workspace_bytes(256, 28672, 3584) == 4 * 256 * 3584 * 4
    # two stages share the workspace: the larger need
    s1 = lib.nq_gemm_onebit_workspace_bytes(256, 11008, 1792)
    s2 = lib.nq_gemm_onebit_workspace_bytes(256, 4096, 1792)  # 28 tiles, 56 of 32 rows: 4 ranges of 16
    assert s2 == 4 * 256 * 1792 * 4
    assert lib.nq_gemm_nanoquant_workspace_bytes(256, 11008, 1792, 4096) == max(s1, 0) > 0
    assert lib.nq_gemm_nanoquant_workspace_bytes(256, 4096, 1792, 11008) == max(s2, 0) > 0


def test_repack_marlin_argument_errors_need_no_gpu():
    lib = _lib.load()
    # padded shape smaller than the matrix, padding not a whole Marlin tile, unknown bit order
    assert lib.nq_repack_marlin(None, 65, 16, 0, None, 64, 16, None) == _lib.NQ_ERR_INVALID_ARGUMENT
    assert lib.nq_repack_marlin(None, 64, 16, 0, None, 96, 16, None) == _lib.NQ_ERR_SHAPE
    assert lib.nq_repack_marlin(None, 64, 16, 0, None, 64, 24, None) == _lib.NQ_ERR_SHAPE
    assert lib.nq_repack_marlin(None, 64, 16, 7, None, 64, 16, None) == _lib.NQ_ERR_INVALID_ARGUMENT
    assert lib.nq_repack_marlin(None, 64, 16, 0, None, 64, 16, None) == _lib.NQ_ERR_INVALID_ARGUMENT  # null dst
    assert lib.nq_repack_marlin(None, 0, 0, 0, None, 0, 0, None) == 0  # empty
    with pytest.raises(RuntimeError, match="must cover"):
        ku.repack_binary_marlin(torch.zeros(64, 1, dtype=torch.int32), (64, 16), (64, 8))
    with pytest.raises(ValueError, match="Expected"):
        ku.repack_binary_marlin(torch.zeros(64, 2, dtype=torch.int32), (64, 16))
