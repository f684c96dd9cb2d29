"""The packers on CPU tensors (no GPU): the product's host path (nanoquant_amd/kernel/_host.py)
against the oracle's known-answer-pinned packers and against vectors the reference's own Marlin
packer wrote, bit for bit, and a NanoQuantLinear's packed state dict written and read on a host
where no GPU and no HIP library are reachable."""
import os

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle as O
from nanoquant_amd import _lib
from nanoquant_amd.kernel import utils as ku
from nanoquant_amd.modules.linear import NanoQuantLinear

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "marlin_vectors.npz")
# 0 rows, single bits, partial words, the 4096-row chunk boundary of the host path
SHAPES = [(0, 5), (1, 1), (3, 31), (7, 32), (5, 33), (2, 95), (4100, 40), (17, 1000)]


def signs(shape, seed):
    return np.where(np.random.default_rng(seed).random(shape) < 0.5, -1, 1).astype(np.int8)


def words_of(t):
    return t.numpy().view(np.uint32)


@pytest.fixture
def no_gpu(monkeypatch):
    """CUDA unavailable and the HIP library unloadable: any GPU route would raise."""
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)

    def refuse():
        raise ImportError("the HIP library is not reachable on this host")
    monkeypatch.setattr(_lib, "load", refuse)


@pytest.mark.parametrize("method", ["lsb_first", "half2"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_sign_pack_unpack_repack(no_gpu, method, shape):
    s = signs(shape, shape[0] * 131 + shape[1])
    w = ku.pack_binary_gemv(torch.from_numpy(s), method=method)
    assert w.dtype == torch.int32 and w.device.type == "cpu"
    np.testing.assert_array_equal(words_of(w), O.pack_binary_gemv(s, method))
    back = ku.unpack_binary_gemv(w, shape, method=method)
    assert back.dtype == torch.int8
    np.testing.assert_array_equal(back.numpy(), s)
    other = "half2" if method == "lsb_first" else "lsb_first"
    re_ = ku.repack_binary_gemv(w, shape, src_method=method, dst_method=other)
    np.testing.assert_array_equal(words_of(re_), O.pack_binary_gemv(s, other))


def test_sign_pack_treats_negative_values_as_minus_one(no_gpu):
    v = torch.tensor([[-7, 0, 3, -1, 1, -128]], dtype=torch.int8)
    np.testing.assert_array_equal(words_of(ku.pack_binary_gemv(v)), np.array([[0b101001]], np.uint32))


def test_repack_clears_set_padding_bits(no_gpu):
    # words whose bits past the last column are set (not what a packer writes): the repacked words
    # are those of the signs alone
    w = torch.from_numpy(np.array([[-1]], dtype=np.int32))
    got = ku.repack_binary_gemv(w, (1, 5), "lsb_first", "half2")
    np.testing.assert_array_equal(words_of(got), O.pack_binary_gemv(-np.ones((1, 5), np.int8), "half2"))


def test_marlin_single_matches_reference_vectors(no_gpu):
    g = np.load(GOLDEN, allow_pickle=False)
    for i in range(int(g["n_single"])):
        t = lambda k: torch.from_numpy(np.ascontiguousarray(g[f"single{i}_{k}"]))  # noqa: E731
        words, s_in, s_out, ws = ku.pack_binary_marlin(t("w"), t("s_in"), t("s_out"))
        np.testing.assert_array_equal(words_of(words), g[f"single{i}_words"].view(np.uint32))
        np.testing.assert_array_equal(s_in.numpy().view(np.uint16), g[f"single{i}_s_in_p"].view(np.uint16))
        np.testing.assert_array_equal(s_out.numpy().view(np.uint16), g[f"single{i}_s_out_p"].view(np.uint16))
        assert ws == int(g[f"single{i}_ws"])


def test_marlin_fused_matches_reference_vectors(no_gpu):
    g = np.load(GOLDEN, allow_pickle=False)
    names = ["V_bits", "U_bits", "s_g_p", "s_l_p", "s_h_p", "workspace"]
    for i in range(int(g["n_fused"])):
        t = lambda k: torch.from_numpy(np.ascontiguousarray(g[f"fused{i}_{k}"]))  # noqa: E731
        res = ku.pack_binary_marlin_fused(t("V_sign"), t("U_sign"), t("s_g"), t("s_l"), t("s_h"))
        for name, got in zip(names, res):
            exp = g[f"fused{i}_{name}"]
            got = got.numpy()
            assert got.shape == exp.shape, (i, name)
            assert (got.view(np.uint16 if got.dtype == np.float16 else np.uint32) ==
                    exp.view(np.uint16 if exp.dtype == np.float16 else np.uint32)).all(), (i, name)


@pytest.mark.parametrize("method", ["lsb_first", "half2"])
def test_marlin_from_packed_matches_dense_route(no_gpu, method):
    r, n, m = 96, 96, 128  # rank padded to 256
    rng = np.random.default_rng(4)
    V, U = signs((r, n), 1), signs((m, r), 2)
    s_g = torch.from_numpy(np.abs(rng.normal(1, .2, n)).astype(np.float16))
    s_l = torch.from_numpy(np.abs(rng.normal(1, .2, r)).astype(np.float16))
    s_h = torch.from_numpy(np.abs(rng.normal(1, .2, m)).astype(np.float16))
    dense = ku.pack_binary_marlin_fused(torch.from_numpy(V.T.copy()), torch.from_numpy(U.T.copy()), s_g, s_l, s_h)
    Vp = ku.pack_binary_gemv(torch.from_numpy(V), method=method)
    Up = ku.pack_binary_gemv(torch.from_numpy(U), method=method)
    packed = ku.pack_binary_marlin_fused_from_packed(Vp, (r, n), Up, (m, r), s_g, s_l, s_h, src_method=method)
    for a, b in zip(dense, packed):
        assert a.dtype == b.dtype and a.shape == b.shape and a.device.type == b.device.type == "cpu"
        assert torch.equal(a, b)


def make_layer(in_f, out_f, rank, seed):
    torch.manual_seed(seed)
    lin = nn.Linear(in_f, out_f, bias=False)
    lin.__class__ = NanoQuantLinear
    lin.init_for_inference(rank, has_scale_mid=True)
    with torch.no_grad():
        lin.V.copy_(torch.from_numpy(signs((rank, in_f), seed).astype(np.float32)))
        lin.U.copy_(torch.from_numpy(signs((out_f, rank), seed + 1).astype(np.float32)))
    return lin


def test_module_packed_state_dict_round_trip_without_a_gpu(no_gpu):
    src = make_layer(100, 70, 40, seed=5)
    sd = src.state_dict()
    assert "V_packed" in sd and "U_packed" in sd and "V" not in sd and "U" not in sd
    np.testing.assert_array_equal(words_of(sd["V_packed"]), O.pack_binary_gemv(src.V.detach().to(torch.int8)
                                                                                .numpy(), "lsb_first"))
    dst = make_layer(100, 70, 40, seed=9)
    dst.load_state_dict(sd)
    assert torch.equal(dst.V, src.V) and torch.equal(dst.U, src.U)
