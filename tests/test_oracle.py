"""Pins for the CPU oracle: known answers, reference fixtures, closed forms."""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "marlin_vectors.npz")


# --------------------------------------------------------------------------- A1/A2

@pytest.mark.parametrize("method", ["lsb_first", "half2"])
def test_all_minus_one_and_all_plus_one(method):
    neg = -np.ones((3, 64), dtype=np.int8)
    pos = np.ones((3, 64), dtype=np.int8)
    assert (O.pack_binary_gemv(neg, method) == 0xFFFFFFFF).all()
    assert (O.pack_binary_gemv(pos, method) == 0).all()


def test_lsb_first_one_hot():
    for j in range(32):
        s = np.ones((1, 32), dtype=np.int8)
        s[0, j] = -1
        assert int(O.pack_binary_gemv(s, "lsb_first")[0, 0]) == 1 << j


def test_half2_known_answers():
    expect = {0: 0x00008000, 1: 0x80000000, 2: 0x00004000, 3: 0x40000000, 30: 0x00000001, 31: 0x00010000}
    for j, word in expect.items():
        s = np.ones((1, 32), dtype=np.int8)
        s[0, j] = -1
        assert int(O.pack_binary_gemv(s, "half2")[0, 0]) == word


@pytest.mark.parametrize("c", [1, 5, 17, 31])
def test_tail_word_padding_is_plus_one(c):
    s = -np.ones((2, 32 + c), dtype=np.int8)
    w = O.pack_binary_gemv(s, "lsb_first")
    assert w.shape == (2, 2)
    assert int(w[0, 1]) == (1 << c) - 1


def test_reference_partial_word_round_trip():
    # tests/test_shaman_transfer.py:239-260: U [7,3] and V [3,5] for Linear(5,7) at
    # rank 3, and the reverse layer; packed words = rows * ceil(cols/32).
    rng = np.random.default_rng(0)
    for shape in [(7, 3), (3, 5), (5, 3), (3, 7)]:
        s = np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8)
        for method in ("lsb_first", "half2"):
            p = O.pack_binary_gemv(s, method)
            assert p.shape == (shape[0], (shape[1] + 31) // 32)
            assert (O.unpack_binary_gemv(p, shape, method) == s).all()
    # packed_bits(block[0], 3) == 32*(3+7) + 16*(5+7): 3 V words + 7 U words + fp16 scales
    words = O.pack_binary_gemv(np.ones((3, 5), np.int8)).size + O.pack_binary_gemv(np.ones((7, 3), np.int8)).size
    assert 32 * words + 16 * (5 + 7) == 32 * (3 + 7) + 16 * (5 + 7)


def test_reference_row_padding_word_counts():
    # tests/test_reconstruction_efficiency.py:161-172: a 4 -> 8 layer at r=2 has
    # V [2,4] -> 2 words and U [8,2] -> 8 words; checkpoint_audit.py:33-35 shape rule.
    assert O.pack_binary_gemv(np.ones((2, 4), np.int8)).shape == (2, 1)
    assert O.pack_binary_gemv(np.ones((8, 2), np.int8)).shape == (8, 1)
    for rows, cols in [(1, 1), (4, 32), (4, 33), (9, 100)]:
        assert O.pack_binary_gemv(np.ones((rows, cols), np.int8)).shape == (rows, (cols + 31) // 32)


def test_half2_matches_reference_kernel_sign_extraction():
    rng = np.random.default_rng(1)
    s = np.where(rng.random((16, 32)) < 0.5, -1, 1).astype(np.int8)
    words = O.pack_binary_gemv(s, "half2")
    for r in range(16):
        for j in range(32):
            assert O.gemv_kernel_sign(int(words[r, 0]), j) == s[r, j]


def test_pack_errors():
    with pytest.raises(TypeError):
        O.pack_binary_gemv(np.ones((2, 2), np.int32))
    with pytest.raises(ValueError):
        O.pack_binary_gemv(np.ones((2, 2), np.int8), "msb")
    with pytest.raises(ValueError):
        O.unpack_binary_gemv(np.zeros(3, np.uint32), (1, 3))
    with pytest.raises(ValueError):
        O.unpack_binary_gemv(np.zeros((2, 2), np.uint32), (2, 3))


# --------------------------------------------------------------------------- A3/A4

def _golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_marlin_single_matches_reference_vectors():
    g = _golden()
    for i in range(int(g["n_single"])):
        words, s_in, s_out, ws = O.pack_binary_marlin(g[f"single{i}_w"], g[f"single{i}_s_in"], g[f"single{i}_s_out"])
        assert (words == g[f"single{i}_words"]).all(), i
        assert (s_in.view(np.uint16) == g[f"single{i}_s_in_p"].view(np.uint16)).all(), i
        assert (s_out.view(np.uint16) == g[f"single{i}_s_out_p"].view(np.uint16)).all(), i
        assert ws == int(g[f"single{i}_ws"]), i
        O_, K_ = g[f"single{i}_w"].shape
        assert (O.unpack_binary_marlin(words, O_, K_) == g[f"single{i}_w"]).all()


def test_marlin_torch_eager_packer_matches_reference_vectors():
    import torch
    g = _golden()
    for i in range(int(g["n_single"])):
        words = O.pack_marlin_torch(torch.from_numpy(g[f"single{i}_w"].astype(np.int8)))
        assert (words.numpy().view(np.uint32) == g[f"single{i}_words"].view(np.uint32)).all(), i


def test_marlin_fused_matches_reference_vectors():
    g = _golden()
    for i in range(int(g["n_fused"])):
        res = O.pack_binary_marlin_fused(g[f"fused{i}_V_sign"], g[f"fused{i}_U_sign"], g[f"fused{i}_s_g"],
                                         g[f"fused{i}_s_l"], g[f"fused{i}_s_h"])
        names = ["V_bits", "U_bits", "s_g_p", "s_l_p", "s_h_p", "workspace"]
        for name, got in zip(names, res):
            exp = g[f"fused{i}_{name}"]
            assert got.shape == exp.shape, (i, name)
            if got.dtype == np.float16:
                assert (got.view(np.uint16) == exp.view(np.uint16)).all(), (i, name)
            else:
                assert (got.astype(np.int64) == exp.astype(np.int64)).all(), (i, name)


def test_marlin_bit_map_is_a_bijection():
    O_, K_ = 128, 64
    row, col, bit = O.marlin_bit_map(O_, K_)
    key = (row.astype(np.int64) * (O_ // 2) + col) * 32 + bit
    assert np.unique(key).size == O_ * K_ and key.min() == 0 and key.max() == O_ * K_ - 1


def test_planted_marlin_mistake_is_caught(monkeypatch):
    # Swap the two roles of the permutation in the oracle: the golden check must fail.
    g = _golden()
    monkeypatch.setattr(O.nq_oracle, "marlin_perm_in", lambda K: np.arange(K))
    _, s_in, _, _ = O.nq_oracle.pack_binary_marlin(g["single1_w"], g["single1_s_in"], g["single1_s_out"])
    assert not (s_in.view(np.uint16) == g["single1_s_in_p"].view(np.uint16)).all()


def test_planted_half2_mistake_is_caught(monkeypatch):
    bad = np.array([15 - j // 2 + 16 * ((j + 1) % 2) for j in range(32)], dtype=np.int64)
    monkeypatch.setattr(O.nq_oracle, "HALF2_BIT", bad)
    s = np.ones((1, 32), dtype=np.int8)
    s[0, 0] = -1
    assert int(O.nq_oracle.pack_binary_gemv(s, "half2")[0, 0]) != 0x00008000


# --------------------------------------------------------------------------- forward

def test_forward_all_plus_one_closed_form():
    rng = np.random.default_rng(2)
    n, r, m = 40, 8, 24
    x = rng.normal(size=(3, n))
    s_in, s_mid, s_out = rng.random(n) + 0.5, rng.random(r) + 0.5, rng.random(m) + 0.5
    y = O.nanoquant_forward_f64(x, s_in, np.ones((r, n)), s_mid, np.ones((m, r)), s_out)
    exp = s_out[None, :] * (s_mid.sum() * (x * s_in).sum(axis=1))[:, None]
    np.testing.assert_allclose(y, exp, rtol=1e-12)


def test_forward_one_hot_selects_sign_column():
    rng = np.random.default_rng(3)
    n, r, m = 32, 16, 8
    V = np.where(rng.random((r, n)) < 0.5, -1, 1)
    U = np.where(rng.random((m, r)) < 0.5, -1, 1)
    k = 11
    x = np.zeros((1, n))
    x[0, k] = 1.0
    y = O.nanoquant_forward_f64(x, np.ones(n), V, None, U, np.ones(m))
    np.testing.assert_array_equal(y[0], U @ V[:, k])


def test_forward_brute_force():
    rng = np.random.default_rng(4)
    B, n, r, m = 2, 6, 4, 5
    c = O.random_case(5, m, n, r, B, with_mid=True)
    y = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], c["s_mid"], c["U"], c["s_out"])
    for b in range(B):
        for i in range(m):
            acc = 0.0
            for j in range(r):
                h = sum(float(c["V"][j, k]) * float(c["s_in"][k]) * float(c["x"][b, k]) for k in range(n))
                acc += float(c["U"][i, j]) * h * float(c["s_mid"][j])
            assert abs(acc * float(c["s_out"][i]) - y[b, i]) <= 1e-12 * max(1.0, abs(y[b, i]))


def test_marlin_f64_identity_rounding_is_the_forward():
    c = O.random_case(7, 40, 64, 24, 3, with_mid=True)
    args = (c["x"], c["s_in"], c["V"], c["s_mid"], c["U"], c["s_out"])
    np.testing.assert_array_equal(O.marlin_nanoquant_f64(*args, round_imm=lambda h: h), O.nanoquant_forward_f64(*args))


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_marlin_f64_rounds_the_intermediate(kind):
    # one input column, all +1 signs: h_j = s_in[0] * x[0] = 1 + 2^-12 for every j, which neither
    # type holds; the nearest value of both is 1.0, so y = s_out * r exactly
    import torch
    rnd = (lambda h: h.astype(np.float16).astype(np.float64)) if kind == "f16" else \
        (lambda h: torch.from_numpy(h.astype(np.float32)).to(torch.bfloat16).double().numpy())
    n, r, m = 1, 6, 5
    x = np.array([[1.0 + 2.0 ** -12]])
    y = O.marlin_nanoquant_f64(x, np.ones(n), np.ones((r, n)), None, np.ones((m, r)), np.full(m, 0.5), round_imm=rnd)
    np.testing.assert_array_equal(y, np.full((1, m), 0.5 * r))
    # and 1 + 2^-6 survives both roundings (8 significant bits suffice)
    y = O.marlin_nanoquant_f64(np.array([[1.0 + 2.0 ** -6]]), np.ones(n), np.ones((r, n)), None, np.ones((m, r)),
                               np.ones(m), round_imm=rnd)
    np.testing.assert_array_equal(y, np.full((1, m), r * (1.0 + 2.0 ** -6)))


def test_marlin_f64_clamps_the_fp16_intermediate():
    # h = 70000 is past the fp16 bound; the first product saturates it to 65504 before stage 2
    y = O.marlin_nanoquant_f64(np.array([[70000.0]]), np.ones(1), np.ones((2, 1)), None, np.ones((3, 2)), np.ones(3),
                               round_imm=lambda h: h, sat_imm=65504.0)
    np.testing.assert_array_equal(y, np.full((1, 3), 2 * 65504.0))


def test_torch_dense_path_matches_f64():
    import torch
    c = O.random_case(6, 48, 64, 32, 2)
    y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], None, c["U"], c["s_out"])
    t = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float32))  # noqa: E731
    y = O.compute_forward_torch(t(c["x"]), t(c["V"]), t(c["U"]), t(c["s_in"]), None, t(c["s_out"]))
    np.testing.assert_allclose(y.numpy(), y64, rtol=1e-4, atol=1e-3)


def test_tuning_rules():
    assert O.check_gemv_tuning(128, 128, 2, 2, 1, 1, 8, 8) is None
    name, msg = O.check_gemv_tuning(128, 128, 2, 2, 4, 4, 2, 2)
    assert name == "n_acc1" and msg == "n_acc1 should be one of [1, 2], but 4 was given"
    assert O.check_gemv_tuning(32, 128, 2, 2, 1, 1, 8, 8)[0] == "n_th1"
    assert O.check_gemv_tuning(128, 128, 2, 3, 1, 1, 8, 8)[0] == "n_rpw2"


@pytest.mark.parametrize("method", ["lsb_first", "half2"])
@pytest.mark.parametrize("shape", [(1, 1), (5, 33), (17, 100), (64, 4096)])
def test_torch_eager_packers_match_the_numpy_oracle(method, shape):
    """The eager-torch packers (the CPU baseline of packing) give the pinned numpy oracle's words,
    including bit 31 (int32 wraparound) and the +1 padding of a partial word."""
    import torch
    rng = np.random.default_rng(shape[0] * 131 + shape[1])
    s = np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8)
    s[0, :min(32, shape[1])] = -1  # a word (or its valid part) of all -1, bit 31 set
    words = O.pack_signs_torch(torch.from_numpy(s), method)
    assert words.dtype == torch.int32
    np.testing.assert_array_equal(words.numpy().view(np.uint32), O.pack_binary_gemv(s, method))
    back = O.unpack_signs_torch(words, shape, method)
    np.testing.assert_array_equal(back.numpy(), s)
