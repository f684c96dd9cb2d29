"""Parity of the HIP path with the CPU oracle on the same seeded inputs (needs a gfx950 GPU).

Bars (written here, checked per case):
* packing, unpacking, reordering: bit-exact;
* GEMV / GEMM outputs: max|y - y*| / max|y*| <= 1e-3 against the float64 oracle computed
  from the same fp16/bf16 inputs. For bf16 outputs, whose own rounding is up to 2^-9
  relative, each element's error is counted beyond half a bf16 unit in the last place of
  y*; the bf16 GEMM is compared with the oracle of its algorithm, whose intermediate is a
  bf16 tensor (gemm.cpp:112-122). Outputs the oracle puts beyond the fp16 saturation
  bound are excluded from the ratio and must equal the bound.
"""
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O
from nanoquant_amd.kernel import utils as ku

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "marlin_vectors.npz")
TOL = {("gemv", torch.float16): 1e-3, ("gemv", torch.bfloat16): 1e-3,
       ("gemm", torch.float16): 1e-3, ("gemm", torch.bfloat16): 1e-3}
SIGNIFICANT_BITS = {torch.float16: 11, torch.bfloat16: 8}
SAT = {("gemv", torch.float16): 64504.0, ("gemm", torch.float16): 65504.0}
NP_DTYPE = {torch.float16: np.float16}


def announce(*what):
    print("\n[case]", *what, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def nq():
    import nanoquant_amd
    from nanoquant_amd import _lib
    _lib.load()  # fail loudly when the HIP library is missing
    return nanoquant_amd


def dev_t(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def as_words(t):
    return t.cpu().numpy().view(np.uint32)


def rel_err(y, y64, kind, dtype):
    y = y.float().cpu().numpy().astype(np.float64)
    sat = SAT.get((kind, dtype))
    mask = np.ones_like(y64, dtype=bool) if sat is None else np.abs(y64) < sat
    if sat is not None and (~mask).any():
        # the clamp bound, stored in the output type (fp16(64504) == 64512, as in the reference)
        stored = float(np.float16(sat))
        assert np.all(np.abs(y[~mask]) == stored), "saturated outputs must sit at the bound"
    denom = np.abs(y64[mask]).max()
    diff = np.abs(y[mask] - y64[mask])
    if dtype == torch.bfloat16:
        diff = np.maximum(diff - half_ulp(y64[mask], dtype), 0.0)
    return float(diff.max() / denom), int((~mask).sum())


def half_ulp(v, dtype):
    """Half a unit in the last place of |v| in `dtype`: the output's own rounding error bound."""
    _, e = np.frexp(np.abs(v))  # |v| = f * 2^e, f in [0.5, 1)
    return np.ldexp(1.0, e - 1 - SIGNIFICANT_BITS[dtype])


def round_bf16(h):
    return torch.from_numpy(np.asarray(h, dtype=np.float32)).to(torch.bfloat16).double().numpy()


# --------------------------------------------------------------------------- packing

# (5, 3200): 500 whole words, so the last 256-word block of the word kernels is partly empty
PACK_SHAPES = [(1, 1), (3, 5), (7, 3), (4, 32), (5, 33), (17, 100), (5, 3200), (64, 4096), (1632, 4096),
               (11008, 1632)]


@pytest.mark.parametrize("method", ["lsb_first", "half2"])
@pytest.mark.parametrize("shape", PACK_SHAPES)
def test_pack_unpack_bit_exact(nq, shape, method):
    announce("pack", shape, method)
    rng = np.random.default_rng(hash(shape) % 1000)
    s = np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8)
    words = nq.pack_binary_gemv(dev_t(s), method=method)
    torch.cuda.synchronize()
    assert words.dtype == torch.int32 and tuple(words.shape) == (shape[0], (shape[1] + 31) // 32)
    np.testing.assert_array_equal(as_words(words), O.pack_binary_gemv(s, method))
    back = nq.unpack_binary_gemv(words, shape, method=method)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(back.cpu().numpy(), s)


@pytest.mark.parametrize("shape", [(3, 5), (17, 100), (5, 3200), (1632, 4096), (4096, 1632)])
def test_repack_between_orders(nq, shape):
    announce("repack", shape)
    rng = np.random.default_rng(7)
    s = np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8)
    lsb = dev_t(O.pack_binary_gemv(s, "lsb_first").view(np.int32))
    h2 = nq.repack_binary_gemv(lsb, shape, "lsb_first", "half2")
    np.testing.assert_array_equal(as_words(h2), O.pack_binary_gemv(s, "half2"))
    back = nq.repack_binary_gemv(h2, shape, "half2", "lsb_first")
    np.testing.assert_array_equal(as_words(back), O.pack_binary_gemv(s, "lsb_first"))


def test_marlin_packers_match_reference_vectors(nq):
    g = np.load(GOLDEN, allow_pickle=False)
    for i in range(int(g["n_single"])):
        announce("marlin single", i, g[f"single{i}_w"].shape)
        w, s_in_p, s_out_p, ws = nq.pack_binary_marlin(dev_t(g[f"single{i}_w"]), dev_t(g[f"single{i}_s_in"]),
                                                       dev_t(g[f"single{i}_s_out"]))
        np.testing.assert_array_equal(as_words(w), g[f"single{i}_words"])
        np.testing.assert_array_equal(s_in_p.cpu().numpy().view(np.uint16), g[f"single{i}_s_in_p"].view(np.uint16))
        np.testing.assert_array_equal(s_out_p.cpu().numpy().view(np.uint16), g[f"single{i}_s_out_p"].view(np.uint16))
        assert ws == int(g[f"single{i}_ws"])
    names = ["V_bits", "U_bits", "s_g_p", "s_l_p", "s_h_p", "workspace"]
    for i in range(int(g["n_fused"])):
        announce("marlin fused", i)
        res = nq.pack_binary_marlin_fused(dev_t(g[f"fused{i}_V_sign"]), dev_t(g[f"fused{i}_U_sign"]),
                                          dev_t(g[f"fused{i}_s_g"]), dev_t(g[f"fused{i}_s_l"]),
                                          dev_t(g[f"fused{i}_s_h"]))
        for name, got in zip(names, res):
            exp = g[f"fused{i}_{name}"]
            a = got.cpu().numpy()
            if a.dtype == np.float16:
                np.testing.assert_array_equal(a.view(np.uint16), exp.view(np.uint16), err_msg=name)
            else:
                np.testing.assert_array_equal(a.view(np.uint32) if name.endswith("bits") else a, exp, err_msg=name)


@pytest.mark.parametrize("OK", [(64, 16), (4096, 1024), (11008, 1792), (1792, 4096)])
def test_marlin_pack_large_and_unpack(nq, OK):
    from nanoquant_amd import _lib
    O_, K_ = OK
    announce("marlin pack", OK)
    rng = np.random.default_rng(O_ + K_)
    w = np.where(rng.random((O_, K_)) < 0.5, -1, 1).astype(np.int8)
    words, _, _, _ = nq.pack_binary_marlin(dev_t(w), torch.ones(K_, dtype=torch.float16, device="cuda"),
                                           torch.ones(O_, dtype=torch.float16, device="cuda"))
    exp, _, _, _ = O.pack_binary_marlin(w, np.ones(K_, np.float16), np.ones(O_, np.float16))
    np.testing.assert_array_equal(as_words(words), exp)
    back = torch.empty((O_, K_), dtype=torch.int8, device="cuda")
    lib = _lib.load()
    _lib.check(lib.nq_unpack_marlin(words.data_ptr(), back.data_ptr(), O_, K_, _lib.stream_of(back.device)), "unpack")
    np.testing.assert_array_equal(back.cpu().numpy(), w)


def test_marlin_pack_from_unaligned_weights(nq):
    """Weights 16-byte aligned take the tiled packer (blocks of 64 outputs x 256 k, the last k tile
    partial here), weights only 2-byte aligned the one-thread-per-word packer: the same words, and
    the oracle's."""
    O_, K_ = 1792, 1104  # 1104 = 4 * 256 + 80
    announce("marlin pack unaligned", O_, K_)
    rng = np.random.default_rng(77)
    w = np.where(rng.random((O_, K_)) < 0.5, -1, 1).astype(np.int8)
    buf = torch.zeros(O_ * K_ + 16, dtype=torch.int8, device="cuda")
    view = buf[2:2 + O_ * K_].view(O_, K_)
    view.copy_(dev_t(w))
    assert view.data_ptr() % 16 == 2
    ones_k = torch.ones(K_, dtype=torch.float16, device="cuda")
    ones_o = torch.ones(O_, dtype=torch.float16, device="cuda")
    words_u, _, _, _ = nq.pack_binary_marlin(view, ones_k, ones_o)
    aligned_w = dev_t(w)
    assert aligned_w.data_ptr() % 16 == 0
    words_a, _, _, _ = nq.pack_binary_marlin(aligned_w, ones_k, ones_o)
    torch.cuda.synchronize()
    assert torch.equal(words_u, words_a)
    exp, _, _, _ = O.pack_binary_marlin(w, np.ones(K_, np.float16), np.ones(O_, np.float16))
    np.testing.assert_array_equal(as_words(words_a), exp)


@pytest.mark.parametrize("shape", [(1, 1), (33, 95), (300, 1000), (1632, 11008)])
def test_host_and_hip_packers_write_the_same_words(nq, shape):
    """The same signs packed as a CPU tensor (host path) and as a CUDA tensor (HIP kernels): sign
    words in both orders, their unpacking and reordering, and the Marlin words and scales of the
    factor padded to whole tiles, bit for bit."""
    rows, cols = shape
    announce("host vs HIP packers", shape)
    rng = np.random.default_rng(rows + cols)
    s = torch.from_numpy(np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8))
    for method in ("lsb_first", "half2"):
        w_host = nq.pack_binary_gemv(s, method=method)
        w_dev = nq.pack_binary_gemv(s.cuda(), method=method)
        assert w_host.device.type == "cpu" and w_dev.is_cuda
        assert torch.equal(w_host, w_dev.cpu()), method
        assert torch.equal(nq.unpack_binary_gemv(w_host, shape, method=method),
                           nq.unpack_binary_gemv(w_dev, shape, method=method).cpu())
        other = "half2" if method == "lsb_first" else "lsb_first"
        assert torch.equal(ku.repack_binary_gemv(w_host, shape, method, other),
                           ku.repack_binary_gemv(w_dev, shape, method, other).cpu())
    O_, K_ = -(-rows // 64) * 64, -(-cols // 16) * 16
    w = torch.ones(O_, K_, dtype=torch.int8)
    w[:rows, :cols] = s
    s_in = torch.from_numpy(np.abs(rng.normal(1, .2, K_)).astype(np.float16))
    s_out = torch.from_numpy(np.abs(rng.normal(1, .2, O_)).astype(np.float16))
    host = nq.pack_binary_marlin(w, s_in, s_out)
    dev = nq.pack_binary_marlin(w.cuda(), s_in.cuda(), s_out.cuda())
    for a, b in zip(host[:3], dev[:3]):
        assert torch.equal(a, b.cpu())
    lsb = nq.pack_binary_gemv(s, method="lsb_first")
    assert torch.equal(ku.repack_binary_marlin(lsb, shape, (O_, K_)),
                       ku.repack_binary_marlin(lsb.cuda(), shape, (O_, K_)).cpu())


# --------------------------------------------------------------------------- GEMV

GEMV_CASES = [
    # name, m, n, r, batch, with_mid
    ("cfg1", 4096, 4096, 1024, 1, False),
    ("tails", 72, 40, 24, 3, True),
    ("odd", 130, 200, 70, 5, False),
    ("wide_batch", 96, 64, 64, 19, True),
    ("llama7b_qkvo_055", 4096, 4096, 1120, 1, False),
    ("llama7b_gate_055_b1", 11008, 4096, 1632, 1, False),
    ("llama7b_gate_055_b4", 11008, 4096, 1632, 4, False),
    ("llama7b_down_055_b16", 4096, 11008, 1632, 16, False),
    ("llama7b_gate_10_b1", 11008, 4096, 2976, 1, False),
    # the VALU stage 1 on wide rows: three words per lane over two waves (n = 11008; n = 10000
    # ends in a half-filled word), two words over two waves at n = 8192; four rows per group
    ("llama7b_down_055_b1", 4096, 11008, 1632, 1, False),
    ("ragged_word_10000_b1", 300, 10000, 100, 1, True),
    ("wide_8192_b2", 600, 8192, 200, 2, True),
    # a stage-2 grid of 1283 blocks of 16 rows (more than one round of resident blocks), the last
    # one ragged: 20520 = 1282 * 16 + 8
    ("tall_ragged_b1", 20520, 256, 96, 1, False),
    # 688 row tiles x two passes of 8 batch rows, with s_mid
    ("tall_b16_mid", 11008, 512, 64, 16, True),
    # batches between the kernels' crossovers: the MFMA stage 1 on 4 .. 33 rows of narrow inputs,
    # n = 1000 (not whole words), ragged ranks and rows
    ("b4_tails", 300, 256, 70, 4, True),
    ("b7_ragged", 1000, 512, 200, 7, True),
    ("b33", 4100, 1024, 300, 33, False),
    ("b32_n1000", 500, 1000, 96, 32, False),
    # the batched stage 1 (k split over blocks, then a finishing launch that adds the ranges in
    # order) runs on rows of 256 words or more: from 16 batch rows, from 8 on rows of 320 words or
    # more, from 3 on rows of 512, from 2 on rows of 513-1024 (whose one-row case runs the VALU
    # kernel with four words per lane over four waves), from 1 on longer rows; a ragged rank and
    # batch, one k range or several, 1, 2, 5 and 7 batch tiles. Narrower rows (64 words) at 64
    # and 100 rows, and each threshold's batch just below it, run the MFMA or VALU stage 1.
    ("sb_b100", 2048, 2048, 512, 100, True),
    ("sb_b64_r200", 1000, 2048, 200, 64, True),
    ("sb_b70_wide", 600, 8192, 500, 70, True),
    ("sb_b20_wide_ragged", 700, 9216, 333, 20, False),
    ("sb_b3_n16384", 500, 16384, 300, 3, True),
    ("sb_b5_n20000_ragged", 300, 20000, 333, 5, False),
    ("sb_b8_n11008", 1000, 11008, 200, 8, True),
    ("s1m_b7_n11008", 600, 11008, 150, 7, False),
    ("s1m_b12_n8192", 500, 8192, 2048, 12, True),
    ("sb_b8_n8192_small_v", 1024, 8192, 448, 8, False),
    ("s1w_b4_n8192_small_v", 1024, 8192, 512, 4, True),
    ("s1m_b4_n8192", 600, 8192, 2600, 4, False),
    ("s1w_b3_n8192_r2400", 500, 8192, 2400, 3, True),
    ("s1w_b1_n20000", 300, 20000, 333, 1, True),
    ("s1w_b1_n32768", 700, 32768, 500, 1, False),
    ("sb_b1_n40000", 200, 40000, 96, 1, True),
    ("sb_b2_n28672", 1000, 28672, 160, 2, False),
    ("s1w_b2_n16384", 400, 16384, 200, 2, False),
    ("llama7b_gate_055_b64", 11008, 4096, 1632, 64, False),
    ("llama7b_down_055_b64", 4096, 11008, 1632, 64, True),
    ("llama7b_gate_055_b128", 11008, 4096, 1632, 128, False),
    # the batched stage 2 (U decoded once per 32 k for all of a block's batch rows, the intermediate
    # streamed through LDS): each of its four launch shapes with ragged rows, batch rows and ranks;
    # m = 4102 takes 2-byte stores, r = 2048 rows of 64 words
    ("s2b_ragged_b37", 5000, 512, 333, 37, True),
    ("s2b_ragged_b90", 9000, 256, 1000, 90, False),
    ("s2b_m4102_b128", 4102, 256, 2048, 128, False),
    ("s2b_tall_b16", 10400, 256, 96, 16, True),
    # the MFMA stage 1 with two and four row tiles per block (chosen to keep its grid to one round
    # of blocks): ragged ranks and batch rows
    ("s1m_rt2_ragged", 300, 512, 700, 120, True),
    ("s1m_rt4_ragged", 700, 1024, 1050, 128, True),
    # the batched stage 2 below 16 rows: a large U (2M words or more) whose rank leaves s2t_kernel two
    # batch rows per pass
    ("s2b_few_rows_big_u", 16400, 256, 4224, 3, False),
    # the MFMA stage 1 on rows of 256+ words, whose tile of V is padded to an odd stride in LDS:
    # an even word count (padded) and an odd one (already odd)
    ("s1m_wide_even_b5", 300, 8192, 160, 5, True),
    ("s1m_wide_odd_b5", 300, 8224, 160, 5, True),
    # 1024-word rows (n = 32737 .. 32768) where the k-split stage 1 does not run (more than 128
    # batch rows; n % 32 != 0): the MFMA kernel with the unpadded stride (the padded one would not
    # fit its staging buffer)
    ("s1m_b130_n32768", 200, 32768, 96, 130, False),
    # one batch row, whole words of up to 384 per row: the stage 1 with s_in and x in LDS, rows in
    # pairs per 64-bit shift, words split over 1-3 waves per row group; ragged ranks (rows past the
    # rank store zeros), s_mid, a rank of 1, each launch shape's width bucket (<= 64, 128, 256, 384)
    ("s1l_b1_n1024_mid", 300, 1024, 70, 1, True),
    ("s1l_b1_n4096_mid_ragged", 500, 4096, 333, 1, True),
    ("s1l_b1_n8192_mid", 600, 8192, 250, 1, True),
    ("s1l_b1_n12288_mid", 400, 12288, 130, 1, True),
    ("s1l_b1_n11008_r1", 64, 11008, 1, 1, True),
    ("s1m_b3_n32760", 300, 32760, 130, 3, True),
    # the batched stage 1 where no plan fits one round of blocks (the x slice of 48+ batch rows
    # leaves too little LDS for the rows' words): two rounds at 48 and 128 rows, three at 100, with
    # ragged ranks and batch
    ("sb_rounds_b48_n28672", 300, 28672, 3000, 48, True),
    ("sb_rounds_b128_n11008", 500, 11008, 2976, 128, False),
    ("sb_rounds_b100_n28672", 200, 28672, 2900, 100, True),
    # the VALU stage 1 that decodes each sign word once for all batch rows: two to four rows on rows of
    # up to 128 words (each launch shape's width bucket), two rows on rows of 257-384 words; ragged
    # ranks and row ends, s_mid, a rank of 1; and the rows next to its bounds, which other kernels take
    ("s1b_b2_n1024_mid_ragged", 300, 1024, 70, 2, True),
    ("s1b_b4_n2048_mid", 600, 2048, 250, 4, True),
    ("s1b_b3_n4096_ragged", 500, 4096, 333, 3, False),
    ("s1b_b4_n4064_mid", 400, 4064, 130, 4, True),
    ("s1b_b2_n11008", 700, 11008, 1632, 2, False),
    ("s1b_b2_n12288_mid", 400, 12288, 130, 2, True),
    ("s1b_b2_n11008_r1", 64, 11008, 1, 2, True),
    ("not_s1b_b4_n8192_mid", 600, 8192, 250, 4, True),
    ("not_s1b_b3_n11008", 700, 11008, 1632, 3, False),
]


def gemv_run(nq, c, dtype, x_shape=None):
    U_bits = nq.pack_binary_gemv(dev_t(c["U"]), method="half2")
    V_bits = nq.pack_binary_gemv(dev_t(c["V"]), method="half2")
    x = dev_t(c["x"], dtype)
    if x_shape is not None:
        x = x.reshape(x_shape)
    s_mid = None if c["s_mid"] is None else dev_t(c["s_mid"], dtype)
    y = torch.ops.binary_kernels.nanoquant_dyn_forward(
        x, dev_t(c["s_in"], dtype), V_bits, s_mid, U_bits, dev_t(c["s_out"], dtype),
        num_thread_stage1=128, num_thread_stage2=128, num_row_per_warp_stage1=2, num_row_per_warp_stage2=2,
        num_acc_stage1=1, num_acc_stage2=1, num_pipeline_stage1=8, num_pipeline_stage2=8)
    torch.cuda.synchronize()
    return y, U_bits, V_bits


def oracle_inputs(c, dtype):
    """The exact values the device sees (fp16 as drawn, or rounded to bf16)."""
    f = (lambda a: a.astype(np.float64)) if dtype == torch.float16 else \
        (lambda a: torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16).double().numpy())
    return {k: (None if v is None else (f(v) if v.dtype == np.float16 else v)) for k, v in c.items()}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", GEMV_CASES, ids=[c[0] for c in GEMV_CASES])
def test_gemv_parity(nq, case, dtype):
    name, m, n, r, B, mid = case
    announce("gemv", name, dtype, (m, n, r, B))
    c = O.random_case(11, m, n, r, B, with_mid=mid)
    y, U_bits, V_bits = gemv_run(nq, c, dtype)
    np.testing.assert_array_equal(as_words(U_bits), O.pack_binary_gemv(c["U"], "half2"))
    np.testing.assert_array_equal(as_words(V_bits), O.pack_binary_gemv(c["V"], "half2"))
    o = oracle_inputs(c, dtype)
    y64 = O.nanoquant_forward_f64(o["x"], o["s_in"], c["V"], o["s_mid"], c["U"], o["s_out"])
    assert tuple(y.shape) == (B, m) and y.dtype == dtype
    err, nsat = rel_err(y, y64, "gemv", dtype)
    print(f"[gemv] {name} {dtype} rel_err={err:.3e} saturated={nsat}", flush=True)
    assert err <= TOL[("gemv", dtype)], err


@pytest.mark.parametrize("shape", [(4096, 4096, 1024, 1), (130, 200, 70, 5), (11008, 4096, 1632, 3),
                                   (11008, 4096, 1632, 32), (4096, 11008, 1632, 64)])
def test_gemv_stage_entry_points_match_nq_gemv(nq, shape):
    """nq_gemv_stage1 then nq_gemv_stage2 give nq_gemv's output bit for bit."""
    from nanoquant_amd import _lib
    m, n, r, B = shape
    announce("gemv stages", shape)
    c = O.random_case(15, m, n, r, B, with_mid=True)
    y, U_bits, V_bits = gemv_run(nq, c, torch.float16)
    lib = _lib.load()
    x, s_in, s_mid, s_out = dev_t(c["x"]), dev_t(c["s_in"]), dev_t(c["s_mid"]), dev_t(c["s_out"])
    ws = torch.zeros(lib.nq_gemv_workspace_bytes(B, n, r, m), dtype=torch.uint8, device="cuda")
    y2 = torch.empty_like(y)
    st = _lib.stream_of(x.device)
    _lib.check(lib.nq_gemv_stage1(_lib.NQ_F16, x.data_ptr(), s_in.data_ptr(), V_bits.data_ptr(), s_mid.data_ptr(), B,
                                  n, r, m, ws.data_ptr(), ws.numel(), st), "stage1")
    _lib.check(lib.nq_gemv_stage2(_lib.NQ_F16, U_bits.data_ptr(), s_out.data_ptr(), y2.data_ptr(), B, n, r, m,
                                  ws.data_ptr(), ws.numel(), st), "stage2")
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int16), y.view(torch.int16))


GENERIC_STAGE1_CASES = [
    # name, m, n, r, batch, with_mid, x offset in elements: n % 8 != 0 or an x that is not 16-byte
    # aligned sends stage 1 to the one-wave-per-row kernel (vector loads only when n % 8 == 0 and
    # both x and s_in are 16-byte aligned)
    ("n70_b1", 72, 70, 24, 1, False, 0),
    ("n70_b3_mid", 72, 70, 24, 3, True, 0),
    ("n4095_b2", 256, 4095, 160, 2, False, 0),
    ("x_offset2_b1", 300, 512, 96, 1, False, 1),
    ("x_offset2_b5_mid", 130, 1024, 64, 5, True, 1),
    ("n5_b1", 40, 5, 3, 1, False, 0),
]


@pytest.mark.parametrize("case", GENERIC_STAGE1_CASES, ids=[c[0] for c in GENERIC_STAGE1_CASES])
def test_gemv_generic_stage1(nq, case):
    name, m, n, r, B, mid, off = case
    announce("gemv generic stage 1", name, (m, n, r, B, off))
    c = O.random_case(16, m, n, r, B, with_mid=mid)
    U_bits = nq.pack_binary_gemv(dev_t(c["U"]), method="half2")
    V_bits = nq.pack_binary_gemv(dev_t(c["V"]), method="half2")
    buf = torch.zeros(off + B * n + 8, dtype=torch.float16, device="cuda")
    buf[off:off + B * n] = dev_t(c["x"]).reshape(-1)
    x = buf[off:off + B * n].view(B, n)
    assert x.is_contiguous() and (x.data_ptr() % 16 == 0) == (off == 0)
    s_mid = None if c["s_mid"] is None else dev_t(c["s_mid"])
    y = torch.ops.binary_kernels.nanoquant_dyn_forward(
        x, dev_t(c["s_in"]), V_bits, s_mid, U_bits, dev_t(c["s_out"]), num_acc_stage1=1, num_acc_stage2=1)
    torch.cuda.synchronize()
    y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], c["s_mid"], c["U"], c["s_out"])
    err, _ = rel_err(y, y64, "gemv", torch.float16)
    print(f"[gemv generic] {name} rel_err={err:.3e}", flush=True)
    assert err <= 1e-3, err


def test_gemv_workspace_survives_graph_capture(nq):
    """A GEMV captured at batch 1, then an eager call that needs a larger workspace on the same
    stream, then a new allocation, then a replay: the replay still gives the eager result and the
    new tensor is left alone (a workspace freed under a captured graph would be overwritten)."""
    announce("gemv workspace under capture")
    # batch 128 at r = 4096 needs a 4 MiB workspace, more than a batch-1 call asks for
    m, n, r = 512, 512, 4096
    c = O.random_case(18, m, n, r, 128)
    U_bits = nq.pack_binary_gemv(dev_t(c["U"]), method="half2")
    V_bits = nq.pack_binary_gemv(dev_t(c["V"]), method="half2")
    s_in, s_out = dev_t(c["s_in"]), dev_t(c["s_out"])
    x1, xb = dev_t(c["x"][:1]), dev_t(c["x"])
    kw = dict(num_acc_stage1=1, num_acc_stage2=1)
    op = torch.ops.binary_kernels.nanoquant_dyn_forward
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        want1 = op(x1, s_in, V_bits, None, U_bits, s_out, **kw)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        y1 = op(x1, s_in, V_bits, None, U_bits, s_out, **kw)
    with torch.cuda.stream(stream):
        yb = op(xb, s_in, V_bits, None, U_bits, s_out, **kw)
        sentinel = torch.full((1 << 20,), 7, dtype=torch.int32, device="cuda")
        del yb
        for _ in range(3):
            graph.replay()
    stream.synchronize()
    assert torch.equal(y1, want1)
    assert bool((sentinel == 7).all())


def test_gemv_1d_and_3d_inputs(nq):
    announce("gemv shapes")
    c = O.random_case(12, 96, 64, 32, 6)
    y2, _, _ = gemv_run(nq, c, torch.float16)
    y3, _, _ = gemv_run(nq, c, torch.float16, x_shape=(2, 3, 64))
    assert tuple(y3.shape) == (2, 3, 96)
    torch.testing.assert_close(y3.reshape(6, 96), y2, rtol=0, atol=0)
    c1 = dict(c, x=c["x"][:1])
    y1, _, _ = gemv_run(nq, c1, torch.float16, x_shape=(64,))
    assert tuple(y1.shape) == (96,)
    torch.testing.assert_close(y1, y2[0], rtol=0, atol=0)


def test_gemv_saturates_like_the_reference(nq):
    announce("gemv saturation")
    c = O.random_case(13, 256, 4096, 1024, 2)
    c["s_out"] = (c["s_out"].astype(np.float32) * 60).astype(np.float16)
    y, _, _ = gemv_run(nq, c, torch.float16)
    y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], None, c["U"], c["s_out"])
    err, nsat = rel_err(y, y64, "gemv", torch.float16)
    assert nsat > 0, "the case must saturate some outputs"
    assert err <= 1e-3


def test_gemv_errors(nq):
    c = O.random_case(14, 64, 64, 32, 1)
    U_bits = nq.pack_binary_gemv(dev_t(c["U"]), method="half2")
    V_bits = nq.pack_binary_gemv(dev_t(c["V"]), method="half2")
    x, s_in, s_out = dev_t(c["x"]), dev_t(c["s_in"]), dev_t(c["s_out"])
    op = torch.ops.binary_kernels.nanoquant_dyn_forward
    with pytest.raises(ValueError, match="n_acc1 should be one of \\[1, 2\\], but 4 was given"):
        op(x, s_in, V_bits, None, U_bits, s_out)
    kw = dict(num_acc_stage1=1, num_acc_stage2=1)
    with pytest.raises(RuntimeError, match="scale_g must be float16 tensor"):
        op(x, s_in.float(), V_bits, None, U_bits, s_out, **kw)
    with pytest.raises(RuntimeError, match="scale_l size mismatch"):
        op(x, s_in, V_bits, s_in, U_bits, s_out, **kw)
    with pytest.raises(RuntimeError, match="Ubits must be"):
        op(x, s_in, U_bits, None, V_bits, s_out, **kw)


# --------------------------------------------------------------------------- GEMM

GEMM_CASES = [
    # name, batch, n, r, m, with_mid
    ("small", 5, 64, 32, 64, False),
    ("tails", 130, 272, 288, 192, True),
    # 64-k step kernel with its k range split over two wave groups, ragged rows and features
    ("ragged_ksplit", 100, 512, 256, 320, True),
    # an odd number of 64-k steps in stage 1 (one wave group), a split stage 2
    ("odd_steps", 70, 192, 192, 320, False),
    ("cfg1_b256", 256, 4096, 1024, 4096, False),
    ("llama7b_gate_055_b256", 256, 4096, 1632, 11008, False),
    ("llama7b_down_055_b256", 256, 11008, 1632, 4096, False),
    ("llama7b_gate_055_b2048", 2048, 4096, 1632, 11008, False),
    # stage 1 of 193 64-k steps on 8 x 16 tiles of 32 rows: too long for two 32-row ranges, so its
    # k ranges (4 of 49 steps) run over four wave groups on 64-row tiles
    ("long_k_groups64_b256", 256, 12352, 4096, 256, False),
    # stage 2 counts 1024 tiles of 64 rows x 256 features, so it runs 512 blocks of 128 rows x 256
    # features (waves of 64 x 128), the last row block ragged: 1000 = 7 * 128 + 104
    ("wide_ragged_rows", 1000, 256, 128, 16384, True),
    # small grids on 32-row tiles, the last one ragged (200 = 6 * 32 + 8): stage 1 splits K across the
    # grid (7 tiles, 8 ranges), stage 2 (4 steps, 224 tiles) splits it over two wave groups
    ("small_grid_ragged", 200, 4096, 256, 8192, True),
    # 32-row tiles with K over two wave groups at 56 steps (stage 2 of a rank-3520 factorisation,
    # 144 tiles of 32 rows, the last ragged: 260 = 8 * 32 + 4)
    ("groups32_56_steps", 260, 512, 3520, 4096, False),
    # K over four wave groups: stage 1 of 128 steps over 160 tiles (16 row tiles, the last ragged:
    # 1000 = 15 * 64 + 40, times 10 feature tiles), group sums added through the step buffers
    ("groups4_long_k", 1000, 8192, 2560, 320, True),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_gemm_parity(nq, case, dtype):
    name, B, n, r, m, mid = case
    announce("gemm", name, dtype, (B, n, r, m))
    c = O.random_case(21, m, n, r, B, with_mid=mid)
    s_mid = c["s_mid"] if mid else np.ones(r, np.float16)
    packed = nq.pack_binary_marlin_fused(dev_t(c["V"].T), dev_t(c["U"].T), dev_t(c["s_in"], dtype),
                                         dev_t(s_mid, dtype), dev_t(c["s_out"], dtype))
    V_bits, U_bits, s1, s2, s3, ws = packed
    if B <= 256:  # packing bit-exact against the oracle's fused packer
        ref = O.pack_binary_marlin_fused(c["V"].T, c["U"].T, c["s_in"], s_mid, c["s_out"])
        np.testing.assert_array_equal(as_words(V_bits), ref[0])
        np.testing.assert_array_equal(as_words(U_bits), ref[1])
    x = dev_t(c["x"], dtype)
    y = torch.ops.binary_kernels.marlin_nanoquant_forward(x, V_bits, U_bits, s1, s2, s3, ws)
    torch.cuda.synchronize()
    o = oracle_inputs(dict(c, s_mid=s_mid), dtype)
    if dtype == torch.bfloat16:
        y64 = O.marlin_nanoquant_f64(o["x"], o["s_in"], c["V"], o["s_mid"], c["U"], o["s_out"], round_imm=round_bf16)
    else:
        y64 = O.nanoquant_forward_f64(o["x"], o["s_in"], c["V"], o["s_mid"], c["U"], o["s_out"])
    assert tuple(y.shape) == (B, m) and y.dtype == dtype
    err, nsat = rel_err(y, y64, "gemm", dtype)
    print(f"[gemm] {name} {dtype} rel_err={err:.3e} saturated={nsat}", flush=True)
    assert err <= TOL[("gemm", dtype)], err


@pytest.mark.parametrize("K", [96, 192], ids=["k96_mfma16", "k192_mfma32"])
@pytest.mark.parametrize("scales", ["none", "in", "out", "both"])
def test_gemm_onebit_scale_variants(nq, scales, K):
    # K % 64 != 0 runs the 16x16x32 kernel, K % 64 == 0 the 32x32x16 one
    announce("gemm onebit", scales, K)
    B, N = 33, 192
    rng = np.random.default_rng(5)
    w = np.where(rng.random((N, K)) < 0.5, -1, 1).astype(np.int8)
    s_in = np.abs(rng.normal(1, 0.2, K)).astype(np.float16)
    s_out = np.abs(rng.normal(1, 0.2, N)).astype(np.float16)
    x = rng.normal(size=(B, K)).astype(np.float16)
    words, p_in, p_out, ws_size = nq.pack_binary_marlin(dev_t(w), dev_t(s_in), dev_t(s_out))
    use_in, use_out = scales in ("in", "both"), scales in ("out", "both")
    ws = torch.zeros(max(ws_size, 32), dtype=torch.int32, device="cuda")
    y = torch.ops.binary_kernels.marlin_onebit_forward(dev_t(x), words, p_in if use_in else None,
                                                       p_out if use_out else None, ws)
    torch.cuda.synchronize()
    y64 = (x.astype(np.float64) * (s_in.astype(np.float64) if use_in else 1.0)) @ w.T.astype(np.float64)
    y64 = y64 * (s_out.astype(np.float64) if use_out else 1.0)
    err, _ = rel_err(y, y64, "gemm", torch.float16)
    assert err <= 1e-3, err


# Plans: 40 tiles of 32 rows in 6 ranges; long K (172 steps) in 10 ranges of 18 steps, each over four
# wave groups of 5, 5, 4 and 4 steps, on a partial row tile; 72 tiles of 64 rows with an odd 65 steps
# (so no split over wave groups) split on 64-row tiles; 257 steps in 16 ranges of 17 and a last range
# of 2, so two of its four wave groups run no step of their own
@pytest.mark.parametrize("B,K,N", [(256, 4096, 1280), (100, 11008, 512), (1100, 4160, 1024), (64, 16448, 512)],
                         ids=["b256_k4096_rows32", "b100_k11008_long_k", "b1100_k4160_rows64",
                              "b64_k16448_short_last_range"])
def test_gemm_split_k(nq, B, K, N):
    """Small grids split K across blocks (fp32 planes in the workspace the op allocates, added
    by a finishing launch); the same call through the C ABI without a workspace runs unsplit.
    Both within 1e-3 of float64."""
    from nanoquant_amd import _lib
    lib = _lib.load()
    announce("gemm split-k", B, K, N, lib.nq_gemm_onebit_workspace_bytes(B, K, N))
    assert lib.nq_gemm_onebit_workspace_bytes(B, K, N) > 0
    rng = np.random.default_rng(9)
    w = np.where(rng.random((N, K)) < 0.5, -1, 1).astype(np.int8)
    s_in = np.abs(rng.normal(1, 0.2, K)).astype(np.float16)
    s_out = (np.abs(rng.normal(1, 0.2, N)) / 16).astype(np.float16)
    x = rng.normal(size=(B, K)).astype(np.float16)
    words, p_in, p_out, ws_size = nq.pack_binary_marlin(dev_t(w), dev_t(s_in), dev_t(s_out))
    ws = torch.zeros(max(ws_size, 32), dtype=torch.int32, device="cuda")
    xd = dev_t(x)
    y_split = torch.ops.binary_kernels.marlin_onebit_forward(xd, words, p_in, p_out, ws)
    y_plain = torch.empty_like(y_split)
    status = lib.nq_gemm_onebit(_lib.NQ_F16, xd.data_ptr(), words.data_ptr(), p_in.data_ptr(), p_out.data_ptr(),
                                y_plain.data_ptr(), B, K, N, None, 0, _lib.stream_of(xd.device))
    assert status == 0
    torch.cuda.synchronize()
    y64 = ((x.astype(np.float64) * s_in.astype(np.float64)) @ w.T.astype(np.float64)) * s_out.astype(np.float64)
    for y in (y_split, y_plain):
        err, _ = rel_err(y, y64, "gemm", torch.float16)
        assert err <= 1e-3, err


# Split plans: 32-row tiles in one wave group (6 ranges); 32-row tiles over four wave groups (4
# ranges of 43 steps; 10 of 18 on a partial row tile); 64-row tiles over four wave groups (193 steps,
# too long for two 32-row ranges: 4 ranges of 49)
@pytest.mark.parametrize("B,K,N", [(256, 4096, 1280), (256, 11008, 1792), (100, 11008, 512), (256, 12352, 4096)],
                         ids=["rows32", "groups32", "groups32_partial_rows", "groups64"])
def test_gemm_split_scratch_and_replays(nq, B, K, N):
    """A split GEMM's results do not depend on what its scratch held: a workspace of random bytes,
    calls one after another and replays of a captured graph (with eager calls between them) give
    the same bits, within 1e-3 of float64."""
    from nanoquant_amd import _lib
    lib = _lib.load()
    nbytes = lib.nq_gemm_onebit_workspace_bytes(B, K, N)
    announce("gemm split scratch", B, K, N, nbytes)
    assert nbytes > 0
    rng = np.random.default_rng(21)
    w = np.where(rng.random((N, K)) < 0.5, -1, 1).astype(np.int8)
    s_in = np.abs(rng.normal(1, 0.2, K)).astype(np.float16)
    s_out = (np.abs(rng.normal(1, 0.2, N)) / 16).astype(np.float16)
    x = rng.normal(size=(B, K)).astype(np.float16)
    words, p_in, p_out, _ = nq.pack_binary_marlin(dev_t(w), dev_t(s_in), dev_t(s_out))
    xd = dev_t(x)
    ws = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")  # whatever the scratch held

    def call(y):
        st = lib.nq_gemm_onebit(_lib.NQ_F16, xd.data_ptr(), words.data_ptr(), p_in.data_ptr(), p_out.data_ptr(),
                                y.data_ptr(), B, K, N, ws.data_ptr(), nbytes, _lib.stream_of(xd.device))
        assert st == 0

    y_first = torch.empty(B, N, dtype=torch.float16, device="cuda")
    y_again = torch.empty_like(y_first)
    call(y_first)
    call(y_again)
    torch.cuda.synchronize()
    assert torch.equal(y_again, y_first)
    y64 = ((x.astype(np.float64) * s_in.astype(np.float64)) @ w.T.astype(np.float64)) * s_out.astype(np.float64)
    err, _ = rel_err(y_first, y64, "gemm", torch.float16)
    assert err <= 1e-3, err
    # a captured graph of two calls, replayed with eager calls in between
    y_graph = torch.empty_like(y_first)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call(y_graph)
        call(y_graph)
    for _ in range(3):
        y_graph.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_first)
        call(y_again)
        torch.cuda.synchronize()
        assert torch.equal(y_again, y_first)


# --------------------------------------------------------------------------- Llama-3-70B shapes

def mixed_rank(base: int, seed: int) -> int:
    """Mixture-of-rank draw: uniform in [0.8, 1.2] x the 0.55-bpw rank, rounded to 32."""
    return int(round(np.random.default_rng(seed).uniform(0.8, 1.2) * base / 32.0)) * 32


BIG_CASES = [
    # kind, name, batch, m, n, r  (Llama-3-70B linears at 0.55 bpw; mixed ranks drawn as above)
    ("gemv", "l3_70b_kv_b4", 4, 1024, 8192, 512),
    ("gemv", "l3_70b_qo_b1", 1, 8192, 8192, 2240),
    ("gemv", "l3_70b_gate_b16", 16, 28672, 8192, 3520),
    ("gemv", "l3_70b_down_b1", 1, 8192, 28672, 3520),
    ("gemv", "l3_70b_gate_mixed_b1", 1, 28672, 8192, mixed_rank(3520, 7)),
    ("gemv", "l3_70b_o_mixed_b4", 4, 8192, 8192, mixed_rank(2240, 3)),
    ("gemv", "l3_70b_gate_r4800_b1", 1, 28672, 8192, 4800),  # past the MFMA stage 2's largest rank
    ("gemm", "l3_70b_kv_b256", 256, 1024, 8192, 512),
    ("gemm", "l3_70b_qo_mixed_b256", 256, 8192, 8192, mixed_rank(2240, 5)),
]


@pytest.mark.parametrize("case", BIG_CASES, ids=[c[1] for c in BIG_CASES])
def test_llama3_70b_shapes(nq, case):
    kind, name, B, m, n, r = case
    announce(kind, name, (B, m, n, r))
    c = O.random_case(33, m, n, r, B)
    if kind == "gemv":
        y, _, _ = gemv_run(nq, c, torch.float16)
    else:
        packed = nq.pack_binary_marlin_fused(dev_t(c["V"].T), dev_t(c["U"].T), dev_t(c["s_in"]),
                                             dev_t(np.ones(r, np.float16)), dev_t(c["s_out"]))
        y = torch.ops.binary_kernels.marlin_nanoquant_forward(dev_t(c["x"]), *packed)
        torch.cuda.synchronize()
    y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], None, c["U"], c["s_out"])
    err, nsat = rel_err(y, y64, kind, torch.float16)
    print(f"[{kind}] {name} r={r} rel_err={err:.3e} saturated={nsat}", flush=True)
    assert err <= TOL[(kind, torch.float16)], err


# --------------------------------------------------------------------------- module

@pytest.mark.parametrize("kernel", ["gemv", "gemm"])
def test_nanoquant_linear_kernel_forward(nq, kernel):
    announce("module", kernel)
    from tests.test_host import make_layer
    lin, c = make_layer(256, 320, 96, seed=9, with_mid=True, device="cuda")
    x = torch.from_numpy(np.random.default_rng(1).normal(size=(2, 3, 256)).astype(np.float32)).cuda()
    f = lambda t: t.detach().double().cpu().numpy().reshape(-1)  # noqa: E731
    s_pre, s_mid, s_post = f(lin.scale_pre), f(lin.scale_mid), f(lin.scale_post)
    lin._prepare_kernel(kernel, torch.float16)
    y = lin(x)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32 and tuple(y.shape) == (2, 3, 320)
    x16 = x.half().double().cpu().numpy().reshape(6, 256)
    y64 = O.nanoquant_forward_f64(x16, s_pre, c["V"], s_mid, c["U"], s_post)
    err = np.abs(y.double().cpu().numpy().reshape(6, 320) - y64).max() / np.abs(y64).max()
    assert err <= 1e-3, err


def test_state_dict_round_trip_on_gpu(nq):
    announce("state_dict")
    from tests.test_host import make_layer
    lin, c = make_layer(70, 33, 5, seed=4, device="cuda")
    state = lin.state_dict()
    assert state["V_packed"].dtype == torch.int32 and tuple(state["V_packed"].shape) == (5, 3)
    np.testing.assert_array_equal(as_words(state["U_packed"]), O.pack_binary_gemv(c["U"], "lsb_first"))
    other, _ = make_layer(70, 33, 5, seed=8, device="cuda")
    other.load_state_dict(state, strict=True)
    torch.testing.assert_close(other.V, lin.V)
    torch.testing.assert_close(other.U, lin.U)


# --------------------------------------------------------------------------- checkpoint words -> kernel words

@pytest.mark.parametrize("method", ["lsb_first", "half2"])
@pytest.mark.parametrize("OK,pad", [((64, 16), (64, 16)), ((100, 80), (128, 96)), ((1632, 4096), (1792, 4096)),
                                    ((4096, 1632), (4096, 1792)), ((5, 40), (256, 48))],
                         ids=["exact", "ragged", "v_gate_055", "u_down_055", "tiny"])
def test_repack_to_marlin_matches_dense_packing(nq, OK, pad, method):
    """Marlin words straight from sign words equal the oracle's Marlin packing of the dense
    matrix padded with +1."""
    announce("repack marlin", OK, pad, method)
    (O_, K_), (Op, Kp) = OK, pad
    rng = np.random.default_rng(O_ * 7 + K_)
    w = np.where(rng.random((O_, K_)) < 0.5, -1, 1).astype(np.int8)
    words_in = O.pack_binary_gemv(w, method)
    padded = np.ones((Op, Kp), np.int8)
    padded[:O_, :K_] = w
    exp, _, _, _ = O.pack_binary_marlin(padded, np.ones(Kp, np.float16), np.ones(Op, np.float16))
    got = nq.repack_binary_marlin(torch.from_numpy(words_in.view(np.int32)).cuda(), (O_, K_), (Op, Kp), method)
    np.testing.assert_array_equal(as_words(got), exp)


@pytest.mark.parametrize("nrm", [(256, 288, 192), (4096, 1632, 11008)], ids=["rank_pad_288", "gate_055"])
def test_fused_marlin_from_packed_matches_fused_packer(nq, nrm):
    """pack_binary_marlin_fused_from_packed on lsb_first checkpoint words equals
    pack_binary_marlin_fused on the dense factors, every output bit for bit."""
    n, r, m = nrm
    announce("fused from packed", nrm)
    c = O.random_case(17, m, n, r, 1, with_mid=True)
    s_g, s_l, s_h = dev_t(c["s_in"]), dev_t(c["s_mid"]), dev_t(c["s_out"])
    ref = nq.pack_binary_marlin_fused(dev_t(c["V"].T), dev_t(c["U"].T), s_g, s_l, s_h)
    Vw = torch.from_numpy(O.pack_binary_gemv(c["V"], "lsb_first").view(np.int32)).cuda()
    Uw = torch.from_numpy(O.pack_binary_gemv(c["U"], "lsb_first").view(np.int32)).cuda()
    got = nq.pack_binary_marlin_fused_from_packed(Vw, (r, n), Uw, (m, r), s_g, s_l, s_h)
    for name, a, b in zip(["V_bits", "U_bits", "s_g", "s_l", "s_h", "workspace"], got, ref):
        assert a.shape == b.shape and a.dtype == b.dtype, name
        assert torch.equal(a, b), name


@pytest.mark.parametrize("kernel", ["gemv", "gemm"])
def test_load_packed_for_kernels_matches_dense_route(nq, kernel):
    """A model loaded from its packed state dict with load_packed_for_kernels has the kernel
    words and outputs of the reference route (load_state_dict, which unpacks to dense factors,
    then _prepare_kernel), and no dense factor."""
    announce("packed loader", kernel)
    import torch.nn as nn
    from tests.test_host import make_layer

    def model(seed):
        a, _ = make_layer(256, 320, 96, seed=seed, with_mid=True, device="cuda")
        b, _ = make_layer(320, 128, 64, seed=seed + 1, device="cuda")
        return nn.Sequential(a, nn.ReLU(), b)

    src = model(3)
    state = {k: v.clone() for k, v in src.state_dict().items()}
    dense_route = model(50)
    dense_route.load_state_dict(state, strict=True)
    for lin in (dense_route[0], dense_route[2]):
        lin._prepare_kernel(kernel, torch.float16)
    packed_route = model(70)
    res = nq.load_packed_for_kernels(packed_route, state, kernel, torch.float16)
    assert not res.unexpected_keys
    x = torch.from_numpy(np.random.default_rng(2).normal(size=(3, 256)).astype(np.float32)).cuda()
    for a, b in ((dense_route[0], packed_route[0]), (dense_route[2], packed_route[2])):
        assert not hasattr(b, "V") and not hasattr(b, "U")
        names = ["V_int8", "U_int8"] + (["s1", "s2", "s3"] if kernel == "gemm" else
                                        ["scale_pre", "scale_mid", "scale_post"])
        for name in names:
            ta, tb = getattr(a, name), getattr(b, name)
            if ta is None:
                assert tb is None, name
                continue
            assert torch.equal(ta, tb), name
    ya, yb = dense_route(x), packed_route(x)
    torch.cuda.synchronize()
    assert torch.equal(ya, yb)


# (in, out, rank) of the auto-routing layers: a small one, whose GEMV limit is the 256-row cap, and
# the Llama-2-7B q/k/v/o shape at 0.55 bpw, whose limit the work bound sets (250 rows)
AUTO_LAYERS = [(256, 320, 96), (4096, 4096, 1120)]


@pytest.mark.parametrize("sizes", AUTO_LAYERS, ids=[f"{i}x{o}_r{r}" for i, o, r in AUTO_LAYERS])
def test_auto_kernel_routes_by_rows(nq, sizes):
    """kernel_type "auto" runs the GEMV up to auto_gemv_max_rows rows and the GEMM beyond: its
    outputs equal those of the layer prepared for that kernel, bit for bit, from the dense
    factors and from the packed state dict alike."""
    announce("auto kernel", sizes)
    import copy
    from nanoquant_amd.modules.linear import auto_gemv_max_rows
    from tests.test_host import make_layer
    n_in, n_out, rank = sizes
    limit = auto_gemv_max_rows(n_in, n_out, rank)
    assert limit == (256 if n_in == 256 else 250), limit
    base, c = make_layer(n_in, n_out, rank, seed=12, with_mid=True, device="cuda")
    state = {k: v.clone() for k, v in base.state_dict().items()}
    layers = {}
    for kt in ("gemv", "gemm", "auto"):
        layers[kt] = copy.deepcopy(base)
        layers[kt]._prepare_kernel(kt, torch.float16)
    packed_auto, _ = make_layer(n_in, n_out, rank, seed=99, with_mid=True, device="cuda")
    nq.load_packed_for_kernels(packed_auto, state, "auto", torch.float16)
    assert layers["auto"].auto_gemv_rows == limit and packed_auto.auto_gemv_rows == limit
    rng = np.random.default_rng(4)
    f = lambda t: t.detach().double().cpu().numpy().reshape(-1)  # noqa: E731
    for rows, kernel in ((1, "gemv"), (limit, "gemv"), (limit + 1, "gemm"), (300, "gemm")):
        x = torch.from_numpy(rng.normal(size=(rows, n_in)).astype(np.float16)).cuda()
        want = layers[kernel](x)
        for got in (layers["auto"](x), packed_auto(x)):
            assert torch.equal(got, want), (rows, kernel)
        y64 = O.nanoquant_forward_f64(x.double().cpu().numpy(), f(base.scale_pre), c["V"], f(base.scale_mid), c["U"],
                                      f(base.scale_post))
        err = np.abs(want.double().cpu().numpy() - y64).max() / np.abs(y64).max()
        assert err <= 1e-3, (rows, err)
    x3 = torch.from_numpy(rng.normal(size=(2, 130, n_in)).astype(np.float16)).cuda()  # 260 rows: the GEMM
    assert torch.equal(layers["auto"](x3), layers["gemm"](x3))
