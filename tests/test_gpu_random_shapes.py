"""Seeded random shapes through the GEMV and GEMM ops against the float64 oracle (needs a gfx950 GPU).

The fixed cases of ``test_gpu_parity.py`` pick shapes at each kernel's switch points; these
draw sizes at random (fixed seeds, so a failure names a reproducible case) over ranges that
cross every launch rule: GEMV rows, columns that are and are not multiples of 8 or 32, ranks
of any size, 1-160 batch rows, with and without s_mid; GEMM batch rows 1-600 (every sixth case
1025-1600 rows on 16384-19200 outputs, which runs stage 2 on 128-row blocks), K and the rank
multiples of 32 (the fused packer rounds the rank to 32 before padding it to 256, and so fails
on others, as the reference's does: kernel/utils.py:255-271), outputs a multiple of 64 (the
Marlin layout). Bar: max|y - y*| / max|y*| <= 1e-3 in fp16, as the reference's own check
(modules/linear.py:282-291 restated in float64).
"""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

N_CASES = 24
BAR = 1e-3


def announce(*what):
    print("\n[case]", *what, flush=True)


@pytest.fixture(scope="module")
def nq():
    import nanoquant_amd
    from nanoquant_amd import _lib
    _lib.load()  # fail loudly when the HIP library is missing
    return nanoquant_amd


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rel(y, y64):
    y = y.float().cpu().numpy().astype(np.float64)
    return float(np.abs(y - y64).max() / np.abs(y64).max())


def gemv_shape(seed):
    rng = np.random.default_rng(1000 + seed)
    m = int(rng.integers(1, 2500))
    n = int(rng.integers(1, 3000)) if seed % 3 else 32 * int(rng.integers(1, 100))
    r = int(rng.integers(1, 700))
    B = int(rng.choice([1, 2, 3, int(rng.integers(4, 33)), int(rng.integers(33, 161))]))
    return m, n, r, B, bool(seed % 2)


def gemm_shape(seed):
    rng = np.random.default_rng(2000 + seed)
    if seed % 6 == 5:  # past 1024 tiles of 64 x 256: stage 2 on 128-row blocks, the last one ragged
        B = int(rng.integers(1025, 1601))
        return B, 32 * int(rng.integers(2, 13)), 32 * int(rng.integers(1, 5)), 64 * int(rng.integers(256, 301)), True
    B = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 257)), int(rng.integers(257, 601))]))
    n = 32 * int(rng.integers(1, 100))
    m = 64 * int(rng.integers(1, 60))
    r = 32 * int(rng.integers(1, 22))
    return B, n, r, m, bool(seed % 2)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_gemv_random_shape(nq, seed):
    m, n, r, B, mid = gemv_shape(seed)
    announce("gemv random", seed, (m, n, r, B, mid))
    c = O.random_case(seed, m, n, r, B, with_mid=mid)
    U = nq.pack_binary_gemv(dev(c["U"]), method="half2")
    V = nq.pack_binary_gemv(dev(c["V"]), method="half2")
    # tuning values from the reference's instantiated sets (its schema defaults are not all among them)
    y = torch.ops.binary_kernels.nanoquant_dyn_forward(
        dev(c["x"]), dev(c["s_in"]), V, None if c["s_mid"] is None else dev(c["s_mid"]), U, dev(c["s_out"]),
        num_acc_stage1=1, num_acc_stage2=1, num_pipeline_stage1=8, num_pipeline_stage2=8)
    torch.cuda.synchronize()
    y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], c["s_mid"], c["U"], c["s_out"])
    assert tuple(y.shape) == (B, m)
    err = rel(y, y64)
    print(f"[gemv random] seed={seed} shape={(m, n, r, B, mid)} rel_err={err:.3e}", flush=True)
    assert err <= BAR, err


@pytest.mark.parametrize("seed", range(N_CASES))
def test_gemm_random_shape(nq, seed):
    B, n, r, m, mid = gemm_shape(seed)
    announce("gemm random", seed, (B, n, r, m, mid))
    c = O.random_case(seed, m, n, r, B, with_mid=mid)
    s_mid = c["s_mid"] if mid else np.ones(r, np.float16)
    V_bits, U_bits, s1, s2, s3, ws = nq.pack_binary_marlin_fused(dev(c["V"].T), dev(c["U"].T), dev(c["s_in"]),
                                                                 dev(s_mid), dev(c["s_out"]))
    y = torch.ops.binary_kernels.marlin_nanoquant_forward(dev(c["x"]), V_bits, U_bits, s1, s2, s3, ws)
    torch.cuda.synchronize()
    y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], s_mid, c["U"], c["s_out"])
    assert tuple(y.shape) == (B, m)
    err = rel(y, y64)
    print(f"[gemm random] seed={seed} shape={(B, n, r, m, mid)} rel_err={err:.3e}", flush=True)
    assert err <= BAR, err
