"""Write golden vectors for the Marlin packers from the reference's own code.

``pack_binary_marlin`` and ``pack_binary_marlin_fused`` (reference
``src/nanoquant/kernel/utils.py:186-284``) fix an arbitrary bit/scale layout that
no closed form, invariant or reference test pins, so their input/output pairs are
taken from the reference implementation itself. This script loads that one file
(which imports only os, typing and torch) by path, runs it on small seeded inputs,
and stores inputs and outputs in ``marlin_vectors.npz`` beside this script.

It runs only where the reference checkout exists (``/root/reference``); the
committed ``.npz`` is what the tests read.
"""
import importlib.util
import os
import sys

import numpy as np
import torch

REF_UTILS = "/root/reference/src/nanoquant/kernel/utils.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "marlin_vectors.npz")


def load_reference_utils():
    spec = importlib.util.spec_from_file_location("_nanoquant_reference_kernel_utils", REF_UTILS)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def signs(rng, shape):
    return torch.from_numpy(np.where(rng.random(shape) < 0.5, -1, 1).astype(np.int8))


def scales(rng, n):
    return torch.from_numpy(np.abs(rng.normal(1.0, 0.2, n)).astype(np.float16))


def main():
    ref = load_reference_utils()
    rng = np.random.default_rng(20240611)
    out = {}
    single = [(64, 16), (64, 32), (128, 16), (128, 64), (192, 48), (256, 256)]
    for idx, (O, K) in enumerate(single):
        w = signs(rng, (O, K))
        s_in = scales(rng, K)
        s_out = scales(rng, O)
        words, s_in_p, s_out_p, ws = ref.pack_binary_marlin(w, s_in, s_out)
        out[f"single{idx}_w"] = w.numpy()
        out[f"single{idx}_s_in"] = s_in.numpy()
        out[f"single{idx}_s_out"] = s_out.numpy()
        out[f"single{idx}_words"] = words.numpy().view(np.uint32)
        out[f"single{idx}_s_in_p"] = s_in_p.numpy()
        out[f"single{idx}_s_out_p"] = s_out_p.numpy()
        out[f"single{idx}_ws"] = np.array(ws, dtype=np.int64)
    fused = [(64, 32, 64), (64, 256, 128), (128, 288, 64), (32, 96, 192)]  # (N, R, M)
    for idx, (N, R, M) in enumerate(fused):
        V_sign = signs(rng, (N, R))
        U_sign = signs(rng, (R, M))
        s_g = scales(rng, N)
        s_l = scales(rng, R)
        s_h = scales(rng, M)
        res = ref.pack_binary_marlin_fused(V_sign, U_sign, s_g, s_l, s_h)
        names = ["V_bits", "U_bits", "s_g_p", "s_l_p", "s_h_p", "workspace"]
        out[f"fused{idx}_V_sign"] = V_sign.numpy()
        out[f"fused{idx}_U_sign"] = U_sign.numpy()
        out[f"fused{idx}_s_g"] = s_g.numpy()
        out[f"fused{idx}_s_l"] = s_l.numpy()
        out[f"fused{idx}_s_h"] = s_h.numpy()
        for name, t in zip(names, res):
            a = t.numpy()
            if name.endswith("bits"):
                a = a.view(np.uint32)
            out[f"fused{idx}_{name}"] = a
    out["n_single"] = np.array(len(single))
    out["n_fused"] = np.array(len(fused))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(single)} single and {len(fused)} fused cases")


if __name__ == "__main__":
    sys.exit(main())
