"""Benchmark of the NanoQuant inference path on one MI355X.

One step = one decode GEMV (``torch.ops.binary_kernels.nanoquant_dyn_forward``) of the
Llama-2-7B gate_proj shape at 0.55 bpw (m=11008, n=4096, r=1632), batch 1, fp16, on a
weight copy that differs from the previous step's: a pool of ``--copies`` packed
copies (default 128, 394 MB) is larger than the 256 MB Infinity Cache, so every
step streams its weights from HBM. Steps are captured in a HIP graph and replayed;
the timed region is bracketed by a device synchronisation on both sides and timed
with HIP events on the capture stream.

The same JSON line carries:
* ``value``: packed bytes per GEMV / measured time per GEMV (both launches), GB/s;
* ``roofline``: the dominant kernel, stage 2 (U's sign words, 2.25 of the 3.08 MB),
  timed on its own through ``nq_gemv_stage2`` in the same way: its packed bytes /
  its time per launch against 8 TB/s; ``traffic`` is the HBM bytes per launch that
  ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` measured for it, scaled by what the
  same counters read for a copy of known size (``profiles/pmc_traffic.json``), when
  that file describes this workload, else null;
* ``gemm``: the prefill GEMM (``marlin_nanoquant_forward``) at B=2048 on the same
  shape, algorithmic TFLOP/s = 2*B*r*(n+m) / time, against 2.5 PFLOP/s dense fp16;
* ``decode_e2e``: greedy decode of a random-init Llama-2-7B-architecture model with
  every linear NanoQuant-factorised at 0.55 bpw (prompt 128, 256 new tokens, batch 1),
  tokens/s as the reference's decode harness reports it, with the bytes one step must
  read against 8 TB/s;
* ``cpu_baseline``: the reference's dense dequantize-and-matmul forward (two
  ``F.linear`` on dense +-1 bf16 factors, modules/linear.py:282-291) on the host
  cores, batch 1, on a bounded sample, in the same unit;
* ``parity``: relative error of one GEMV and one GEMM against the float64 oracle on the
  same inputs, computed in the CPU leg (null with ``--skip-cpu``).

``--batch-sweep`` prints the GEMV and the GEMM at batch 1..256 on the 7B gate and down shapes.

``--sweep`` instead prints one line per config shape: the GEMV at batch 1, 4, 16 and
the GEMM at batch 256 and 2048 on Llama-2-7B (1.0 and 0.55 bpw) and Llama-3-70B
(0.55 bpw, uniform and mixture-of-rank) linears.

Multi-GPU runs are not part of this build: ``--gpus`` above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode GEMV µs + % HBM roofline; prefill GEMM TFLOP/s (Llama-7B shapes)"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
M, N, R = 11008, 4096, 1632  # Llama-2-7B gate_proj at 0.55 bpw: r = round32(0.55*m*n/(m+n))
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "pmc_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def stage1_bytes(n, r):
    return 4 * r * ((n + 31) // 32)


def stage2_bytes(m, r):
    return 4 * m * ((r + 31) // 32)


def packed_bytes(m, n, r):
    return stage1_bytes(n, r) + stage2_bytes(m, r)


def gemv_total_bytes(m, n, r, batch):
    return packed_bytes(m, n, r) + 2 * (n + m) + 2 * batch * (n + m)


def gemv_kwargs():
    # the tuning ints NanoQuantLinear passes (modules/linear.py:210-219)
    return dict(num_thread_stage1=128, num_thread_stage2=128, num_row_per_warp_stage1=2, num_row_per_warp_stage2=2,
                num_acc_stage1=1, num_acc_stage2=1, num_pipeline_stage1=8, num_pipeline_stage2=8)


def time_graph(fn_steps, n_steps, replays, warmup_replays, stream):
    """Capture ``fn_steps`` (which enqueues n_steps steps) in a graph; return ms per step."""
    with torch.cuda.stream(stream):
        fn_steps()  # eager warm-up on the capture stream (workspaces, allocator)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = fn_steps()
    for _ in range(warmup_replays):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * n_steps), graph, outs


def make_case(seed, m, n, r, batch):
    """Seeded synthetic inputs in a fixed draw order: U signs [m, r], V signs [r, n], s_in [n], s_out [m] as
    fp16 |N(1, 0.2)|, x [batch, n] fp16 N(0, 1)."""
    rng = np.random.default_rng(seed)
    U = np.where(rng.random((m, r)) < 0.5, -1, 1).astype(np.int8)
    V = np.where(rng.random((r, n)) < 0.5, -1, 1).astype(np.int8)
    s_in = np.abs(rng.normal(1.0, 0.2, n)).astype(np.float16)
    s_out = np.abs(rng.normal(1.0, 0.2, m)).astype(np.float16)
    x = rng.normal(0.0, 1.0, (batch, n)).astype(np.float16)
    return dict(U=U, V=V, s_in=s_in, s_out=s_out, x=x)


def bench_gemv(args, dev):
    import nanoquant_amd as nq
    from nanoquant_amd import _lib

    batch = args.batch
    c = make_case(2024, M, N, R, batch)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    # copy 0 is packed from known signs (parity); the others are random words, which are
    # valid half2 words of random signs (the padding-free shape leaves no unused bits)
    U0 = nq.pack_binary_gemv(t(c["U"]), method="half2")
    V0 = nq.pack_binary_gemv(t(c["V"]), method="half2")
    gen = torch.Generator(device=dev).manual_seed(7)
    Us = [U0] + [torch.randint(-2**31, 2**31 - 1, U0.shape, dtype=torch.int32, device=dev, generator=gen)
                 for _ in range(args.copies - 1)]
    Vs = [V0] + [torch.randint(-2**31, 2**31 - 1, V0.shape, dtype=torch.int32, device=dev, generator=gen)
                 for _ in range(args.copies - 1)]
    x, s_in, s_out = t(c["x"]), t(c["s_in"]), t(c["s_out"])
    op = torch.ops.binary_kernels.nanoquant_dyn_forward
    kw = gemv_kwargs()

    y_eager = op(x, s_in, V0, None, U0, s_out, **kw)
    torch.cuda.synchronize()

    n_steps = args.copies
    replays = max(1, args.steps // n_steps)
    warm = max(1, args.warmup // n_steps)

    def steps():
        return [op(x, s_in, Vs[i], None, Us[i], s_out, **kw) for i in range(n_steps)]

    stream = torch.cuda.Stream(device=dev)
    ms, graph, outs = time_graph(steps, n_steps, replays, warm, stream)
    graph_ok = bool(torch.equal(outs[0], y_eager))
    del graph, outs

    # each launch on its own, through the stage entry points, same rotation
    lib = _lib.load()
    ws = torch.zeros(lib.nq_gemv_workspace_bytes(batch, N, R, M), dtype=torch.uint8, device=dev)
    y = torch.empty(batch, M, dtype=torch.float16, device=dev)

    def stage1_steps():
        st = torch.cuda.current_stream(dev).cuda_stream
        for i in range(n_steps):
            _lib.check(lib.nq_gemv_stage1(_lib.NQ_F16, x.data_ptr(), s_in.data_ptr(), Vs[i].data_ptr(), None, batch,
                                          N, R, M, ws.data_ptr(), ws.numel(), st), "stage 1")

    def stage2_steps():
        st = torch.cuda.current_stream(dev).cuda_stream
        for i in range(n_steps):
            _lib.check(lib.nq_gemv_stage2(_lib.NQ_F16, Us[i].data_ptr(), s_out.data_ptr(), y.data_ptr(), batch, N,
                                          R, M, ws.data_ptr(), ws.numel(), st), "stage 2")

    ms1, g1, _ = time_graph(stage1_steps, n_steps, replays, warm, stream)
    ms2, g2, _ = time_graph(stage2_steps, n_steps, replays, warm, stream)
    del g1, g2
    pb = packed_bytes(M, N, R)
    return dict(ms=ms, ms1=ms1, ms2=ms2, steps=replays * n_steps, warmup=warm * n_steps, case=c,
                y=y_eager.double().cpu().numpy(),
                graph_matches_eager=graph_ok, packed_bytes=pb, total_bytes=gemv_total_bytes(M, N, R, batch),
                pool_bytes=pb * args.copies)


def bench_gemm(args, dev):
    import nanoquant_amd as nq

    dtype = torch.float16
    B = args.gemm_batch
    c = make_case(2025, M, N, R, B)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    packed = nq.pack_binary_marlin_fused(t(c["V"].T), t(c["U"].T), t(c["s_in"]),
                                         torch.ones(R, dtype=dtype, device=dev), t(c["s_out"]))
    x = t(c["x"])
    op = torch.ops.binary_kernels.marlin_nanoquant_forward
    y = op(x, *packed)
    torch.cuda.synchronize()
    n_steps = 4

    def steps():
        return [op(x, *packed) for _ in range(n_steps)]

    stream = torch.cuda.Stream(device=dev)
    # warm-up replays first: with 8 warm-up calls, 64 timed calls measured 138 us per call against 127 us at steady
    # state (the clock ramps up under the first ~100 calls); every timed call still computes its full output
    ms, _, _ = time_graph(steps, n_steps, max(1, args.gemm_steps // n_steps), max(2, args.gemm_warmup // n_steps),
                          stream)
    flops = 2.0 * B * R * (N + M)
    tflops = flops / (ms * 1e-3) / 1e12
    return dict(ms=ms, tflops=tflops, flops=flops, r_pad=packed[1].shape[0] * 16, case=c,
                y=y.double().cpu().numpy())


def check_parity(results):
    """Relative error of the GPU outputs against the float64 oracle on the same inputs (the CPU leg of the
    bench: the oracle is the checker here, never the measured path). ``results`` maps a name to a dict with
    ``case`` and ``y``."""
    import oracle as O

    out = {}
    for name, res in results.items():
        c = res["case"]
        y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], None, c["U"], c["s_out"])
        out[name] = float(np.abs(res["y"] - y64).max() / np.abs(y64).max())
    return out


def cpu_baseline(args):
    """The reference's dense path on the host cores (oracle.compute_forward_torch)."""
    import oracle as O

    cores = min(len(os.sched_getaffinity(0)), args.cpu_threads)
    torch.set_num_threads(cores)
    c = make_case(2026, M, N, R, 1)
    dt = torch.bfloat16  # the reference module dtype (modules/linear.py:57)
    V = torch.from_numpy(c["V"].astype(np.float32)).to(dt)
    U = torch.from_numpy(c["U"].astype(np.float32)).to(dt)
    s_in = torch.from_numpy(c["s_in"].astype(np.float32)).to(dt)
    s_out = torch.from_numpy(c["s_out"].astype(np.float32)).to(dt)
    x = torch.from_numpy(c["x"].astype(np.float32)).to(dt)
    O.compute_forward_torch(x, V, U, s_in, None, s_out)  # warm-up
    times = []
    deadline = time.perf_counter() + args.cpu_seconds
    while time.perf_counter() < deadline or len(times) < 10:
        t0 = time.perf_counter()
        O.compute_forward_torch(x, V, U, s_in, None, s_out)
        times.append(time.perf_counter() - t0)
        if len(times) >= 2000:
            break
    med = float(np.median(times))
    gbs = packed_bytes(M, N, R) / med / 1e9
    return dict(value=round(gbs, 4), unit="GB/s", cores=cores, kind="port",
                sample=f"oracle compute_forward_torch (reference dense path, linear.py:282-291), bf16, B=1, "
                       f"m={M} n={N} r={R}; median of {len(times)} calls = {med * 1e6:.1f} us/GEMV, packed bytes "
                       f"of the factorised layer per call")


def measured_traffic(batch):
    """HBM bytes per launch of the stage-2 kernel from profiles/pmc_traffic.json, when it
    describes this workload; else None."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None, None
    w = rec.get("workload", {})
    if (w.get("m"), w.get("n"), w.get("r"), w.get("batch")) != (M, N, R, batch):
        return None, None
    k = rec.get("kernels", {}).get("gemv_stage2")
    if not k:
        return None, None
    return int(k["fetch_bytes"] + k["write_bytes"]), rec.get("source")


def calibration_copy(dev, mib):
    """One device copy of a known size, for scaling PMC byte counters (run under rocprofv3)."""
    src = torch.empty(mib << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] calibration copy of {mib} MiB done")


def bench_decode(args, dev):
    """Greedy decode of a random-init Llama-2-7B-architecture model (32 layers, hidden 4096,
    32 heads, FFN 11008, vocab 32000) with all seven linears per layer NanoQuant-factorised at
    0.55 bpw on the GEMV kernel: prompt of ``--e2e-prompt`` uniform-random ids, then
    ``--e2e-new`` tokens, the one-token step replayed from a HIP graph.
    tokens/s = B * (new - 1) / decode wall time, as the reference's harness reports it."""
    from nanoquant_amd.decode import LlamaShape, generate, random_llama

    shape = LlamaShape()
    t0 = time.perf_counter()
    model = random_llama(shape, bpw=0.55, seed=0, device=dev, kernel_type="gemv", dtype=torch.float16)
    torch.cuda.synchronize(dev)
    build_s = time.perf_counter() - t0
    B, T, new = args.e2e_batch, args.e2e_prompt, args.e2e_new
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    prompt = torch.randint(0, shape.vocab, (B, T), device=dev, generator=gen)
    runs = {}  # (fused, steps per graph) -> (tokens/s, prof, ids)
    variants = [(False, args.e2e_steps_per_graph)] + [(True, k) for k in sorted({1, args.e2e_steps_per_graph})]
    for fused, spg in variants:
        if (new - 1) % spg:
            continue
        generate(model, prompt, 1 + spg, steps_per_graph=spg, fused=fused)  # warm-up of kernels and allocator
        ids, tps, prof = generate(model, prompt, new, steps_per_graph=spg, fused=fused)
        runs[(fused, spg)] = (tps, prof, ids)
        log(f"[bench] decode e2e B={B} fused={fused} steps/graph={spg}: {tps:.1f} tok/s, "
            f"{prof['ms_per_token']:.3f} ms/token")
    best = max((k for k in runs if k[0]), key=lambda k: runs[k][0])
    tps, prof, ids = runs[best]
    same = all(torch.equal(r[2], ids) for k, r in runs.items() if k[0])
    # first decode step of both step kinds from the same prefix: the fused step rounds the folded
    # norm and the epilogues differently, so its logits are compared, not its greedy tokens (a
    # random-init model's logits are nearly flat, so any rounding difference flips near-ties)
    from nanoquant_amd.decode import FusedDecoder, GraphDecoder
    first = []
    for cls in (GraphDecoder, FusedDecoder):
        dec = cls(model, B, T + 2, device=dev)
        dec.prefill(prompt)
        first.append(dec.decode(1, use_graph=False).double())
        del dec
    step_rel = float((first[1] - first[0]).abs().max() / first[0].abs().max())
    # bytes one step must read: packed sign words and scales of every linear, the fp16
    # lm_head, one embedding row, and the K/V cache up to the step's position (mean over steps)
    lin_bytes = 0
    for lin in model.linears():
        lin_bytes += (lin.U_int8.numel() + lin.V_int8.numel()) * 4
        lin_bytes += 2 * (lin.scale_pre.numel() + lin.scale_post.numel())
    head_bytes = model.lm_head.weight.numel() * 2 + shape.hidden * 2
    mean_pos = T + (new - 1) / 2.0
    kv_bytes = 2 * shape.layers * B * shape.kv_heads * shape.head_dim * 2 * mean_pos
    step_bytes = lin_bytes + head_bytes + kv_bytes
    gbs = step_bytes / (prof["ms_per_token"] * 1e-3) / 1e9
    return {"model": "random-init Llama-2-7B architecture, 7 NanoQuant linears per layer at 0.55 bpw (GEMV kernel)",
            "batch": B, "prompt": T, "new_tokens": new, "tokens_per_s": round(tps, 2),
            "ms_per_token": round(prof["ms_per_token"], 4), "step": "fused (9 launches per layer)",
            "steps_per_graph": best[1],
            "tokens_per_s_by_variant": {("fused" if k[0] else "unfused") + f"_spg{k[1]}": round(v[0], 2)
                                        for k, v in runs.items()},
            "same_tokens_across_graph_sizes": bool(same), "fused_vs_unfused_first_step_logits_rel": step_rel,
            "prefill_s": round(prof["prefill_time_s_wall"], 4),
            "model_build_s": round(build_s, 2),
            "roofline": {"bound": "hbm", "bytes_per_step": int(step_bytes), "achieved": round(gbs, 2),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "tokens_per_s_at_peak": round(B * HBM_PEAK_GBS * 1e9 / step_bytes, 1)}}


def sweep_shapes():
    """(model, linear, m, n, r) of the benchmark configs: Llama-2-7B at 1.0 and 0.55 bpw and Llama-3-70B at
    0.55 bpw, then Llama-3-70B with mixture-of-rank (each rank uniform in [0.8, 1.2] x the 0.55 rank, to 32)."""
    from nanoquant_amd.decode import rank_for_bpw

    l2 = [("q,k,v,o", 4096, 4096), ("gate,up", 11008, 4096), ("down", 4096, 11008)]
    l3 = [("q,o", 8192, 8192), ("k,v", 1024, 8192), ("gate,up", 28672, 8192), ("down", 8192, 28672)]
    out = []
    for bpw in (1.0, 0.55):
        out += [(f"llama2-7b@{bpw}", name, m, n, rank_for_bpw(m, n, bpw)) for name, m, n in l2]
    out += [("llama3-70b@0.55", name, m, n, rank_for_bpw(m, n, 0.55)) for name, m, n in l3]
    rng = np.random.default_rng(2024)
    for name, m, n in [("q", 8192, 8192), ("k", 1024, 8192), ("v", 1024, 8192), ("o", 8192, 8192),
                       ("gate", 28672, 8192), ("up", 28672, 8192), ("down", 8192, 28672)]:
        base = rank_for_bpw(m, n, 0.55)
        out.append(("llama3-70b@0.55 mixed", name, m, n, int(round(rng.uniform(0.8, 1.2) * base / 32.0)) * 32))
    return out


def run_sweep(args, dev):
    """One JSON line per (shape, kind, batch): GEMV at batch 1, 4, 16 over rotating packed copies (more than 512 MB
    in total, so the weights stream from HBM), GEMM at batch 256 and 2048. Weights are random sign words."""
    op_gemv = torch.ops.binary_kernels.nanoquant_dyn_forward
    op_gemm = torch.ops.binary_kernels.marlin_nanoquant_forward
    kw = gemv_kwargs()
    gen = torch.Generator(device=dev).manual_seed(11)
    stream = torch.cuda.Stream(device=dev)
    words = lambda *shape: torch.randint(-2**31, 2**31 - 1, shape, dtype=torch.int32, device=dev,  # noqa: E731
                                         generator=gen)
    scales = lambda k: (torch.rand(k, device=dev, generator=gen) * 0.4 + 0.8).half()  # noqa: E731
    for model, name, m, n, r in sweep_shapes():
        pb = packed_bytes(m, n, r)
        copies = int(min(128, max(8, -(-(512 << 20) // pb))))
        Vs = [words(r, (n + 31) // 32) for _ in range(copies)]
        Us = [words(m, (r + 31) // 32) for _ in range(copies)]
        s_in, s_out = scales(n), scales(m)
        for B in (1, 4, 16):
            x = torch.randn(B, n, device=dev, generator=gen).half()

            def steps():
                return [op_gemv(x, s_in, Vs[i], None, Us[i], s_out, **kw) for i in range(copies)]

            ms, graph, _ = time_graph(steps, copies, max(1, 1024 // copies), 1, stream)
            del graph
            print(json.dumps({"kind": "gemv", "model": model, "linear": name, "m": m, "n": n, "r": r, "batch": B,
                              "us": round(ms * 1e3, 3), "packed_gbs": round(pb / (ms * 1e-3) / 1e9, 1),
                              "frac_hbm": round(pb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              "copies": copies}), flush=True)
        del Vs, Us
        r_pad = -(-r // 256) * 256
        wv, wu = words(n // 16, r_pad // 2), words(r_pad // 16, m // 2)
        s_g, s_l, s_h = scales(n), scales(r_pad), scales(m)
        ws = torch.zeros(m // 128 * 32, dtype=torch.int32, device=dev)
        for B in (256, 2048):
            x = torch.randn(B, n, device=dev, generator=gen).half()

            def gsteps():
                return [op_gemm(x, wv, wu, s_g, s_l, s_h, ws) for _ in range(4)]

            ms, graph, _ = time_graph(gsteps, 4, 32, 16, stream)  # 64 warm-up calls, as the default GEMM line
            del graph
            flops = 2.0 * B * r * (n + m)
            print(json.dumps({"kind": "gemm", "model": model, "linear": name, "m": m, "n": n, "r": r, "r_pad": r_pad,
                              "batch": B, "us": round(ms * 1e3, 2),
                              "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                              "frac_mfma": round(flops / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}),
                  flush=True)
        torch.cuda.empty_cache()


def run_batch_sweep(args, dev):
    """One JSON line per (shape, batch, kind): the GEMV and the GEMM at batch 1, 2, 4, 8, 16, 32, 64, 128, 256 on
    the Llama-2-7B gate and down shapes at 0.55 bpw, both over the same rotating copies (more than 512 MB of packed
    weights in all, so both stream from HBM). This is where one kernel should hand over to the other."""
    from nanoquant_amd.decode import rank_for_bpw

    op_gemv = torch.ops.binary_kernels.nanoquant_dyn_forward
    op_gemm = torch.ops.binary_kernels.marlin_nanoquant_forward
    kw = gemv_kwargs()
    gen = torch.Generator(device=dev).manual_seed(12)
    stream = torch.cuda.Stream(device=dev)
    words = lambda *shape: torch.randint(-2**31, 2**31 - 1, shape, dtype=torch.int32, device=dev,  # noqa: E731
                                         generator=gen)
    scales = lambda k: (torch.rand(k, device=dev, generator=gen) * 0.4 + 0.8).half()  # noqa: E731
    for name, m, n in [("gate,up", 11008, 4096), ("down", 4096, 11008)]:
        r = rank_for_bpw(m, n, 0.55)
        r_pad = -(-r // 256) * 256
        pb = packed_bytes(m, n, r)
        copies = int(min(128, max(8, -(-(512 << 20) // pb))))
        Vs = [words(r, (n + 31) // 32) for _ in range(copies)]
        Us = [words(m, (r + 31) // 32) for _ in range(copies)]
        Wv = [words(n // 16, r_pad // 2) for _ in range(copies)]
        Wu = [words(r_pad // 16, m // 2) for _ in range(copies)]
        s_in, s_out, s_l = scales(n), scales(m), scales(r_pad)
        ws = torch.zeros(m // 128 * 32, dtype=torch.int32, device=dev)
        for B in (1, 2, 4, 8, 16, 32, 64, 128, 256):
            x = torch.randn(B, n, device=dev, generator=gen).half()
            reps = max(1, 512 // copies)

            def gemv_steps():
                return [op_gemv(x, s_in, Vs[i], None, Us[i], s_out, **kw) for i in range(copies)]

            def gemm_steps():
                return [op_gemm(x, Wv[i], Wu[i], s_in, s_l, s_out, ws) for i in range(copies)]

            for kind, fn in (("gemv", gemv_steps), ("gemm", gemm_steps)):
                ms, graph, _ = time_graph(fn, copies, reps, 1, stream)
                del graph
                print(json.dumps({"kind": kind, "linear": name, "m": m, "n": n, "r": r, "batch": B,
                                  "us": round(ms * 1e3, 3),
                                  "packed_gbs": round(pb / (ms * 1e-3) / 1e9, 1),
                                  "tflops": round(2.0 * B * r * (n + m) / (ms * 1e-3) / 1e12, 2)}), flush=True)
        del Vs, Us, Wv, Wu
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048, help="timed GEMV steps (rounded to whole graph replays)")
    ap.add_argument("--warmup", type=int, default=256, help="untimed GEMV steps before timing")
    ap.add_argument("--copies", type=int, default=128, help="distinct weight copies rotated through")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--gemm-batch", type=int, default=2048)
    ap.add_argument("--gemm-steps", type=int, default=256, help="timed GEMM calls")
    ap.add_argument("--gemm-warmup", type=int, default=64, help="untimed GEMM calls before timing")
    ap.add_argument("--skip-gemm", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--skip-decode", action="store_true", help="skip the end-to-end decode measurement")
    ap.add_argument("--sweep", action="store_true",
                    help="measure GEMV (batch 1/4/16) and GEMM (batch 256/2048) on every config shape instead")
    ap.add_argument("--batch-sweep", action="store_true",
                    help="measure GEMV and GEMM at batch 1..256 on the 7B gate and down shapes instead")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the end-to-end decode and print its result alone (for kernel traces)")
    ap.add_argument("--e2e-batch", type=int, default=1)
    ap.add_argument("--e2e-prompt", type=int, default=128)
    ap.add_argument("--e2e-new", type=int, default=256)
    ap.add_argument("--e2e-steps-per-graph", type=int, default=15)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one device copy of this many MiB (PMC byte-counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the path has no "
              "multi-GPU collective to measure. Run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no GPU available", file=sys.stderr)
        return 1

    import nanoquant_amd  # noqa: F401
    from nanoquant_amd import _lib
    _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    if args.sweep:  # every config shape, one JSON line each (not the headline line)
        import nanoquant_amd  # noqa: F401
        run_sweep(args, dev)
        return 0

    if args.batch_sweep:  # the hand-over between the GEMV and the GEMM, one JSON line each
        run_batch_sweep(args, dev)
        return 0

    if args.decode_only:  # profiling aid: only the end-to-end decode, reported on its own line
        log(f"[bench] decode e2e B={args.e2e_batch} prompt={args.e2e_prompt} new={args.e2e_new}")
        print(json.dumps({"decode_e2e": bench_decode(args, dev)}), flush=True)
        return 0

    log(f"[bench] gemv m={M} n={N} r={R} B={args.batch} copies={args.copies}")
    g = bench_gemv(args, dev)
    gemv_us = g["ms"] * 1e3
    achieved = g["packed_bytes"] / (g["ms"] * 1e-3) / 1e9
    s1_gbs = stage1_bytes(N, R) / (g["ms1"] * 1e-3) / 1e9
    s2_gbs = stage2_bytes(M, R) / (g["ms2"] * 1e-3) / 1e9
    log(f"[bench] gemv {gemv_us:.3f} us/step, {achieved:.1f} GB/s packed; "
        f"stage 1 {g['ms1'] * 1e3:.3f} us ({s1_gbs:.1f} GB/s), stage 2 {g['ms2'] * 1e3:.3f} us ({s2_gbs:.1f} GB/s)")

    if args.calib_copy_mib > 0:
        calibration_copy(dev, args.calib_copy_mib)

    gemm = None
    if not args.skip_gemm:
        log(f"[bench] gemm B={args.gemm_batch}")
        gm = bench_gemm(args, dev)
        gemm = {"batch": args.gemm_batch, "us": round(gm["ms"] * 1e3, 2), "tflops": round(gm["tflops"], 2),
                "roofline": {"bound": "mfma", "achieved": round(gm["tflops"], 2), "peak": MFMA_F16_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(gm["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                             "traffic": None},
                "flops_per_call": gm["flops"], "r_pad": gm["r_pad"]}
        log(f"[bench] gemm {gm['ms'] * 1e3:.1f} us, {gm['tflops']:.1f} TFLOP/s")

    decode = None
    if not args.skip_decode:
        log(f"[bench] decode e2e B={args.e2e_batch} prompt={args.e2e_prompt} new={args.e2e_new}")
        decode = bench_decode(args, dev)

    cpu = None
    parity = {"gemv_rel_err": None, "gemm_rel_err": None}
    if not args.skip_cpu:
        log("[bench] cpu baseline and parity check")
        cpu = cpu_baseline(args)
        log(f"[bench] cpu {cpu['value']} GB/s ({cpu['sample']})")
        checked = check_parity({"gemv": g} if gemm is None else {"gemv": g, "gemm": gm})
        parity = {"gemv_rel_err": checked["gemv"], "gemm_rel_err": checked.get("gemm")}
        log(f"[bench] parity {parity}")

    traffic, traffic_src = measured_traffic(args.batch)
    line = {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": g["steps"],
        "warmup": g["warmup"],
        "ms_per_step": round(g["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"decode GEMV, Llama-2-7B gate_proj at 0.55 bpw (m={M}, n={N}, r={R}), batch "
                               f"{args.batch}, fp16 in / fp32 accumulate, {args.copies} rotating packed weight copies "
                               f"({g['pool_bytes'] / 1e6:.0f} MB) replayed in a HIP graph",
                   "m": M, "n": N, "r": R, "batch": args.batch, "copies": args.copies},
        "gemv_us": round(gemv_us, 4),
        "roofline": {"bound": "hbm", "kernel": "GEMV stage 2 (s2t_kernel, U sign words)",
                     "achieved": round(s2_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(s2_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": stage2_bytes(M, R), "us_per_launch": round(g["ms2"] * 1e3, 4),
                     "traffic_source": traffic_src},
        "gemv_stages": {"stage1_us": round(g["ms1"] * 1e3, 4), "stage1_gbs": round(s1_gbs, 2),
                        "stage1_bytes": stage1_bytes(N, R), "stage2_us": round(g["ms2"] * 1e3, 4),
                        "stage2_gbs": round(s2_gbs, 2), "stage2_bytes": stage2_bytes(M, R),
                        "op_frac_of_hbm_peak": round(achieved / HBM_PEAK_GBS, 4)},
        "gemv_total_bytes_gbs": round(g["total_bytes"] / (g["ms"] * 1e-3) / 1e9, 2),
        "gemm": gemm,
        "decode_e2e": decode,
        "cpu_baseline": cpu,
        "parity": {**parity, "gemv_graph_matches_eager": g["graph_matches_eager"], "bar": 1e-3},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
