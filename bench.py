"""Benchmark of the NanoQuant inference path on one MI355X.

A step is one decode GEMV (``torch.ops.binary_kernels.nanoquant_dyn_forward``: both launches)
of the Llama-2-7B down_proj shape at 0.55 bpw (m=4096, n=11008, r=1632; the 4096x11008
0.55-bpw GEMV), batch 1, fp16, on a weight copy that differs from the previous step's: step i
uses copy i mod ``--copies`` of a pool (128 copies, 394 MB) larger than the 256 MB Infinity
Cache, so every step streams its weights from HBM. One HIP graph holds ``--warmup`` untimed
steps, a GPU wall-clock stamp (``nq_timestamp``), exactly ``--steps`` timed steps and a second
stamp. The graph is replayed once untimed (its first dispatches), then once more behind a spin
kernel, between device synchronisations; the time per step is the difference of the second
replay's stamps divided by ``--steps``.

The JSON line carries:
* ``value``: packed bytes per GEMV / time per GEMV, GB/s (``ms_per_step`` the time);
* ``roofline``: the whole GEMV (its two launches) against 8 TB/s on the packed bytes of both
  factors, with each launch's own figure (stage 1 over V's words, stage 2 over U's) timed
  through ``nq_gemv_stage1`` / ``nq_gemv_stage2`` in the same rotation; ``traffic`` is the HBM
  bytes per GEMV from ``rocprofv3 --pmc`` runs on these kernels (``profiles/pmc_traffic.json``)
  when that file describes this workload, else null;
* ``gemv``: the down and gate shapes at batch 1, each timed over 2048 steps at steady state;
* ``floor``: what every decode-sized launch pays before any arithmetic, in the same 128-copy
  graph rotation: an empty launch, a bare cold read of 1, 2 and 3 MB, and the GEMV's own two
  reads (V's words, then U's) as two dependent launches with nothing else in them;
* ``gemm``: the prefill GEMM (``marlin_nanoquant_forward``) at B=2048 on the gate and down
  shapes, TFLOP/s = 2*B*r*(n+m) / time against 2.5 PFLOP/s dense fp16;
* ``pack``: sign packing, unpacking, reordering and Marlin packing of the down factors, GB/s of
  bytes read plus written against 8 TB/s;
* ``dense``: the fused decode step's final norm and lm_head (``nq_dense_gemv``, 32000 x 4096 fp16)
  at batch 1 and 4 on cold weights, GB/s on the weight bytes against 8 TB/s;
* ``decode_e2e``: greedy decode of a random-init Llama-2-7B-architecture model with every linear
  NanoQuant-factorised at 0.55 bpw (prompt 128, 256 new tokens, batch 1): the fused-linears step
  with attention in torch (the headline), the unfused step, the step whose q/k/v launch also
  applies RoPE and writes the cache rows and the causal mask (attention products in torch), and
  the step with the HIP attention;
* ``cpu_baseline``: the reference's dense dequantize-and-matmul forward (two ``F.linear`` on
  dense +-1 factors, modules/linear.py:282-291) on the host cores at batch 1 in bf16 (the
  reference's module dtype; ``value``) and fp32, and its packers in eager torch;
* ``parity``: relative error of the GEMVs and GEMMs against the float64 oracle on the same
  inputs (the CPU leg; null with ``--skip-cpu``).

``--floor`` prints the ``floor`` section alone; ``--sweep`` prints one line per config shape (GEMV
at batch 1/4/16, GEMM at 256/2048); ``--batch-sweep`` the GEMV and the GEMM at batch 1..256 on the
7B gate and down shapes (every config shape with ``--batch-sweep-shapes configs``); ``--gemv-only``,
``--decode-only`` (with ``--decode-variants``), ``--dense-only`` and the ``--skip-*`` switches narrow a
run for kernel traces.
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
R_055 = 1632  # round32(0.55 * m * n / (m + n)) for 4096 x 11008 and 11008 x 4096
SHAPES = {"down": (4096, 11008, R_055), "gate": (11008, 4096, R_055)}  # (m, n, r)
HEADLINE = "down"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "pmc_traffic.json")
SPIN_CYCLES = 2_000_000  # about 1 ms of GPU clock ahead of each timed replay


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


def capture(fn, stream, eager_first=True):
    """Record ``fn`` into a graph on ``stream``, after one eager run of it (allocator warm-up)
    unless ``eager_first`` is False."""
    if eager_first:
        with torch.cuda.stream(stream):
            fn()
        stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = fn()
    return graph, outs


def timed_replay(graph, stream, replays=1, before=None):
    """Milliseconds of ``replays`` back-to-back replays of ``graph`` on ``stream``: ``before``
    (an untimed graph, e.g. the warm-up steps) and a spin kernel run first, the events bracket
    only the timed replays, and the device is synchronised on both sides."""
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        if before is not None:
            before.replay()
        torch.cuda._sleep(SPIN_CYCLES)
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def steady_ms(fn_steps, n_steps, stream, replays=8, warm_replays=2):
    """ms per step of a graph of ``n_steps`` steps replayed ``replays`` times after warm-up."""
    graph, outs = capture(fn_steps, stream)
    for _ in range(warm_replays):
        with torch.cuda.stream(stream):
            graph.replay()
    ms = timed_replay(graph, stream, replays) / (replays * n_steps)
    return ms, graph, outs


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


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


class GemvPool:
    """Packed copies of one linear: copy 0 from known signs (checked against the oracle), the
    others random words (valid half2 words of random signs: these shapes leave no padding bits)."""

    def __init__(self, name, copies, batch, dev, seed):
        import nanoquant_amd as nq

        self.name = name
        self.m, self.n, self.r = SHAPES[name]
        self.batch, self.copies = batch, copies
        self.case = make_case(seed, self.m, self.n, self.r, batch)
        c = self.case
        U0 = nq.pack_binary_gemv(dev_t(c["U"], dev), method="half2")
        V0 = nq.pack_binary_gemv(dev_t(c["V"], dev), method="half2")
        gen = torch.Generator(device=dev).manual_seed(seed + 1)
        rand = lambda like: torch.randint(-2**31, 2**31 - 1, like.shape, dtype=torch.int32, device=dev,  # noqa: E731
                                          generator=gen)
        self.Us = [U0] + [rand(U0) for _ in range(copies - 1)]
        self.Vs = [V0] + [rand(V0) for _ in range(copies - 1)]
        self.x, self.s_in, self.s_out = dev_t(c["x"], dev), dev_t(c["s_in"], dev), dev_t(c["s_out"], dev)

    def op_steps(self, count, first=0):
        op = torch.ops.binary_kernels.nanoquant_dyn_forward
        kw = gemv_kwargs()

        def fn():
            return [op(self.x, self.s_in, self.Vs[(first + i) % self.copies], None,
                       self.Us[(first + i) % self.copies], self.s_out, **kw) for i in range(count)]
        return fn

    def stage_steps(self, stage, count, ws, y):
        from nanoquant_amd import _lib
        lib = _lib.load()
        b, n, r, m = self.batch, self.n, self.r, self.m

        def fn():
            st = torch.cuda.current_stream().cuda_stream
            for i in range(count):
                k = i % self.copies
                if stage == 1:
                    s = lib.nq_gemv_stage1(_lib.NQ_F16, self.x.data_ptr(), self.s_in.data_ptr(), self.Vs[k].data_ptr(),
                                           None, b, n, r, m, ws.data_ptr(), ws.numel(), st)
                else:
                    s = lib.nq_gemv_stage2(_lib.NQ_F16, self.Us[k].data_ptr(), self.s_out.data_ptr(), y.data_ptr(),
                                           b, n, r, m, ws.data_ptr(), ws.numel(), st)
                _lib.check(s, f"stage {stage}")
        return fn


def bench_gemv_headline(args, dev):
    """``--warmup`` untimed then exactly ``--steps`` timed GEMVs of the headline shape."""
    pool = GemvPool(HEADLINE, args.copies, args.batch, dev, seed=2024)
    op = torch.ops.binary_kernels.nanoquant_dyn_forward
    kw = gemv_kwargs()
    # copy 0 (known signs, for parity) and the copy of the first timed step, eagerly: this also
    # loads both kernels before any capture
    y_eager = op(pool.x, pool.s_in, pool.Vs[0], None, pool.Us[0], pool.s_out, **kw)
    k0 = args.warmup % pool.copies
    y_first = op(pool.x, pool.s_in, pool.Vs[k0], None, pool.Us[k0], pool.s_out, **kw)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    warm_steps, timed_steps = pool.op_steps(args.warmup), pool.op_steps(args.steps, first=args.warmup)
    # one graph: the warm-up steps, a GPU timestamp, exactly the timed steps, a GPU timestamp; the
    # graph's own launch gap falls before the timed region, which spans the timed steps and the
    # dispatch of the closing timestamp kernel
    from nanoquant_amd import _lib
    lib = _lib.load()
    stamps = torch.zeros(2, dtype=torch.int64, device=dev)

    def stamp(i):
        _lib.check(lib.nq_timestamp(stamps.data_ptr() + 8 * i, torch.cuda.current_stream().cuda_stream), "stamp")

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        warm_steps()
        stamp(0)
        outs = timed_steps()
        stamp(1)
    torch.cuda.synchronize()
    # the first replay (untimed) takes the graph's first dispatches; the second one is stamped
    for _ in range(2):
        with torch.cuda.stream(stream):
            torch.cuda._sleep(SPIN_CYCLES)
            graph.replay()
        torch.cuda.synchronize()
    t0, t1 = stamps.tolist()
    ms = (t1 - t0) / lib.nq_wall_clock_hz() * 1e3 / args.steps
    how = ("GPU wall-clock stamps inside the graph, after the warm-up steps and after the timed steps, on the "
           "graph's second replay")
    del graph
    graph_ok = bool(torch.equal(outs[0], y_first))
    del outs
    return pool, ms, y_eager, graph_ok, how


def bench_gemv_shape(pool, dev, steps=2048):
    """Steady-state ms per GEMV and per launch (stage entry points, same rotation)."""
    from nanoquant_amd import _lib
    lib = _lib.load()
    stream = torch.cuda.Stream(device=dev)
    n_steps = pool.copies
    replays = max(1, steps // n_steps)
    ms, g, _ = steady_ms(pool.op_steps(n_steps), n_steps, stream, replays)
    del g
    ws = torch.empty(lib.nq_gemv_workspace_bytes(pool.batch, pool.n, pool.r, pool.m), dtype=torch.uint8, device=dev)
    y = torch.empty(pool.batch, pool.m, dtype=torch.float16, device=dev)
    ms1, g1, _ = steady_ms(pool.stage_steps(1, n_steps, ws, y), n_steps, stream, replays)
    ms2, g2, _ = steady_ms(pool.stage_steps(2, n_steps, ws, y), n_steps, stream, replays)
    del g1, g2
    m, n, r = pool.m, pool.n, pool.r
    pb = packed_bytes(m, n, r)
    kern = lambda b, t: {"us_per_launch": round(t * 1e3, 4), "bytes": b,  # noqa: E731
                         "achieved": round(b / (t * 1e-3) / 1e9, 2), "frac": round(b / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return {"m": m, "n": n, "r": r, "batch": pool.batch, "steps": replays * n_steps, "us": round(ms * 1e3, 4),
            "packed_bytes": pb, "packed_gbs": round(pb / (ms * 1e-3) / 1e9, 2),
            "frac_hbm": round(pb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "total_bytes_gbs": round(gemv_total_bytes(m, n, r, pool.batch) / (ms * 1e-3) / 1e9, 2),
            "stage1": dict(kernel="s1l_kernel (V's sign words)" if pool.batch == 1 and n % 32 == 0 and (n // 32) <= 384
                           else "stage-1 kernel (V's sign words)", **kern(stage1_bytes(n, r), ms1)),
            "stage2": dict(kernel="s2t_kernel (U's sign words)", **kern(stage2_bytes(m, r), ms2))}


FLOOR_READS_MB = (1, 2, 3)


def bench_floor(dev, copies=128, replays=8):
    """The fixed costs of a decode-sized launch, each as a graph of ``copies`` steps replayed at
    steady state (``steady_ms``), reads rotating over ``copies`` distinct buffers (more bytes than
    the 256 MB Infinity Cache holds, so every read comes from HBM):

    * an empty launch of 1 x 64 and of 256 x 256 threads, and two dependent empty launches of the
      GEMV's grids (204 and 256 blocks of 256 threads) per step;
    * a bare cold read of 1, 2 and 3 MB over 256 blocks (one per CU), 16 bytes a lane, every load
      issued first; the 2 MB read with one word stored per block; the same 2 MB read from one
      buffer every step (L2 / Infinity Cache warm);
    * the headline GEMV's reads alone: V's 2,245,632 bytes over 204 blocks, then U's 835,584 over
      256 blocks, as two dependent launches (without and with a word stored per block), and all
      3,081,216 bytes in one launch.
    """
    from nanoquant_amd import _lib
    lib = _lib.load()
    stream = torch.cuda.Stream(device=dev)
    m, n, r = SHAPES[HEADLINE]
    v_bytes, u_bytes = stage1_bytes(n, r), stage2_bytes(m, r)
    per_copy = max(FLOOR_READS_MB[-1] << 20, v_bytes + u_bytes)
    bufs = [torch.zeros(per_copy, dtype=torch.uint8, device=dev) for _ in range(copies)]
    sink = torch.zeros(1 << 12, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    def launches(parts, rotate=True):
        # parts: (kind, byte offset, bytes or threads, blocks) launched in order in every step; kind
        # "read" loads only, "read+store" also stores one word per block
        def fn():
            st = torch.cuda.current_stream().cuda_stream
            for i in range(copies):
                base = bufs[i if rotate else 0].data_ptr()
                for kind, off, size, blocks in parts:
                    if kind == "empty":
                        _lib.check(lib.nq_probe_empty(blocks, size, st), "probe empty")
                    else:
                        _lib.check(lib.nq_probe_read(base + off, size, blocks, sink.data_ptr(),
                                                     int(kind == "read+store"), st), "probe read")
        return fn

    two = [("read", 0, v_bytes, 204), ("read", v_bytes, u_bytes, 256)]
    cases = [("empty_1x64", [("empty", 0, 64, 1)], True),
             ("empty_256x256", [("empty", 0, 256, 256)], True),
             ("two_dependent_empty_204_256", [("empty", 0, 256, 204), ("empty", 0, 256, 256)], True)]
    cases += [(f"read_{mb}MB_cold_256_blocks", [("read", 0, mb << 20, 256)], True) for mb in FLOOR_READS_MB]
    cases += [("read_2MB_cold_256_blocks_store", [("read+store", 0, 2 << 20, 256)], True),
              ("read_2MB_warm_256_blocks", [("read", 0, 2 << 20, 256)], False),
              ("gemv_reads_two_launches", two, True),
              ("gemv_reads_two_launches_store", [("read+store",) + p[1:] for p in two], True),
              ("gemv_reads_one_launch", [("read", 0, v_bytes + u_bytes, 256)], True)]
    out = {}
    for name, parts, rotate in cases:
        ms, g, _ = steady_ms(launches(parts, rotate), copies, stream, replays)
        del g
        read = sum(p[2] for p in parts if p[0] != "empty")
        out[name] = {"us": round(ms * 1e3, 4), "launches": len(parts)}
        if read:
            out[name].update(bytes=read, gbs=round(read / (ms * 1e-3) / 1e9, 2),
                             frac_hbm=round(read / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        log(f"[bench] floor {name}: {out[name]}")
    del bufs
    torch.cuda.empty_cache()
    return {"method": f"graph of {copies} steps, {replays} timed replays after 2 warm ones, GPU events around them; "
                      "reads rotate over distinct buffers unless marked warm", "cases": out}


def bench_gemm(name, args, dev):
    import nanoquant_amd as nq

    m, n, r = SHAPES[name]
    B = args.gemm_batch
    c = make_case(2025, m, n, r, B)
    packed = nq.pack_binary_marlin_fused(dev_t(c["V"].T, dev), dev_t(c["U"].T, dev), dev_t(c["s_in"], dev),
                                         torch.ones(r, dtype=torch.float16, device=dev), dev_t(c["s_out"], dev))
    x = dev_t(c["x"], dev)
    op = torch.ops.binary_kernels.marlin_nanoquant_forward
    y = op(x, *packed)
    torch.cuda.synchronize()
    n_steps = 4
    stream = torch.cuda.Stream(device=dev)
    # warm-up replays first: the clock ramps up under the first ~100 calls; every timed call
    # still computes its full output
    ms, _, _ = steady_ms(lambda: [op(x, *packed) for _ in range(n_steps)], n_steps, stream,
                         max(1, args.gemm_steps // n_steps), max(2, args.gemm_warmup // n_steps))
    flops = 2.0 * B * r * (n + m)
    tflops = flops / (ms * 1e-3) / 1e12
    return {"m": m, "n": n, "r": r, "r_pad": packed[1].shape[0] * 16, "batch": B, "us": round(ms * 1e3, 2),
            "tflops": round(tflops, 2), "flops_per_call": flops,
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                         "traffic": measured_traffic(f"gemm_{name}", (m, n, r, B))[0],
                         "traffic_unit": "HBM bytes per call (both launches)"}}, c, y


def bench_dense(dev, copies=3):
    """The decode step's lm_head as the fused step runs it: ``nq_dense_gemv`` with its RMS-norm prologue
    and float32 logits, Llama-2-7B shapes (32000 x 4096 fp16), batch 1 and 4, over ``copies``
    rotating weight copies (786 MB: more than the Infinity Cache holds, so every read is cold),
    graph-replayed. GB/s on the weight bytes; the logits are checked against torch's RMS norm and
    linear in float64 on the first copy."""
    from nanoquant_amd import _lib
    lib = _lib.load()
    m, n, eps = 32000, 4096, 1e-5
    gen = torch.Generator(device=dev).manual_seed(9)
    stream = torch.cuda.Stream(device=dev)
    ws = [(torch.randn(m, n, device=dev, generator=gen) * 0.02).half() for _ in range(copies)]
    g = (torch.rand(n, device=dev, generator=gen) + 0.5).half()
    out = {}
    for B in (1, 4):
        x = (torch.randn(B, n, device=dev, generator=gen) * 3.0).half()
        y = torch.empty(B, m, device=dev, dtype=torch.float32)

        def fn():
            st = torch.cuda.current_stream().cuda_stream
            for i in range(copies):
                _lib.check(lib.nq_dense_gemv(_lib.NQ_F16, ws[i].data_ptr(), x.data_ptr(), g.data_ptr(), eps,
                                             y.data_ptr(), 1, B, n, m, m, st), "dense gemv")
        ms, graph, _ = steady_ms(fn, copies, stream, replays=16)
        del graph
        # the last replay's call was copy copies - 1; one more call on copy 0 for the check
        _lib.check(lib.nq_dense_gemv(_lib.NQ_F16, ws[0].data_ptr(), x.data_ptr(), g.data_ptr(), eps, y.data_ptr(), 1,
                                     B, n, m, m, torch.cuda.current_stream().cuda_stream), "dense gemv")
        xn = (g * torch.nn.functional.rms_norm(x.float(), (n,), eps=eps).half()).double()
        ref = xn @ ws[0].double().T
        rel = float((y.double() - ref).abs().max() / ref.abs().max())
        nbytes = m * n * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"b{B}"] = {"us": round(ms * 1e3, 3), "weight_bytes": nbytes, "achieved": round(gbs, 1),
                        "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "rel_err_vs_f64": rel}
    out["what"] = ("lm_head of the fused decode step: RMS norm + 32000 x 4096 fp16 linear, float32 logits "
                   f"(nq_dense_gemv), {copies} rotating weight copies")
    return out


def bench_pack(dev):
    """Packing work on the down linear's factors, each kind of launch over 16 rotating inputs (more
    than the Infinity Cache holds), graph-replayed: GB/s of bytes read plus written."""
    from nanoquant_amd import _lib
    lib = _lib.load()
    m, n, r = SHAPES[HEADLINE]
    copies = 16
    gen = torch.Generator(device=dev).manual_seed(5)
    stream = torch.cuda.Stream(device=dev)
    rows, cols = r, n  # V [r, n]: 18.0 MB of int8, 2.2 MB of words
    wn = (cols + 31) // 32
    signs = [torch.randint(0, 2, (rows, cols), dtype=torch.int8, device=dev, generator=gen).mul_(2).sub_(1)
             for _ in range(copies)]
    words = [torch.empty(rows, wn, dtype=torch.int32, device=dev) for _ in range(copies)]
    back = [torch.empty(rows, cols, dtype=torch.int8, device=dev) for _ in range(copies)]
    h2 = [torch.empty(rows, wn, dtype=torch.int32, device=dev) for _ in range(copies)]
    r_pad = -(-r // 256) * 256  # Marlin: V^T padded to [r_pad, n] -> words [n / 16, r_pad / 2]
    mar_src = [torch.randint(0, 2, (r_pad, cols), dtype=torch.int8, device=dev, generator=gen).mul_(2).sub_(1)
               for _ in range(copies)]
    mar = [torch.empty(cols // 16, r_pad // 2, dtype=torch.int32, device=dev) for _ in range(copies)]
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    L, H2 = _lib.NQ_PACK_LSB_FIRST, _lib.NQ_PACK_HALF2
    kinds = {
        "pack_signs": (lambda i: lib.nq_pack_signs(signs[i].data_ptr(), words[i].data_ptr(), rows, cols, L, st()),
                       rows * cols + 4 * rows * wn, "int8 V [1632, 11008] -> lsb_first words"),
        "unpack_signs": (lambda i: lib.nq_unpack_signs(words[i].data_ptr(), back[i].data_ptr(), rows, cols, L, st()),
                         rows * cols + 4 * rows * wn, "lsb_first words -> int8 V"),
        "repack_signs": (lambda i: lib.nq_repack_signs(words[i].data_ptr(), h2[i].data_ptr(), rows, cols, L, H2, st()),
                         8 * rows * wn, "lsb_first -> half2 words of V"),
        "pack_marlin": (lambda i: lib.nq_pack_marlin(mar_src[i].data_ptr(), mar[i].data_ptr(), r_pad, cols, st()),
                        r_pad * cols + 4 * (cols // 16) * (r_pad // 2), f"int8 V^T [{r_pad}, 11008] -> Marlin words"),
    }
    out = {}
    for name, (call, nbytes, what) in kinds.items():
        def fn(call=call, name=name):
            for i in range(copies):
                _lib.check(call(i), name)
        ms, g, _ = steady_ms(fn, copies, stream, replays=8)
        del g
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"what": what, "bytes_per_launch": nbytes, "us_per_launch": round(ms * 1e3, 3),
                     "achieved": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    # the packers' output is the oracle's (a sample of the last copy)
    import oracle as O
    s0 = signs[0][:64].cpu().numpy()
    out["checked_bits"] = bool((words[0][:64].cpu().numpy().view(np.uint32) == O.pack_binary_gemv(s0)).all()
                               and torch.equal(back[0], signs[0]))
    return out


def check_parity(results):
    """Relative error of the GPU outputs against the float64 oracle on the same inputs (the CPU leg of the
    bench: the oracle is the checker here, never the measured path). ``results`` maps a name to (case, y)."""
    import oracle as O

    out = {}
    for name, (c, y) in results.items():
        y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], None, c["U"], c["s_out"])
        out[name] = float(np.abs(y.double().cpu().numpy() - y64).max() / np.abs(y64).max())
    return out


def _median_time(fn, seconds, min_reps=10, max_reps=2000):
    fn()  # warm-up
    times = []
    deadline = time.perf_counter() + seconds
    while (time.perf_counter() < deadline or len(times) < min_reps) and len(times) < max_reps:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(args):
    """The reference's dense path and its packers on the host cores (the oracle's restatements)."""
    import oracle as O

    cores = min(len(os.sched_getaffinity(0)), args.cpu_threads)
    torch.set_num_threads(cores)
    m, n, r = SHAPES[HEADLINE]
    c = make_case(2026, m, n, r, 1)
    per = {}
    for dt, secs in ((torch.bfloat16, args.cpu_seconds), (torch.float32, args.cpu_seconds)):
        t = {k: torch.from_numpy(c[k].astype(np.float32)).to(dt) for k in ("V", "U", "s_in", "s_out", "x")}
        med, reps = _median_time(lambda: O.compute_forward_torch(t["x"], t["V"], t["U"], t["s_in"], None, t["s_out"]),
                                 secs)
        per[str(dt).replace("torch.", "")] = {"us_per_gemv": round(med * 1e6, 1), "reps": reps,
                                              "packed_gbs": round(packed_bytes(m, n, r) / med / 1e9, 4)}
    V = torch.from_numpy(c["V"])
    med_p, reps_p = _median_time(lambda: O.pack_signs_torch(V, "lsb_first"), args.cpu_pack_seconds)
    words = O.pack_signs_torch(V, "lsb_first")
    med_u, reps_u = _median_time(lambda: O.unpack_signs_torch(words, tuple(V.shape), "lsb_first"),
                                 args.cpu_pack_seconds)
    nbytes = V.numel() + 4 * words.numel()
    # the Marlin packer on the shape the GPU pack leg times: V^T padded to [r_pad, n]
    r_pad = -(-r // 256) * 256
    W = torch.from_numpy(np.where(np.random.default_rng(7).random((r_pad, n)) < 0.5, -1, 1).astype(np.int8))
    med_m, reps_m = _median_time(lambda: O.pack_marlin_torch(W), args.cpu_pack_seconds)
    mbytes = W.numel() + 4 * (n // 16) * (r_pad // 2)
    pack = {"pack_signs": {"us": round(med_p * 1e6, 1), "gbs": round(nbytes / med_p / 1e9, 3), "reps": reps_p},
            "unpack_signs": {"us": round(med_u * 1e6, 1), "gbs": round(nbytes / med_u / 1e9, 3), "reps": reps_u},
            "pack_marlin": {"us": round(med_m * 1e6, 1), "gbs": round(mbytes / med_m / 1e9, 3), "reps": reps_m,
                            "what": f"int8 V^T [{r_pad}, {n}] -> Marlin words (kernel/utils.py:186-205)"},
            "sample": f"eager-torch restatements of kernel/utils.py:51-205 on V [{r}, {n}] int8 (lsb_first) and "
                      f"V^T [{r_pad}, {n}] (Marlin), {args.cpu_pack_seconds:.0f} s bounded sample each"}
    bf = per["bfloat16"]
    return {"value": bf["packed_gbs"], "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": (f"oracle compute_forward_torch (reference dense path, linear.py:282-291), bf16, B=1, m={m} "
                       f"n={n} r={r}: median of {bf['reps']} calls = {bf['us_per_gemv']} us/GEMV, packed bytes of the "
                       f"factorised layer per call; {args.cpu_seconds:.0f} s bounded sample per dtype"),
            "by_dtype": per, "pack": pack}


def measured_traffic(kernel_key, workload):
    """HBM bytes per launch of ``kernel_key`` from profiles/pmc_traffic.json when it was measured on
    ``workload`` (m, n, r, batch); else (None, None)."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None, None
    k = rec.get("kernels", {}).get(kernel_key)
    if not k or tuple(k.get("workload", ())) != tuple(workload):
        return None, None
    return int(k["fetch_bytes"] + k["write_bytes"]), rec.get("sources", rec.get("source"))


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
    from nanoquant_amd.decode import FusedDecoder, GraphDecoder, LlamaShape, generate, random_llama

    shape = LlamaShape()
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    model = random_llama(shape, bpw=0.55, seed=0, device=dev, kernel_type="gemv", dtype=torch.float16)
    torch.cuda.synchronize(dev)
    build_s = time.perf_counter() - t0
    model_bytes = torch.cuda.memory_allocated(dev)
    B, T, new = args.e2e_batch, args.e2e_prompt, args.e2e_new
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    prompt = torch.randint(0, shape.vocab, (B, T), device=dev, generator=gen)
    spg = args.e2e_steps_per_graph
    variants = {  # name -> (fused, attention, steps per graph)
        "fused_torch_attention": (True, "torch", spg),
        "fused_torch_attention_spg1": (True, "torch", 1),
        "unfused": (False, "torch", spg),
        "fused_rope_kernel_torch_attention": (True, "rope", spg),
        "fused_hip_attention": (True, "hip", spg),
    }
    only = [v for v in args.decode_variants.split(",") if v] if args.decode_variants else list(variants)
    unknown = [v for v in only if v not in variants]
    if unknown:
        raise SystemExit(f"bench.py: unknown decode variant(s) {unknown}; known: {list(variants)}")
    runs = {}
    for name, (fused, attention, k) in variants.items():
        if (new - 1) % k or name not in only:
            continue
        generate(model, prompt, 1 + k, steps_per_graph=k, fused=fused, attention=attention)  # warm-up
        torch.cuda.reset_peak_memory_stats(dev)
        ids, tps, prof = generate(model, prompt, new, steps_per_graph=k, fused=fused, attention=attention)
        runs[name] = (tps, prof, ids, torch.cuda.max_memory_allocated(dev))
        log(f"[bench] decode e2e {name}: {tps:.1f} tok/s, {prof['ms_per_token']:.3f} ms/token")
    head = "fused_torch_attention" if "fused_torch_attention" in runs else next(iter(runs))
    tps, prof, ids, peak = runs[head]
    same = all(torch.equal(r[2], ids) for k, r in runs.items() if k.startswith("fused_torch"))
    # first decode step of each step kind from the same prefix: the fused step rounds the folded
    # norm and the epilogues differently, so its logits are compared, not its greedy tokens (a
    # random-init model's logits are nearly flat, so any rounding difference flips near-ties)
    first = {}
    steps_kinds = () if args.decode_variants else (
        ("unfused", lambda: GraphDecoder(model, B, T + 2, device=dev)),
        ("fused_torch_attention", lambda: FusedDecoder(model, B, T + 2, device=dev)),
        ("fused_rope_kernel_torch_attention", lambda: FusedDecoder(model, B, T + 2, device=dev, attention="rope")),
        ("fused_hip_attention", lambda: FusedDecoder(model, B, T + 2, device=dev, attention="hip")))
    for name, make in steps_kinds:
        dec = make()
        dec.prefill(prompt)
        first[name] = dec.decode(1, use_graph=False).double()
        del dec
    rel = {k: float((v - first["unfused"]).abs().max() / first["unfused"].abs().max())
           for k, v in first.items() if k != "unfused"} if first else None
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
            "ms_per_token": round(prof["ms_per_token"], 4),
            "step": head if head != "fused_torch_attention" else
                    ("fused linears (q/k/v and gate/up stage 1 each one launch with RMSNorm folded in, SiLU*mul "
                     "and residual epilogues; the q/k/v stage 2 writes the value cache row) with the rotary "
                     "embedding (one complex product), key-cache write, causal mask, scores, softmax and value "
                     "product in torch ops; final norm and lm_head one dense GEMV launch; HIP graph"),
            "variants": {"fused_torch_attention": "the step above (config 5 as written: non-linear ops of the "
                                                  "attention in torch)",
                         "fused_torch_attention_spg1": "the same, one step per graph",
                         "unfused": "one NanoQuantLinear GEMV op per linear, everything else in torch",
                         "fused_rope_kernel_torch_attention": "the q/k/v stage 2 also applies RoPE, writes the KV "
                                                              "cache rows and the step's causal mask; the scores, "
                                                              "softmax and value products in torch",
                         "fused_hip_attention": "RoPE, KV write and attention in nq_attention_decode"},
            "steps_per_graph": spg,
            "tokens_per_s_by_variant": {k: round(v[0], 2) for k, v in runs.items()},
            "peak_memory_bytes_by_variant": {k: int(v[3]) for k, v in runs.items()},
            "model_bytes": int(model_bytes), "linear_bytes": int(lin_bytes),
            "same_tokens_across_graph_sizes": bool(same), "first_step_logits_rel_vs_unfused": rel,
            "prefill_s": round(prof["prefill_time_s_wall"], 4), "model_build_s": round(build_s, 2),
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


def _words(gen, dev):
    return lambda *shape: torch.randint(-2**31, 2**31 - 1, shape, dtype=torch.int32, device=dev, generator=gen)


def run_sweep(args, dev):
    """One JSON line per (shape, kind, batch): GEMV at batch 1, 4, 16 over rotating packed copies (more than 512 MB
    in total, so the weights stream from HBM), GEMM at batch 256 and 2048. Weights are random sign words."""
    op_gemv = torch.ops.binary_kernels.nanoquant_dyn_forward
    op_gemm = torch.ops.binary_kernels.marlin_nanoquant_forward
    kw = gemv_kwargs()
    gen = torch.Generator(device=dev).manual_seed(11)
    stream = torch.cuda.Stream(device=dev)
    words = _words(gen, dev)
    scales = lambda k: (torch.rand(k, device=dev, generator=gen) * 0.4 + 0.8).half()  # noqa: E731
    for model, name, m, n, r in sweep_shapes():
        pb = packed_bytes(m, n, r)
        copies = int(min(128, max(8, -(-(512 << 20) // pb))))
        Vs = [words(r, (n + 31) // 32) for _ in range(copies)]
        Us = [words(m, (r + 31) // 32) for _ in range(copies)]
        s_in, s_out = scales(n), scales(m)
        for B in (1, 4, 16):
            x = torch.randn(B, n, device=dev, generator=gen).half()
            ms, graph, _ = steady_ms(lambda: [op_gemv(x, s_in, Vs[i], None, Us[i], s_out, **kw)
                                              for i in range(copies)], copies, stream, max(1, 1024 // copies), 1)
            del graph
            print(json.dumps({"kind": "gemv", "model": model, "linear": name, "m": m, "n": n, "r": r, "batch": B,
                              "us": round(ms * 1e3, 3), "packed_gbs": round(pb / (ms * 1e-3) / 1e9, 1),
                              "frac_hbm": round(pb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                              "copies": copies}), flush=True)
        del Vs, Us
        r_pad = -(-r // 256) * 256
        wv, wu = words(n // 16, r_pad // 2), words(r_pad // 16, m // 2)
        s_g, s_l, s_h = scales(n), scales(r_pad), scales(m)
        s_l[r:] = 0  # as pack_binary_marlin_fused pads the rank (r is a multiple of 32, so the zeros stay last)
        ws = torch.zeros(m // 128 * 32, dtype=torch.int32, device=dev)
        for B in (256, 2048):
            x = torch.randn(B, n, device=dev, generator=gen).half()
            ms, graph, _ = steady_ms(lambda: [op_gemm(x, wv, wu, s_g, s_l, s_h, ws) for _ in range(4)], 4, stream,
                                     32, 16)  # 64 warm-up calls, as the default GEMM line
            del graph
            flops = 2.0 * B * r * (n + m)
            print(json.dumps({"kind": "gemm", "model": model, "linear": name, "m": m, "n": n, "r": r, "r_pad": r_pad,
                              "batch": B, "us": round(ms * 1e3, 2),
                              "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                              "frac_mfma": round(flops / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}),
                  flush=True)
        torch.cuda.empty_cache()


def batch_sweep_shapes(which):
    """(model, linear, m, n, r) of the batch sweep: the Llama-2-7B gate and down shapes at 0.55 bpw ("7b"), or
    every distinct shape of the benchmark configs without the mixture-of-rank ones ("configs")."""
    from nanoquant_amd.decode import rank_for_bpw

    if which == "7b":
        return [("llama2-7b@0.55", name, m, n, rank_for_bpw(m, n, 0.55))
                for name, m, n in [("gate,up", 11008, 4096), ("down", 4096, 11008)]]
    return [s for s in sweep_shapes() if not s[0].endswith("mixed")]


def run_batch_sweep(args, dev):
    """One JSON line per (shape, batch, kind): the GEMV and the GEMM at the --batches sizes (1, 2, 4, ..., 256 by
    default) on the --batch-sweep-shapes shapes, both over the same rotating copies (more than 512 MB of packed
    weights in all, so both stream from HBM). This is where one kernel should hand over to the other. Kinds
    gemv_stage1 and gemv_stage2 time the GEMV's two launches alone (the C ABI's stage entry points, same copies)."""
    from nanoquant_amd import _lib

    lib = _lib.load()

    op_gemv = torch.ops.binary_kernels.nanoquant_dyn_forward
    op_gemm = torch.ops.binary_kernels.marlin_nanoquant_forward
    kw = gemv_kwargs()
    gen = torch.Generator(device=dev).manual_seed(12)
    stream = torch.cuda.Stream(device=dev)
    words = _words(gen, dev)
    scales = lambda k: (torch.rand(k, device=dev, generator=gen) * 0.4 + 0.8).half()  # noqa: E731
    batches = [int(b) for b in args.batches.split(",")]
    for model, name, m, n, r in batch_sweep_shapes(args.batch_sweep_shapes):
        r_pad = -(-r // 256) * 256
        pb = packed_bytes(m, n, r)
        copies = int(min(128, max(8, -(-(512 << 20) // pb))))
        Vs = [words(r, (n + 31) // 32) for _ in range(copies)]
        Us = [words(m, (r + 31) // 32) for _ in range(copies)]
        Wv = [words(n // 16, r_pad // 2) for _ in range(copies)]
        Wu = [words(r_pad // 16, m // 2) for _ in range(copies)]
        s_in, s_out, s_l = scales(n), scales(m), scales(r_pad)
        s_l[r:] = 0  # the packer's zero scale_l over the padded rank
        ws = torch.zeros(m // 128 * 32, dtype=torch.int32, device=dev)
        for B in batches:
            x = torch.randn(B, n, device=dev, generator=gen).half()
            reps = max(1, 512 // copies)
            ws_b = torch.zeros(lib.nq_gemv_workspace_bytes(B, n, r, m), dtype=torch.uint8, device=dev)
            y_b = torch.empty(B, m, dtype=torch.float16, device=dev)

            def stage(which):
                def fn():
                    st = torch.cuda.current_stream().cuda_stream
                    for i in range(copies):
                        if which == 1:
                            s = lib.nq_gemv_stage1(_lib.NQ_F16, x.data_ptr(), s_in.data_ptr(), Vs[i].data_ptr(), None,
                                                   B, n, r, m, ws_b.data_ptr(), ws_b.numel(), st)
                        else:
                            s = lib.nq_gemv_stage2(_lib.NQ_F16, Us[i].data_ptr(), s_out.data_ptr(), y_b.data_ptr(), B,
                                                   n, r, m, ws_b.data_ptr(), ws_b.numel(), st)
                        _lib.check(s, f"stage {which}")
                return fn

            for kind in ("gemv", "gemm", "gemv_stage1", "gemv_stage2"):
                if kind == "gemv":
                    fn = lambda: [op_gemv(x, s_in, Vs[i], None, Us[i], s_out, **kw) for i in range(copies)]  # noqa
                elif kind == "gemm":
                    fn = lambda: [op_gemm(x, Wv[i], Wu[i], s_in, s_l, s_out, ws) for i in range(copies)]  # noqa
                else:
                    fn = stage(1 if kind == "gemv_stage1" else 2)
                ms, graph, _ = steady_ms(fn, copies, stream, reps, 1)
                del graph
                print(json.dumps({"kind": kind, "model": model, "linear": name, "m": m, "n": n, "r": r, "batch": B,
                                  "us": round(ms * 1e3, 3),
                                  "packed_gbs": round(pb / (ms * 1e-3) / 1e9, 1),
                                  "tflops": round(2.0 * B * r * (n + m) / (ms * 1e-3) / 1e12, 2)}), flush=True)
        del Vs, Us, Wv, Wu
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed GEMV steps of the headline line")
    ap.add_argument("--warmup", type=int, default=64, help="untimed GEMV steps before them")
    ap.add_argument("--copies", type=int, default=128, help="distinct weight copies rotated through")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--gemm-batch", type=int, default=2048)
    ap.add_argument("--gemm-steps", type=int, default=256, help="timed GEMM calls")
    ap.add_argument("--gemm-warmup", type=int, default=64, help="untimed GEMM calls before timing")
    ap.add_argument("--skip-gemm", action="store_true")
    ap.add_argument("--gemm-shapes", default="gate,down", help="GEMM shapes to measure (gate, down)")
    ap.add_argument("--skip-pack", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="bounded CPU sample per dtype of the dense path")
    ap.add_argument("--cpu-pack-seconds", type=float, default=3.0, help="bounded CPU sample per packer")
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--skip-decode", action="store_true", help="skip the end-to-end decode measurement")
    ap.add_argument("--dense-only", action="store_true", help="measure the decode step's lm_head GEMV alone")
    ap.add_argument("--sweep", action="store_true",
                    help="measure GEMV (batch 1/4/16) and GEMM (batch 256/2048) on every config shape instead")
    ap.add_argument("--batch-sweep", action="store_true",
                    help="measure GEMV and GEMM at the --batches sizes on the 7B gate and down shapes instead")
    ap.add_argument("--batches", default="1,2,4,8,16,32,64,128,256")
    ap.add_argument("--batch-sweep-shapes", choices=("7b", "configs"), default="7b",
                    help="shapes of --batch-sweep: the 7B gate and down (0.55 bpw), or every config shape")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the end-to-end decode and print its result alone (for kernel traces)")
    ap.add_argument("--gemv-only", action="store_true",
                    help="run only the headline GEMV shape, with its per-launch figures (for kernel traces)")
    ap.add_argument("--e2e-batch", type=int, default=1)
    ap.add_argument("--e2e-prompt", type=int, default=128)
    ap.add_argument("--e2e-new", type=int, default=256)
    ap.add_argument("--e2e-steps-per-graph", type=int, default=15)
    ap.add_argument("--decode-variants", default="",
                    help="comma-separated decode variants to run (default: all; a subset skips the first-step "
                         "logits comparison, for kernel traces of one variant)")
    ap.add_argument("--floor", action="store_true",
                    help="measure only the launch and cold-read floor of decode-sized kernels and print it")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one device copy of this many MiB (PMC byte-counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the path has no "
              "multi-GPU collective to measure. Run with --gpus 1.", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
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
        run_sweep(args, dev)
        return 0
    if args.batch_sweep:  # the hand-over between the GEMV and the GEMM, one JSON line each
        run_batch_sweep(args, dev)
        return 0
    if args.floor:  # the launch and cold-read floor alone
        print(json.dumps({"floor": bench_floor(dev)}), flush=True)
        return 0
    if args.dense_only:  # profiling aid: only the decode step's lm_head GEMV
        print(json.dumps({"dense": bench_dense(dev)}), flush=True)
        return 0
    if args.decode_only:  # profiling aid: only the end-to-end decode, reported on its own line
        log(f"[bench] decode e2e B={args.e2e_batch} prompt={args.e2e_prompt} new={args.e2e_new}")
        print(json.dumps({"decode_e2e": bench_decode(args, dev)}), flush=True)
        return 0

    m, n, r = SHAPES[HEADLINE]
    log(f"[bench] gemv {HEADLINE} m={m} n={n} r={r} B={args.batch} copies={args.copies} "
        f"warmup={args.warmup} steps={args.steps}")
    pool, ms, y_head, graph_ok, timing_how = bench_gemv_headline(args, dev)
    pb = packed_bytes(m, n, r)
    achieved = pb / (ms * 1e-3) / 1e9
    log(f"[bench] gemv {HEADLINE}: {ms * 1e3:.3f} us/step over {args.steps} steps, {achieved:.1f} GB/s packed")
    shapes = {HEADLINE: bench_gemv_shape(pool, dev)}
    if args.gemv_only:  # profiling aid: the headline shape alone, so kernel names do not mix shapes
        if args.calib_copy_mib > 0:
            calibration_copy(dev, args.calib_copy_mib)
        print(json.dumps({"gemv_headline_us": round(ms * 1e3, 4), "gemv": shapes}), flush=True)
        return 0
    other = "gate" if HEADLINE == "down" else "down"
    pool_other = GemvPool(other, args.copies, args.batch, dev, seed=2023)
    shapes[other] = bench_gemv_shape(pool_other, dev)
    parity_cases = {f"gemv_{HEADLINE}": (pool.case, y_head)}
    op = torch.ops.binary_kernels.nanoquant_dyn_forward
    y_other = op(pool_other.x, pool_other.s_in, pool_other.Vs[0], None, pool_other.Us[0], pool_other.s_out,
                 **gemv_kwargs())
    parity_cases[f"gemv_{other}"] = (pool_other.case, y_other)
    for k, v in shapes.items():
        log(f"[bench] gemv {k} steady: {v['us']} us ({v['frac_hbm']} of HBM peak), stage 1 "
            f"{v['stage1']['us_per_launch']} us, stage 2 {v['stage2']['us_per_launch']} us")
    del pool_other

    if args.calib_copy_mib > 0:
        calibration_copy(dev, args.calib_copy_mib)

    log("[bench] floor")
    floor = bench_floor(dev)

    gemm = None
    if not args.skip_gemm:
        gemm = {}
        for name in args.gemm_shapes.split(","):
            log(f"[bench] gemm {name} B={args.gemm_batch}")
            res, c, y = bench_gemm(name, args, dev)
            gemm[name] = res
            parity_cases[f"gemm_{name}"] = (c, y)
            log(f"[bench] gemm {name}: {res['us']} us, {res['tflops']} TFLOP/s")
        torch.cuda.empty_cache()

    pack = None
    if not args.skip_pack:
        log("[bench] pack")
        pack = bench_pack(dev)
        log(f"[bench] pack {json.dumps(pack)}")
        torch.cuda.empty_cache()

    log("[bench] dense (lm_head)")
    dense = bench_dense(dev)
    log(f"[bench] dense {json.dumps(dense)}")
    torch.cuda.empty_cache()

    decode = None
    if not args.skip_decode:
        log(f"[bench] decode e2e B={args.e2e_batch} prompt={args.e2e_prompt} new={args.e2e_new}")
        decode = bench_decode(args, dev)

    cpu = None
    parity = {}
    if not args.skip_cpu:
        log("[bench] cpu baseline and parity check")
        cpu = cpu_baseline(args)
        log(f"[bench] cpu {json.dumps(cpu)}")
        parity = {f"{k}_rel_err": v for k, v in check_parity(parity_cases).items()}
        log(f"[bench] parity {parity}")

    head = shapes[HEADLINE]
    traffic, traffic_src = measured_traffic("gemv", (m, n, r, args.batch))
    line = {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"decode GEMV, Llama-2-7B down_proj at 0.55 bpw (m={m}, n={n}, r={r}), batch "
                               f"{args.batch}, fp16 in / fp32 accumulate, {args.copies} rotating packed weight copies "
                               f"({pb * args.copies / 1e6:.0f} MB) replayed in a HIP graph",
                   "m": m, "n": n, "r": r, "batch": args.batch, "copies": args.copies, "timing": timing_how},
        "gemv_us": round(ms * 1e3, 4),
        "roofline": {"bound": "hbm", "kernel": "the GEMV's two launches (s1l_kernel, then s2t_kernel)",
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "algorithmic_bytes": pb, "us_per_op": round(ms * 1e3, 4),
                     "kernels": {"stage1": head["stage1"], "stage2": head["stage2"]}},
        "gemv": shapes,
        "floor": floor,
        "gemm": gemm,
        "pack": pack,
        "dense": dense,
        "decode_e2e": decode,
        "cpu_baseline": cpu,
        "parity": {**parity, "gemv_graph_matches_eager": graph_ok, "bar": 1e-3},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
