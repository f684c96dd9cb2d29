"""``torch.compile(fullgraph=True, mode="reduce-overhead", backend="inductor")`` through the
``binary_kernels`` ops, as the reference compiles its decode step (kernel/test_decode.py:385-402):
the fake (Meta) implementations let dynamo trace the ops without graph breaks, and the ops' real
implementations then run inside the CUDA-graph trees of "reduce-overhead", allocating their
outputs and the GEMV workspace from the graphs' pools.

Bars: the compiled ops give the eager outputs bit for bit over repeated (graph-replayed) calls;
the compiled decode step of a 2-layer model gives logits within 2e-2 of the eager step (inductor
fuses the torch ops around the linears, which rounds differently).
"""
import sys

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


def announce(*what):
    print("\n[case]", *what, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def nq():
    import nanoquant_amd
    from nanoquant_amd import _lib
    _lib.load()
    torch._dynamo.reset()
    return nanoquant_amd


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _gemv_case(nq):
    m, n, r = 320, 256, 96
    c = O.random_case(31, m, n, r, 4, with_mid=True)
    U = nq.pack_binary_gemv(_dev(c["U"]), method="half2")
    V = nq.pack_binary_gemv(_dev(c["V"]), method="half2")
    s_in, s_mid, s_out = _dev(c["s_in"]), _dev(c["s_mid"]), _dev(c["s_out"])
    return c, U, V, s_in, s_mid, s_out


def _cudagraph_skips():
    from torch._dynamo.utils import counters
    return sum(counters["inductor"].get(k, 0) for k in ("cudagraph_skips",))


def test_compiled_gemv_runs_in_cudagraphs(nq):
    """The GEMV op (nothing mutated) runs inside the CUDA graphs of "reduce-overhead": its output and
    its workspace come from the graph pool, and every replay gives the eager result."""
    announce("compiled gemv op, cudagraph trees")
    c, U, V, s_in, s_mid, s_out = _gemv_case(nq)
    kw = dict(num_acc_stage1=1, num_acc_stage2=1)

    def f(x):
        return torch.ops.binary_kernels.nanoquant_dyn_forward(x, s_in, V, s_mid, U, s_out, **kw) * 2

    before = _cudagraph_skips()
    compiled = torch.compile(f, fullgraph=True, mode="reduce-overhead", dynamic=False, backend="inductor")
    rng = np.random.default_rng(3)
    for i in range(5):  # the first calls warm up and record, the later ones replay
        x = _dev(rng.normal(size=(4, c["x"].shape[1])).astype(np.float16))
        want = f(x)
        got = compiled(x).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want), i
    assert _cudagraph_skips() == before, "the GEMV graph was not captured"


def test_compiled_gemm_op_matches_eager(nq):
    """The GEMM op's schema marks its workspace mutated (Tensor(a!), as the reference's), so the
    compiled function runs without CUDA graphs; its outputs equal eager's."""
    announce("compiled gemm op")
    c, _, _, s_in, s_mid, s_out = _gemv_case(nq)
    marlin = nq.pack_binary_marlin_fused(_dev(c["V"].T), _dev(c["U"].T), s_in, s_mid, s_out)

    def f(x):
        return torch.ops.binary_kernels.marlin_nanoquant_forward(x, *marlin) + 1

    compiled = torch.compile(f, fullgraph=True, mode="reduce-overhead", dynamic=False, backend="inductor")
    rng = np.random.default_rng(4)
    for i in range(3):
        x = _dev(rng.normal(size=(70, c["x"].shape[1])).astype(np.float16))
        want = f(x)
        got = compiled(x)
        torch.cuda.synchronize()
        assert torch.equal(got, want), i


def test_compiled_decode_step_matches_eager(nq):
    from nanoquant_amd.decode import GraphDecoder, LlamaShape, random_llama
    shape = LlamaShape(hidden=256, layers=2, heads=4, kv_heads=2, ffn=512, vocab=1000)
    announce("compiled decode step", shape)
    model = random_llama(shape, bpw=0.55, seed=5, device="cuda", kernel_type="gemv", dtype=torch.float16)
    B, T, steps = 2, 12, 6
    prompt = torch.randint(0, shape.vocab, (B, T), device="cuda", generator=torch.Generator("cuda").manual_seed(2))
    eager = GraphDecoder(model, B, T + steps + 1)
    comp = GraphDecoder(model, B, T + steps + 1)
    eager.prefill(prompt)
    comp.prefill(prompt)
    cache = comp.cache
    for t in cache.k + cache.v:  # written in place by every step, as a static cache's tensors are
        torch._dynamo.mark_static_address(t)
    before = _cudagraph_skips()

    @torch.no_grad()
    def step(tok, pos):
        return model(tok, pos, cache)[:, -1]

    compiled = torch.compile(step, mode="reduce-overhead", fullgraph=True, dynamic=False, backend="inductor")
    worst = 0.0
    for i in range(steps):
        tok = eager.ids.index_select(1, eager.pos)  # teacher-forced on the eager tokens
        pos = eager.pos.clone()
        got = compiled(tok, pos).float()
        want = eager.decode(1, use_graph=False).float()
        torch.cuda.synchronize()
        rel = float((got - want).abs().max() / want.abs().max())
        worst = max(worst, rel)
        assert rel <= 2e-2, (i, rel)
    print(f"[compile] worst logits rel diff {worst:.3e}", flush=True)
    assert _cudagraph_skips() == before, "the decode step was not captured"
