"""nq_gemv_noalloc (the GEMV whose intermediate lives in the library's static device scratch)
against nq_gemv with a caller workspace, through the C ABI: bit-identical outputs on two calls
in a row, the second with a smaller input, and a clear error past the scratch size."""
import sys

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 4 << 20  # NQ_GEMV_NOALLOC_SCRATCH_BYTES in include/nq_hip.h


def announce(*what):
    print("\n[case]", *what, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    import nanoquant_amd  # noqa: F401
    from nanoquant_amd import _lib
    return _lib.load()


def _case(seed, m, n, r, batch, with_mid, dtype):
    import nanoquant_amd as nq
    c = O.random_case(seed, m, n, r, batch, with_mid=with_mid)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    return dict(
        x=t(c["x"]).to(dtype), s_in=t(c["s_in"]).to(dtype), s_out=t(c["s_out"]).to(dtype),
        s_mid=None if c["s_mid"] is None else t(c["s_mid"]).to(dtype),
        V=nq.pack_binary_gemv(t(c["V"]), method="half2"), U=nq.pack_binary_gemv(t(c["U"]), method="half2"),
        dims=(batch, n, r, m), raw=c)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _gemv_with_workspace(lib, d, code):
    from nanoquant_amd import _lib
    batch, n, r, m = d["dims"]
    ws = torch.empty(lib.nq_gemv_workspace_bytes(batch, n, r, m), dtype=torch.uint8, device="cuda")
    y = torch.empty(batch, m, dtype=d["x"].dtype, device="cuda")
    _lib.check(lib.nq_gemv(code, d["x"].data_ptr(), d["s_in"].data_ptr(), d["V"].data_ptr(), _ptr(d["s_mid"]),
                           d["U"].data_ptr(), d["s_out"].data_ptr(), y.data_ptr(), batch, n, r, m, ws.data_ptr(),
                           ws.numel(), _lib.stream_of(y.device)), "nq_gemv")
    return y


def _gemv_noalloc(lib, d, code):
    from nanoquant_amd import _lib
    batch, n, r, m = d["dims"]
    y = torch.empty(batch, m, dtype=d["x"].dtype, device="cuda")
    _lib.check(lib.nq_gemv_noalloc(code, d["x"].data_ptr(), d["s_in"].data_ptr(), d["V"].data_ptr(),
                                   _ptr(d["s_mid"]), d["U"].data_ptr(), d["s_out"].data_ptr(), y.data_ptr(), batch, n,
                                   r, m, _lib.stream_of(y.device)), "nq_gemv_noalloc")
    return y


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_noalloc_matches_nq_gemv_twice_second_smaller(lib, dtype):
    from nanoquant_amd import _lib
    code = _lib.dtype_code(dtype)
    # first a large call (the 7B gate shape at batch 16, with s_mid), then a smaller one in every
    # dimension, so the second call runs over scratch the first one left filled
    cases = [(11008, 4096, 1632, 16, True), (1000, 1024, 288, 3, False)]
    outs = []
    for i, (m, n, r, batch, mid) in enumerate(cases):
        announce("gemv noalloc", dtype, (m, n, r, batch, mid))
        d = _case(40 + i, m, n, r, batch, mid, dtype)
        want = _gemv_with_workspace(lib, d, code)
        got = _gemv_noalloc(lib, d, code)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (m, n, r, batch)
        if dtype == torch.float16:  # and both meet the parity bar against float64
            c = d["raw"]
            y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], c["s_mid"], c["U"], c["s_out"])
            err = np.abs(got.double().cpu().numpy() - y64).max() / np.abs(y64).max()
            assert err <= 1e-3, err
        outs.append(got)
    assert outs[1].shape == (3, 1000)


def test_noalloc_refuses_more_than_its_scratch(lib):
    from nanoquant_amd import _lib
    announce("gemv noalloc over the limit")
    batch, n, r, m = 631, 4096, 1632, 4096
    assert lib.nq_gemv_workspace_bytes(batch, n, r, m) > SCRATCH_BYTES >= lib.nq_gemv_workspace_bytes(630, n, r, m)
    status = lib.nq_gemv_noalloc(_lib.NQ_F16, None, None, None, None, None, None, None, batch, n, r, m, None)
    assert status == _lib.NQ_ERR_WORKSPACE
    assert b"static buffer" in lib.nq_last_error_message()


def test_noalloc_batched_call_beyond_the_per_range_sums(lib):
    """At 64 rows on the 4096 x 11008 shape, nq_gemv's batched stage 1 keeps per-range sums that do
    not fit in the static array (nq_gemv_workspace_bytes exceeds it); the call still runs, with the
    stage-1 kernel that keeps none, and agrees with nq_gemv and with float64 to the parity bar."""
    from nanoquant_amd import _lib
    m, n, r, batch = 4096, 11008, 1632, 64
    announce("gemv noalloc past the per-range sums", (m, n, r, batch))
    assert lib.nq_gemv_workspace_bytes(batch, n, r, m) > SCRATCH_BYTES
    d = _case(44, m, n, r, batch, True, torch.float16)
    want = _gemv_with_workspace(lib, d, _lib.NQ_F16)
    got = _gemv_noalloc(lib, d, _lib.NQ_F16)
    torch.cuda.synchronize()
    c = d["raw"]
    y64 = O.nanoquant_forward_f64(c["x"], c["s_in"], c["V"], c["s_mid"], c["U"], c["s_out"])
    scale = np.abs(y64).max()
    assert np.abs(got.double().cpu().numpy() - y64).max() / scale <= 1e-3
    assert (got.double() - want.double()).abs().max().item() / scale <= 1e-3


@pytest.mark.parametrize("shape", [(4096, 11008, 1632, 1, False), (1000, 1024, 288, 5, True)])
def test_noalloc_captured_in_a_graph(lib, shape):
    """nq_gemv_noalloc recorded into a HIP graph (torch.cuda.graph) and replayed three times, each
    time after new contents were written into x and with eager nq_gemv calls between the replays:
    every replay bit-identical to nq_gemv on the same inputs."""
    from nanoquant_amd import _lib
    m, n, r, batch, mid = shape
    announce("gemv noalloc under graph capture", shape)
    d = _case(50, m, n, r, batch, mid, torch.float16)
    y = torch.empty(batch, m, dtype=torch.float16, device="cuda")
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        status = lib.nq_gemv_noalloc(_lib.NQ_F16, d["x"].data_ptr(), d["s_in"].data_ptr(), d["V"].data_ptr(),
                                     _ptr(d["s_mid"]), d["U"].data_ptr(), d["s_out"].data_ptr(), y.data_ptr(),
                                     batch, n, r, m, torch.cuda.current_stream().cuda_stream)
    assert status == _lib.NQ_OK, lib.nq_last_error_message()
    gen = torch.Generator(device="cuda").manual_seed(7)
    for rep in range(3):
        d["x"].copy_(torch.randn(batch, n, device="cuda", generator=gen).half())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = _gemv_with_workspace(lib, d, _lib.NQ_F16)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), rep
