"""The fused decode-step entry points on the GPU: grouped GEMV stages (with the RMSNorm fold
and the residual / gated epilogues) and decode attention, through the C ABI.

Bars (written here):
* grouped GEMV without a norm or epilogue: bit-identical to nq_gemv per item;
* norm fold, residual and gated epilogues: max|y - y*| / max|y*| against float64 on the same
  fp16 inputs, <= 1e-3 (norm, residual) and <= 2e-3 (gated: three more fp16 roundings);
* attention: the rotated key stored in the cache is bit-identical to torch's fp16 rotary
  arithmetic; the stored value is the input value; rows other than the position are
  untouched; the output is within 2e-3 of float64 attention (relative to its max), across
  one and several 64-position chunks;
* a position outside the cache leaves the caches untouched and writes zeros.
"""
import ctypes
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
def lib():
    from nanoquant_amd import _lib
    return _lib.load()


def words(signs):
    return torch.from_numpy(O.pack_binary_gemv(signs, "half2").view(np.int32)).cuda()


def item(_lib, v_bits, s_in, s_mid, u_bits, s_out, y, y_off, y_stride, resid, r, m):
    it = _lib.GemvItem()
    it.v_bits, it.s_in = v_bits.data_ptr(), s_in.data_ptr()
    it.s_mid = None if s_mid is None else s_mid.data_ptr()
    it.u_bits, it.s_out = u_bits.data_ptr(), s_out.data_ptr()
    it.y = y.data_ptr() + y_off * y.element_size()
    it.resid = None if resid is None else resid.data_ptr()
    it.r, it.m, it.y_stride = r, m, y_stride
    return it


def make_linear(seed, m, n, r, with_mid=False):
    c = O.random_case(seed, m, n, r, 1, with_mid=with_mid)
    return c


def group_call(lib, dtype_code, items, x, batch, n, eps, epilogue):
    from nanoquant_amd import _lib
    arr = (_lib.GemvItem * len(items))(*items)
    need = lib.nq_gemv_group_workspace_bytes(len(items), arr, batch)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.nq_gemv_group_stage1(dtype_code, len(items), arr, x.data_ptr(), batch, n, eps, ws.data_ptr(),
                                        need, st), "group stage 1")
    _lib.check(lib.nq_gemv_group_stage2(dtype_code, len(items), arr, batch, epilogue, ws.data_ptr(), need, st),
               "group stage 2")
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("batch", [1, 3, 17])
def test_group_matches_single_gemv(lib, dtype, batch):
    from nanoquant_amd import _lib
    announce("group vs single", dtype, batch)
    n = 256
    shapes = [(192, 96), (64, 352), (64, 96)]  # (m, r): two stage-2 configurations
    x = torch.from_numpy(np.random.default_rng(3).normal(size=(batch, n)).astype(np.float16)).cuda().to(dtype)
    width = sum(m for m, _ in shapes)
    yg = torch.zeros(batch, width, dtype=dtype, device="cuda")
    items, refs, off = [], [], 0
    keep = []
    for i, (m, r) in enumerate(shapes):
        c = make_linear(10 + i, m, n, r, with_mid=(i == 1))
        V, U = words(c["V"]), words(c["U"])
        s_in = torch.from_numpy(c["s_in"]).cuda().to(dtype)
        s_out = torch.from_numpy(c["s_out"]).cuda().to(dtype)
        s_mid = None if c["s_mid"] is None else torch.from_numpy(c["s_mid"]).cuda().to(dtype)
        keep += [V, U, s_in, s_out, s_mid]
        refs.append(torch.ops.binary_kernels.nanoquant_dyn_forward(
            x, s_in, V, s_mid, U, s_out, num_acc_stage1=1, num_acc_stage2=1))
        items.append(item(_lib, V, s_in, s_mid, U, s_out, yg, off, width, None, r, m))
        off += m
    group_call(lib, _lib.dtype_code(dtype), items, x, batch, n, -1.0, _lib.NQ_EPI_STORE)
    off = 0
    for (m, _), ref in zip(shapes, refs):
        got = yg[:, off:off + m]
        assert torch.equal(got.contiguous().view(torch.int16), ref.view(torch.int16)), (m, off)
        off += m


def rel(y, y64):
    y = y.float().cpu().numpy().astype(np.float64)
    return float(np.abs(y - y64).max() / np.abs(y64).max())


# n = 512: VALU stage 1 for 1-4 rows (2-4 rows decoding each sign word once for all of them), MFMA
# stage 1 from 5; n = 20000 (625-word rows): the VALU shape with four words per lane over four waves
# at one row, the MFMA stage 1 from 2; n = 32768 (1024-word rows): the same, the MFMA stage 1 with
# its tile of V at the unpadded stride
@pytest.mark.parametrize("n", [512, 20000, 32768])
@pytest.mark.parametrize("batch", [1, 2, 4, 5, 18])
def test_group_norm_and_residual(lib, batch, n):
    from nanoquant_amd import _lib
    announce("group norm + residual", batch, n)
    m, r, eps = 320, 160, 1e-5
    c = make_linear(21, m, n, r, with_mid=True)
    rng = np.random.default_rng(5)
    x = (rng.normal(size=(batch, n)) * 3.0).astype(np.float16)
    w = np.abs(rng.normal(1.0, 0.3, n)).astype(np.float16)
    s_in_folded = (c["s_in"].astype(np.float32) * w.astype(np.float32)).astype(np.float16)
    resid = rng.normal(size=(batch, m)).astype(np.float16)
    V, U = words(c["V"]), words(c["U"])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    s_in, s_mid, s_out, xg, rg = t(s_in_folded), t(c["s_mid"]), t(c["s_out"]), t(x), t(resid)
    y = torch.zeros(batch, m, dtype=torch.float16, device="cuda")
    it = item(_lib, V, s_in, s_mid, U, s_out, y, 0, m, rg, r, m)
    group_call(lib, _lib.NQ_F16, [it], xg, batch, n, eps, _lib.NQ_EPI_RESIDUAL)
    x64 = x.astype(np.float64)
    rstd = 1.0 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps)
    lin = O.nanoquant_forward_f64(x64 * rstd, s_in_folded, c["V"], c["s_mid"], c["U"], c["s_out"])
    err = rel(y, resid.astype(np.float64) + lin)
    print(f"[fused] norm+residual rel err {err:.3e}", flush=True)
    assert err <= 1e-3, err
    # in place: y is also the residual
    y2 = rg.clone()
    it2 = item(_lib, V, s_in, s_mid, U, s_out, y2, 0, m, y2, r, m)
    group_call(lib, _lib.NQ_F16, [it2], xg, batch, n, eps, _lib.NQ_EPI_RESIDUAL)
    assert torch.equal(y2, y)


def test_group_gated(lib):
    from nanoquant_amd import _lib
    announce("group gated")
    batch, n, m, r = 2, 256, 448, 96
    cg, cu = make_linear(31, m, n, r), make_linear(32, m, n, r)
    for c in (cg, cu):  # gate and up of order 10, so that silu(gate) * up stays inside fp16
        c["s_out"] = (c["s_out"].astype(np.float32) / 16).astype(np.float16)
    x = torch.from_numpy(np.random.default_rng(7).normal(size=(batch, n)).astype(np.float16)).cuda()
    keep, its = [], []
    act = torch.zeros(batch, m, dtype=torch.float16, device="cuda")
    for c in (cg, cu):
        V, U = words(c["V"]), words(c["U"])
        s_in, s_out = torch.from_numpy(c["s_in"]).cuda(), torch.from_numpy(c["s_out"]).cuda()
        keep += [V, U, s_in, s_out]
        its.append(item(_lib, V, s_in, None, U, s_out, act, 0, m, None, r, m))
    group_call(lib, _lib.NQ_F16, its, x, batch, n, -1.0, _lib.NQ_EPI_GATED)
    x64 = x.double().cpu().numpy()
    g = O.nanoquant_forward_f64(x64, cg["s_in"], cg["V"], None, cg["U"], cg["s_out"])
    u = O.nanoquant_forward_f64(x64, cu["s_in"], cu["V"], None, cu["U"], cu["s_out"])
    want = g / (1.0 + np.exp(-g)) * u
    err = rel(act, want)
    print(f"[fused] gated rel err {err:.3e}", flush=True)
    assert err <= 2e-3, err


def test_group_argument_errors(lib):
    from nanoquant_amd import _lib
    arr = (_lib.GemvItem * 3)()
    for it in arr:
        it.r, it.m, it.y_stride = 32, 64, 64
    ws = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    assert lib.nq_gemv_group_stage2(0, 3, arr, 1, _lib.NQ_EPI_GATED, ws.data_ptr(), ws.numel(), None) == \
        _lib.NQ_ERR_SHAPE
    assert lib.nq_gemv_group_stage1(0, 0, arr, None, 1, 64, -1.0, ws.data_ptr(), ws.numel(), None) == \
        _lib.NQ_ERR_INVALID_ARGUMENT


# --------------------------------------------------------------------------- attention

def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


@pytest.mark.parametrize("G", [1, 2, 4, 8])
@pytest.mark.parametrize("pos", [0, 17, 63, 64, 130, 199])
def test_attention_decode(lib, G, pos):
    from nanoquant_amd import _lib
    announce("attention", G, pos)
    B, KV, D, L = 2, 2, 128, 200
    H = KV * G
    gen = torch.Generator().manual_seed(100 * G + pos)
    qkv = torch.randn(B, (H + 2 * KV) * D, generator=gen).half()
    kc = torch.randn(B, KV, L, D, generator=gen).half()
    vc = torch.randn(B, KV, L, D, generator=gen).half()
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2).float() / D))
    fr = torch.arange(L).float().view(-1, 1) * inv.view(1, -1)
    emb = torch.cat((fr, fr), dim=-1)
    cos, sin = emb.cos().half(), emb.sin().half()
    d_qkv, d_kc, d_vc = qkv.cuda(), kc.clone().cuda(), vc.clone().cuda()
    d_cos, d_sin = cos.cuda(), sin.cuda()
    d_pos = torch.tensor([pos], dtype=torch.int64, device="cuda")
    out = torch.zeros(B, H * D, dtype=torch.float16, device="cuda")
    W = (H + 2 * KV) * D
    p0 = d_qkv.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(lib.nq_attention_decode_workspace_bytes(B, H, KV, D, L), dtype=torch.uint8, device="cuda")
    _lib.check(lib.nq_attention_decode(_lib.NQ_F16, p0, p0 + 2 * H * D, p0 + 2 * (H + KV) * D, W, d_kc.data_ptr(),
                                       d_vc.data_ptr(), d_cos.data_ptr(), d_sin.data_ptr(), d_pos.data_ptr(),
                                       out.data_ptr(), B, H, KV, D, L, D ** -0.5, ws.data_ptr(), ws.numel(), st),
               "attention")
    torch.cuda.synchronize()
    q = qkv[:, :H * D].view(B, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(B, KV, D)
    v = qkv[:, (H + KV) * D:].view(B, KV, D)
    # the cache rows: rotary arithmetic in fp16 as torch rounds it
    k_rot = (k * cos[pos]) + (rotate_half(k) * sin[pos])
    got_kc, got_vc = d_kc.cpu(), d_vc.cpu()
    assert torch.equal(got_kc[:, :, pos].view(torch.int16), k_rot.view(torch.int16))
    assert torch.equal(got_vc[:, :, pos], v)
    others = [j for j in range(L) if j != pos]
    assert torch.equal(got_kc[:, :, others], kc[:, :, others])
    assert torch.equal(got_vc[:, :, others], vc[:, :, others])
    # attention in float64 over positions 0..pos
    q_rot = ((q * cos[pos]) + (rotate_half(q) * sin[pos])).double()
    keys = got_kc[:, :, :pos + 1].double()  # [B, KV, P, D]
    vals = got_vc[:, :, :pos + 1].double()
    kk = keys.repeat_interleave(G, dim=1)
    vv = vals.repeat_interleave(G, dim=1)
    s = torch.einsum("bhd,bhpd->bhp", q_rot, kk) * D ** -0.5
    p = torch.softmax(s, dim=-1)
    want = torch.einsum("bhp,bhpd->bhd", p, vv).reshape(B, H * D).numpy()
    err = rel(out, want)
    assert err <= 2e-3, err


def test_attention_position_outside_cache(lib):
    from nanoquant_amd import _lib
    announce("attention position outside")
    B, KV, H, D, L = 1, 2, 2, 128, 16
    qkv = torch.randn(B, (H + 2 * KV) * D, device="cuda").half()
    kc = torch.randn(B, KV, L, D, device="cuda").half()
    vc = torch.randn(B, KV, L, D, device="cuda").half()
    kc0, vc0 = kc.clone(), vc.clone()
    cs = torch.ones(L, D, device="cuda").half()
    out = torch.ones(B, H * D, dtype=torch.float16, device="cuda")
    ws = torch.zeros(lib.nq_attention_decode_workspace_bytes(B, H, KV, D, L), dtype=torch.uint8, device="cuda")
    W = (H + 2 * KV) * D
    p0 = qkv.data_ptr()
    for bad in (L, -1):
        d_pos = torch.tensor([bad], dtype=torch.int64, device="cuda")
        _lib.check(lib.nq_attention_decode(_lib.NQ_F16, p0, p0 + 2 * H * D, p0 + 2 * (H + KV) * D, W,
                                           kc.data_ptr(), vc.data_ptr(), cs.data_ptr(), cs.data_ptr(),
                                           d_pos.data_ptr(), out.data_ptr(), B, H, KV, D, L, 0.1, ws.data_ptr(),
                                           ws.numel(), None), "attn")
        torch.cuda.synchronize()
        assert torch.equal(kc, kc0) and torch.equal(vc, vc0)
        assert torch.count_nonzero(out) == 0
    assert lib.nq_attention_decode(_lib.NQ_F16, p0, p0, p0, W, kc.data_ptr(), vc.data_ptr(), cs.data_ptr(),
                                   cs.data_ptr(), d_pos.data_ptr(), out.data_ptr(), B, H, KV, 64, L, 0.1,
                                   ws.data_ptr(), ws.numel(), None) == _lib.NQ_ERR_UNSUPPORTED
    assert lib.nq_attention_decode(_lib.NQ_F16, p0, p0, p0, W, kc.data_ptr(), vc.data_ptr(), cs.data_ptr(),
                                   cs.data_ptr(), d_pos.data_ptr(), out.data_ptr(), B, H, KV, D, L, 0.1,
                                   ws.data_ptr(), 16, None) == _lib.NQ_ERR_WORKSPACE


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("B,heads,kv_heads,D,r_qkv,pos", [(1, 4, 4, 128, (96, 96, 96), 37), (2, 8, 2, 128, (160, 96, 96), 0),
                                                          (3, 4, 1, 64, (64, 64, 64), 63), (1, 2, 2, 64, (96, 96, 96), 80)])
def test_group_stage2_rope_equals_store_then_rope_kernel(lib, dtype, B, heads, kv_heads, D, r_qkv, pos):
    """nq_gemv_group_stage2_rope (the q/k/v stage 2 with the rotary embedding and cache write in its
    store) against nq_gemv_group_stage2 (NQ_EPI_STORE) followed by nq_rope_kv_write on the same
    intermediate: q, the caches' new rows and every other cache row bit for bit; ranks equal and
    unequal (two launches); a position past the cache (80 of 64 rows) zeroes q and writes no row. The
    scores buffer it is given holds the step's causal mask afterwards (0 up to the position, -inf
    after; all visible past the cache)."""
    from nanoquant_amd import _lib
    announce("group stage 2 rope", dtype, (B, heads, kv_heads, D, r_qkv, pos))
    n, L = 256, 64
    ms = (heads * D, kv_heads * D, kv_heads * D)
    width = sum(ms)
    rng = np.random.default_rng(B * 100 + heads + pos)
    x = torch.from_numpy((rng.normal(size=(B, n)) * 2.0).astype(np.float16)).cuda().to(dtype)
    keep, its_store, its_rope = [], [], []
    qkv = torch.zeros(B, width, dtype=dtype, device="cuda")
    q_rot = torch.full((B, heads * D), 3.0, dtype=dtype, device="cuda")
    off = 0
    for i, (m, r) in enumerate(zip(ms, r_qkv)):
        c = make_linear(70 + i, m, n, r, with_mid=(i == 2))
        V, U = words(c["V"]), words(c["U"])
        s_in = torch.from_numpy(c["s_in"]).cuda().to(dtype)
        s_out = torch.from_numpy(c["s_out"]).cuda().to(dtype)
        s_mid = None if c["s_mid"] is None else torch.from_numpy(c["s_mid"]).cuda().to(dtype)
        keep += [V, U, s_in, s_out, s_mid]
        its_store.append(item(_lib, V, s_in, s_mid, U, s_out, qkv, off, width, None, r, m))
        its_rope.append(item(_lib, V, s_in, s_mid, U, s_out, q_rot if i == 0 else qkv, 0,
                             heads * D if i == 0 else width, None, r, m))
        off += m
    gen = torch.Generator(device="cuda").manual_seed(pos)
    caches = [torch.randn(B, kv_heads, L, D, device="cuda", generator=gen).to(dtype) for _ in range(2)]
    caches_ref = [t.clone() for t in caches]
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device="cuda").float() / D))
    emb = torch.arange(L, device="cuda").float()[:, None] * inv[None, :]
    emb = torch.cat((emb, emb), dim=-1)
    cos, sin = emb.cos().to(dtype).contiguous(), emb.sin().to(dtype).contiguous()
    position = torch.tensor([pos], dtype=torch.int64, device="cuda")
    dc = _lib.dtype_code(dtype)
    st = torch.cuda.current_stream().cuda_stream
    arr_s = (_lib.GemvItem * 3)(*its_store)
    arr_r = (_lib.GemvItem * 3)(*its_rope)
    need = lib.nq_gemv_group_workspace_bytes(3, arr_s, B)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    # reference: stage 1, stage 2 with plain stores, then the rotary kernel
    _lib.check(lib.nq_gemv_group_stage1(dc, 3, arr_s, x.data_ptr(), B, n, -1.0, ws.data_ptr(), need, st), "s1")
    _lib.check(lib.nq_gemv_group_stage2(dc, 3, arr_s, B, _lib.NQ_EPI_STORE, ws.data_ptr(), need, st), "s2")
    q_ref = torch.full_like(q_rot, 3.0)
    _lib.check(lib.nq_rope_kv_write(dc, qkv.data_ptr(), width, caches_ref[0].data_ptr(), caches_ref[1].data_ptr(),
                                    cos.data_ptr(), sin.data_ptr(), position.data_ptr(), q_ref.data_ptr(),
                                    heads * D, B, heads, kv_heads, D, L, st), "rope")
    # fused: the same intermediate, stage 2 with the rotary store
    # the scores buffer of the step's attention, which the launch fills with the causal mask
    scores = torch.full((B * kv_heads, L, heads // kv_heads), 7.0, dtype=dtype, device="cuda")
    _lib.check(lib.nq_gemv_group_stage2_rope(dc, arr_r, B, caches[0].data_ptr(), caches[1].data_ptr(),
                                             cos.data_ptr(), sin.data_ptr(), position.data_ptr(), D, L,
                                             scores.data_ptr(), ws.data_ptr(), need, st), "s2 rope")
    torch.cuda.synchronize()
    visible = (torch.arange(L, device="cuda") <= pos).view(1, L, 1).expand_as(scores)
    want_mask = torch.zeros_like(scores).masked_fill_(~visible, float("-inf"))
    assert torch.equal(scores.view(torch.int16), want_mask.view(torch.int16))
    assert torch.equal(q_rot.view(torch.int16), q_ref.view(torch.int16))
    assert torch.equal(caches[0].view(torch.int16), caches_ref[0].view(torch.int16))
    assert torch.equal(caches[1].view(torch.int16), caches_ref[1].view(torch.int16))
    if pos >= L:
        assert torch.equal(q_rot, torch.zeros_like(q_rot))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("B,heads,kv_heads,D,r_qkv,pos", [(1, 4, 4, 128, (96, 96, 96), 37), (2, 8, 2, 128, (160, 96, 96), 0),
                                                          (3, 4, 1, 64, (64, 64, 64), 63), (1, 2, 2, 64, (96, 96, 96), 80)])
def test_group_stage2_kv_equals_store_then_value_copy(lib, dtype, B, heads, kv_heads, D, r_qkv, pos):
    """nq_gemv_group_stage2_kv (the q/k/v stage 2 storing q and k, and copying v into its cache row)
    against nq_gemv_group_stage2 (NQ_EPI_STORE) on the same intermediate: q and k bit for bit, the
    value cache's row at the position equal to the stored v, every other cache row and v's own
    output untouched; ranks equal and unequal (two launches); a position past the cache (80 of 64
    rows) writes no row."""
    from nanoquant_amd import _lib
    announce("group stage 2 kv", dtype, (B, heads, kv_heads, D, r_qkv, pos))
    n, L = 256, 64
    ms = (heads * D, kv_heads * D, kv_heads * D)
    width = sum(ms)
    rng = np.random.default_rng(B * 100 + heads + pos + 1)
    x = torch.from_numpy((rng.normal(size=(B, n)) * 2.0).astype(np.float16)).cuda().to(dtype)
    keep, its = [], []
    ref = torch.zeros(B, width, dtype=dtype, device="cuda")
    got = torch.full((B, width), 5.0, dtype=dtype, device="cuda")
    off = 0
    for i, (m, r) in enumerate(zip(ms, r_qkv)):
        c = make_linear(80 + i, m, n, r, with_mid=(i == 1))
        V, U = words(c["V"]), words(c["U"])
        s_in = torch.from_numpy(c["s_in"]).cuda().to(dtype)
        s_out = torch.from_numpy(c["s_out"]).cuda().to(dtype)
        s_mid = None if c["s_mid"] is None else torch.from_numpy(c["s_mid"]).cuda().to(dtype)
        keep += [V, U, s_in, s_out, s_mid]
        its.append((V, s_in, s_mid, U, s_out, off, r, m))
        off += m
    arr_ref = (_lib.GemvItem * 3)(*[item(_lib, V, si, sm, U, so, ref, o, width, None, r, m)
                                    for V, si, sm, U, so, o, r, m in its])
    arr_kv = (_lib.GemvItem * 3)(*[item(_lib, V, si, sm, U, so, got, o, width, None, r, m)
                                   for V, si, sm, U, so, o, r, m in its])
    gen = torch.Generator(device="cuda").manual_seed(pos + 1)
    v_cache = torch.randn(B, kv_heads, L, D, device="cuda", generator=gen).to(dtype)
    v_ref = v_cache.clone()
    position = torch.tensor([pos], dtype=torch.int64, device="cuda")
    dc = _lib.dtype_code(dtype)
    st = torch.cuda.current_stream().cuda_stream
    need = lib.nq_gemv_group_workspace_bytes(3, arr_ref, B)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    _lib.check(lib.nq_gemv_group_stage1(dc, 3, arr_ref, x.data_ptr(), B, n, -1.0, ws.data_ptr(), need, st), "s1")
    _lib.check(lib.nq_gemv_group_stage2(dc, 3, arr_ref, B, _lib.NQ_EPI_STORE, ws.data_ptr(), need, st), "s2")
    _lib.check(lib.nq_gemv_group_stage2_kv(dc, arr_kv, B, v_cache.data_ptr(), position.data_ptr(), D, L,
                                           ws.data_ptr(), need, st), "s2 kv")
    torch.cuda.synchronize()
    qk = ms[0] + ms[1]
    assert torch.equal(got[:, :qk].view(torch.int16), ref[:, :qk].view(torch.int16))
    assert torch.equal(got[:, qk:], torch.full_like(got[:, qk:], 5.0))  # v's own output is not written
    if pos < L:
        v_ref[:, :, pos, :] = ref[:, qk:].view(B, kv_heads, D)
    assert torch.equal(v_cache.view(torch.int16), v_ref.view(torch.int16))


def test_group_stage2_kv_argument_errors(lib):
    from nanoquant_amd import _lib
    announce("group stage 2 kv errors")
    t = torch.zeros(64, dtype=torch.int32, device="cuda")
    it = _lib.GemvItem()
    it.v_bits = it.u_bits = it.s_in = it.s_out = it.y = t.data_ptr()
    it.r, it.m, it.y_stride = 32, 100, 100
    arr = (_lib.GemvItem * 3)(it, it, it)
    pos = torch.zeros(1, dtype=torch.int64, device="cuda")
    assert lib.nq_gemv_group_stage2_kv(_lib.NQ_F16, arr, 1, t.data_ptr(), pos.data_ptr(), 64, 8, t.data_ptr(), 256,
                                       None) == _lib.NQ_ERR_SHAPE  # m = 100 is not whole heads of 64
    assert lib.nq_gemv_group_stage2_kv(_lib.NQ_F16, arr, 1, t.data_ptr(), pos.data_ptr(), 24, 8, t.data_ptr(), 256,
                                       None) == _lib.NQ_ERR_INVALID_ARGUMENT  # head_dim not a multiple of 16
    assert lib.nq_gemv_group_stage2_kv(_lib.NQ_F16, None, 1, t.data_ptr(), pos.data_ptr(), 64, 8, t.data_ptr(), 256,
                                       None) == _lib.NQ_ERR_INVALID_ARGUMENT


def half_ulp(v, bits):
    """Half a unit in the last place of |v| for a float of `bits` significant bits."""
    _, e = np.frexp(np.abs(v))
    return np.ldexp(1.0, e - 1 - bits)


DENSE_CASES = [  # m, n, batch, ldy
    (32000, 4096, 1, 32000),  # the Llama-2-7B lm_head
    (7, 8, 3, 7),             # one 16-byte chunk per row, a ragged block of rows
    (1000, 4104, 5, 1000),    # a second, nearly empty 4096-column group; batch past one 4-row pass
    (513, 8200, 2, 600),      # output rows wider than m (the gap is not written)
    (64, 12288, 4, 64),       # three column groups; two batch rows per block (LDS)
]


def dense_call(lib, dtype, w, x, g, eps, y, y_f32, batch, n, m, ldy):
    from nanoquant_amd import _lib
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.nq_dense_gemv(_lib.dtype_code(dtype), w.data_ptr(), x.data_ptr(), None if g is None else g.data_ptr(),
                                 eps, y.data_ptr(), int(y_f32), batch, n, m, ldy, st), "dense gemv")
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("m,n,batch,ldy", DENSE_CASES)
@pytest.mark.parametrize("norm", [False, True], ids=["plain", "rmsnorm"])
def test_dense_gemv_against_fp32(lib, dtype, m, n, batch, ldy, norm):
    """nq_dense_gemv against a float64 product of the same dtype inputs: each output within half a
    unit in the last place of the rounded exact value plus 1e-5 of the largest output (fp32
    summation order); with the norm prologue the input is the decoder's RMSNorm of x computed by
    torch (an element of it may differ by a unit in the last place: the mean's summation order),
    bar 5e-5. float32 outputs (norm cases) hold the dtype-rounded values exactly; the padding of y
    past m is untouched."""
    announce("dense gemv", dtype, (m, n, batch, ldy), "norm" if norm else "")
    gen = torch.Generator(device="cuda").manual_seed(m + n + batch)
    w = (torch.randn(m, n, device="cuda", generator=gen) * 0.05).to(dtype)
    x = (torch.randn(batch, n, device="cuda", generator=gen) * 3.0).to(dtype)
    g = (torch.rand(n, device="cuda", generator=gen) + 0.5).to(dtype) if norm else None
    eps = 1e-5
    y_f32 = norm  # the decode step's use: norm folded in, float32 logits
    y = torch.full((batch, ldy), 9.0, dtype=torch.float32 if y_f32 else dtype, device="cuda")
    dense_call(lib, dtype, w, x, g, eps, y, y_f32, batch, n, m, ldy)
    xin = (g * torch.nn.functional.rms_norm(x.float(), (n,), eps=eps).to(dtype)) if norm else x
    ref = (xin.double().cpu() @ w.double().cpu().T).numpy()
    got = y[:, :m].double().cpu().numpy()
    if y_f32:  # float32 outputs carry values already rounded to dtype
        assert torch.equal(y[:, :m].to(dtype).float(), y[:, :m])
    bits = 11 if dtype == torch.float16 else 8
    # half a unit of the rounded value's binade (the larger one where rounding carried into the next)
    allowed = np.maximum(half_ulp(ref, bits), half_ulp(got, bits))
    excess = np.maximum(np.abs(got - ref) - allowed, 0.0).max() / np.abs(ref).max()
    print(f"[dense] {dtype} {(m, n, batch)} norm={norm} excess={excess:.2e}", flush=True)
    assert excess <= (5e-5 if norm else 1e-5), excess
    if ldy > m:
        assert torch.equal(y[:, m:], torch.full_like(y[:, m:], 9.0))


def test_dense_gemv_argument_errors(lib):
    from nanoquant_amd import _lib
    announce("dense gemv errors")
    w = torch.zeros(16, 64, dtype=torch.float16, device="cuda")
    x = torch.zeros(2, 64, dtype=torch.float16, device="cuda")
    y = torch.zeros(2, 16, dtype=torch.float16, device="cuda")
    f = lib.nq_dense_gemv
    F16 = _lib.NQ_F16
    wp, xp, yp = w.data_ptr(), x.data_ptr(), y.data_ptr()
    assert f(F16, wp, xp, None, 0.0, yp, 0, 2, 60, 16, 16, None) == _lib.NQ_ERR_SHAPE
    assert f(F16, wp + 2, xp, None, 0.0, yp, 0, 2, 64, 15, 16, None) == _lib.NQ_ERR_ALIGNMENT
    assert f(F16, wp, xp, xp + 2, 0.0, yp, 0, 2, 64, 16, 16, None) == _lib.NQ_ERR_ALIGNMENT  # norm weight
    assert f(F16, wp, xp, None, 0.0, yp + 2, 1, 2, 64, 16, 16, None) == _lib.NQ_ERR_ALIGNMENT  # float32 y
    assert f(F16, wp, xp, None, 0.0, yp, 0, 2, 64, 16, 15, None) == _lib.NQ_ERR_INVALID_ARGUMENT
    assert f(F16, wp, xp, None, 0.0, yp, 0, 2, 40000, 16, 16, None) == _lib.NQ_ERR_UNSUPPORTED  # n past the LDS
    assert f(7, wp, xp, None, 0.0, yp, 0, 2, 64, 16, 16, None) == _lib.NQ_ERR_DTYPE
    assert f(F16, None, None, None, 0.0, None, 0, 0, 64, 16, 16, None) == _lib.NQ_OK  # empty batch


@pytest.mark.parametrize("rows,n,ldx", [(1, 32000, 32000), (4, 32000, 32000), (3, 1000, 1024), (2, 1, 1),
                                        (5, 128256, 128256), (3, 1001, 1001)])
def test_argmax_rows_is_torch_argmax(lib, rows, n, ldx):
    """The decode step's greedy choice: the same index as torch.argmax on every row, including
    repeated maxima (the first wins), NaNs (the first NaN wins), rows of -inf only, and rows read
    at a stride larger than their length."""
    from nanoquant_amd import _lib
    announce("argmax rows", rows, n, ldx)
    g = torch.Generator(device="cuda").manual_seed(rows * 7 + n)
    x = torch.randn(rows, ldx, generator=g, device="cuda", dtype=torch.float32)
    x[:, n:] = 1e30  # past the row: never read
    if n > 8:
        x[0, n // 3] = x[0, n - 2] = x[0, :n].max() + 1.0  # a repeated maximum: the first one
    if rows > 1 and n > 4:
        x[1, n - 3] = float("nan")
        x[1, n // 2] = float("nan")  # two NaNs: the first one
    if rows > 2:
        x[2, :n] = float("-inf")  # index 0
    out = torch.full((rows,), -1, dtype=torch.int64, device="cuda")
    st = lib.nq_argmax_rows(x.data_ptr(), rows, n, ldx, out.data_ptr(), _lib.stream_of(x.device))
    assert st == 0
    torch.cuda.synchronize()
    want = torch.argmax(x[:, :n], dim=-1)
    assert torch.equal(out, want), (out.tolist(), want.tolist())


def test_argmax_rows_argument_errors(lib):
    from nanoquant_amd import _lib
    announce("argmax rows errors")
    x = torch.zeros(2, 64, dtype=torch.float32, device="cuda")
    out = torch.zeros(2, dtype=torch.int64, device="cuda")
    f = lib.nq_argmax_rows
    xp, op = x.data_ptr(), out.data_ptr()
    assert f(xp, 2, 0, 64, op, None) == _lib.NQ_ERR_INVALID_ARGUMENT  # no logits
    assert f(xp, 2, 64, 32, op, None) == _lib.NQ_ERR_INVALID_ARGUMENT  # stride shorter than a row
    assert f(xp + 2, 2, 62, 64, op, None) == _lib.NQ_ERR_ALIGNMENT
    assert f(xp, 2, 64, 64, op + 4, None) == _lib.NQ_ERR_ALIGNMENT
    assert f(None, 2, 64, 64, op, None) == _lib.NQ_ERR_INVALID_ARGUMENT
    assert f(None, 0, 64, 64, None, None) == _lib.NQ_OK  # no rows
