"""End-to-end greedy decode on the GPU: a small Llama-architecture model whose linears run
the HIP GEMV (or GEMM) kernels, stepped from a HIP graph, against the same model in its
dense fp32 reference state on the CPU (``linear.py:282-291`` for every linear).

Bars (written here):
* graph replay and eager stepping of the kernel model give identical tokens and logits;
* logits of every decode position, teacher-forced on the generated sequence, within
  max|l - l*| / max|l*| <= 2e-2 of the fp32 reference (fp16 activations through every
  layer; each linear alone meets 1e-3);
* each greedy token equals the reference argmax wherever the reference's top-2 margin
  exceeds twice the measured logit error.
"""
import copy
import sys

import pytest
import torch

from nanoquant_amd.decode import GraphDecoder, LlamaShape, random_llama

pytestmark = pytest.mark.gpu

SHAPE = LlamaShape(hidden=256, layers=2, heads=4, kv_heads=2, ffn=512, vocab=1000)
E2E_TOL = 2e-2
E2E_TOL_BF16 = 1e-1  # bfloat16 keeps 8 significant bits against float16's 11


def announce(*what):
    print("\n[case]", *what, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def models():
    from nanoquant_amd import _lib
    _lib.load()
    dense = random_llama(SHAPE, bpw=0.55, seed=11, device="cpu", with_mid=True)
    return dense


def kernel_model(dense, kernel_type, dtype=torch.float16):
    return copy.deepcopy(dense).to("cuda").prepare_kernels(kernel_type, dtype)


def run(model, prompt, new, use_graph, steps_per_graph=1):
    B, T = prompt.shape
    dec = GraphDecoder(model, B, T + new, steps_per_graph=steps_per_graph)
    if use_graph:
        dec.capture()
    logits = [dec.prefill(prompt.cuda()).clone()]
    if use_graph:
        # one replay per graph; the captured logits buffer holds the last step of each replay
        for _ in range((new - 1) // steps_per_graph):
            dec.decode(steps_per_graph, use_graph=True)
            logits.append(dec.last_logits.clone())
    else:
        for _ in range(new - 1):
            logits.append(dec.decode(1, use_graph=False).clone())
    torch.cuda.synchronize()
    return dec.ids[:, :T + new].cpu(), [lg.cpu() for lg in logits]


def check_against_dense(dense, ids, logits, T, every=1, tol=E2E_TOL):
    with torch.no_grad():
        ref = dense(ids[:, :-1], torch.arange(ids.shape[1] - 1), _cache_for(dense, ids)).double()
    worst = 0.0
    for j, lg in enumerate(logits):
        pos = T - 1 + j * every
        r = ref[:, pos]
        err = float((lg.double() - r).abs().max() / r.abs().max())
        worst = max(worst, err)
        top2 = r.topk(2, dim=-1).values
        sure = (top2[:, 0] - top2[:, 1]) > 2 * err * r.abs().max()
        got = ids[:, pos + 1]
        assert torch.equal(got[sure], r.argmax(-1)[sure]), (j, got, r.argmax(-1))
    print(f"[decode] worst logits rel err {worst:.3e}", flush=True)
    assert worst <= tol, worst


def _cache_for(model, ids):
    from nanoquant_amd.decode import StaticKVCache
    return StaticKVCache(model.shape, ids.shape[0], ids.shape[1], "cpu", torch.float32)


def test_graph_decode_matches_eager_and_dense(models):
    announce("decode gemv graph vs eager vs dense", SHAPE)
    dense = models
    model = kernel_model(dense, "gemv")
    prompt = torch.randint(0, SHAPE.vocab, (2, 16), generator=torch.Generator().manual_seed(4))
    new = 9
    ids_g, lg_g = run(model, prompt, new, use_graph=True)
    ids_e, lg_e = run(model, prompt, new, use_graph=False)
    assert torch.equal(ids_g, ids_e)
    for a, b in zip(lg_g, lg_e):
        assert torch.equal(a, b)
    check_against_dense(dense, ids_g, lg_g, prompt.shape[1])


def test_multi_step_graph(models):
    announce("decode gemv, 4 steps per graph", SHAPE)
    model = kernel_model(models, "gemv")
    prompt = torch.randint(0, SHAPE.vocab, (1, 10), generator=torch.Generator().manual_seed(6))
    ids4, lg4 = run(model, prompt, 9, use_graph=True, steps_per_graph=4)
    ids1, _ = run(model, prompt, 9, use_graph=False)
    assert torch.equal(ids4, ids1)
    check_against_dense(models, ids4, lg4, prompt.shape[1], every=4)


def test_gemm_kernel_decode(models):
    announce("decode gemm eager", SHAPE)
    model = kernel_model(models, "gemm")
    prompt = torch.randint(0, SHAPE.vocab, (3, 12), generator=torch.Generator().manual_seed(8))
    ids, lg = run(model, prompt, 5, use_graph=False)
    check_against_dense(models, ids, lg, prompt.shape[1])


# --------------------------------------------------------------------------- fused decode step

FUSED_SHAPES = {
    "gqa": LlamaShape(hidden=512, layers=2, heads=4, kv_heads=2, ffn=1024, vocab=1000),
    "mha": LlamaShape(hidden=512, layers=2, heads=4, kv_heads=4, ffn=768, vocab=1000),
}


def run_fused(model, prompt, new, use_graph, steps_per_graph=1, attention="torch"):
    from nanoquant_amd.decode import FusedDecoder
    B, T = prompt.shape
    dec = FusedDecoder(model, B, T + new, steps_per_graph=steps_per_graph, attention=attention)
    if use_graph:
        dec.capture()
    logits = [dec.prefill(prompt.cuda()).clone()]
    if use_graph:
        for _ in range((new - 1) // steps_per_graph):
            dec.decode(steps_per_graph, use_graph=True)
            logits.append(dec.last_logits.clone())
    else:
        for _ in range(new - 1):
            logits.append(dec.decode(1, use_graph=False).clone())
    torch.cuda.synchronize()
    return dec.ids[:, :T + new].cpu(), [lg.cpu() for lg in logits]


@pytest.mark.parametrize("attention", ["torch", "rope", "hip"])
@pytest.mark.parametrize("name", list(FUSED_SHAPES))
def test_fused_decode_matches_dense(name, attention):
    shape = FUSED_SHAPES[name]
    announce("fused decode", name, attention, shape)
    from nanoquant_amd import _lib
    _lib.load()
    dense = random_llama(shape, bpw=0.55, seed=13, device="cpu", with_mid=(name == "gqa"))
    with torch.no_grad():
        for layer in dense.model.layers:  # norm weights away from 1 so that the fold is exercised
            layer.input_layernorm.weight.uniform_(0.5, 1.5)
            layer.post_attention_layernorm.weight.uniform_(0.5, 1.5)
    model = kernel_model(dense, "gemv")
    prompt = torch.randint(0, shape.vocab, (2, 12), generator=torch.Generator().manual_seed(3))
    new = 9
    ids_g, lg_g = run_fused(model, prompt, new, use_graph=True, steps_per_graph=2, attention=attention)
    ids_e, lg_e = run_fused(model, prompt, new, use_graph=False, attention=attention)
    assert torch.equal(ids_g, ids_e)
    for j, (a, b) in enumerate(zip(lg_g, lg_e[::2])):
        assert torch.equal(a, b), j
    check_against_dense(dense, ids_e, lg_e, prompt.shape[1])


@pytest.mark.parametrize("name", list(FUSED_SHAPES))
def test_fused_torch_decode_bf16(name):
    """The torch-attention fused step in bfloat16, where the rotary embedding stays the [D, D]
    product with the features in their natural order (torch has no complex bfloat16): graph equals
    eager, and the logits and greedy tokens follow the float32 dense model (bar E2E_TOL_BF16)."""
    shape = FUSED_SHAPES[name]
    announce("fused decode bf16", name, shape)
    from nanoquant_amd import _lib
    _lib.load()
    dense = random_llama(shape, bpw=0.55, seed=17, device="cpu", with_mid=(name == "gqa"))
    model = kernel_model(dense, "gemv", torch.bfloat16)
    prompt = torch.randint(0, shape.vocab, (2, 12), generator=torch.Generator().manual_seed(5))
    new = 7
    ids_g, lg_g = run_fused(model, prompt, new, use_graph=True, steps_per_graph=2)
    ids_e, lg_e = run_fused(model, prompt, new, use_graph=False)
    assert torch.equal(ids_g, ids_e)
    for j, (a, b) in enumerate(zip(lg_g, lg_e[::2])):
        assert torch.equal(a, b), j
    check_against_dense(dense, ids_e, lg_e, prompt.shape[1], tol=E2E_TOL_BF16)


@pytest.mark.parametrize("heads,kv_heads,pos", [(32, 32, 200), (8, 2, 77), (32, 32, 0)])
def test_attention_step_against_rotary_attention(heads, kv_heads, pos):
    """The decode step's attention (``rotary_attention_step``: RoPE as one [D, D] product, the scale
    and causal mask folded into ``baddbmm``, fp16 scores) against ``rotary_attention`` (elementwise
    RoPE, fp32 scores) on the same fp16 cache and inputs, one layer at a time: outputs within 2e-3
    of their largest magnitude and the written K/V rows within fp16 rounding of each other."""
    from nanoquant_amd.decode import StaticKVCache, rotary_attention, rotary_attention_step, rotary_step_tables
    shape = LlamaShape(hidden=heads * 128, layers=2, heads=heads, kv_heads=kv_heads, ffn=512, vocab=1000)
    announce("attention step vs rotary_attention", heads, kv_heads, pos)
    D, B, L = shape.head_dim, 1, 384
    gen = torch.Generator(device="cuda").manual_seed(pos + heads)
    caches = [StaticKVCache(shape, B, L, "cuda", torch.float16) for _ in range(2)]
    for layer in range(shape.layers):
        k0 = torch.randn(B, kv_heads, L, D, device="cuda", generator=gen).half()
        v0 = torch.randn(B, kv_heads, L, D, device="cuda", generator=gen).half()
        for c in caches:
            c.k[layer].copy_(k0)
            c.v[layer].copy_(v0)
    positions = torch.tensor([pos], device="cuda")
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device="cuda").float() / D))
    ang = positions.float()[:, None] * inv[None, :]
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos().half(), emb.sin().half()
    tables = rotary_step_tables(cos, sin, positions, caches[1], torch.float16)
    for layer in range(shape.layers):
        q = torch.randn(B, 1, heads * D, device="cuda", generator=gen).half()
        k = torch.randn(B, 1, kv_heads * D, device="cuda", generator=gen).half()
        v = torch.randn(B, 1, kv_heads * D, device="cuda", generator=gen).half()
        ref = rotary_attention(shape, layer, q, k, v, cos, sin, positions, caches[0]).double()
        qk = torch.cat((q, k), dim=-1).view(B, -1)
        got = rotary_attention_step(shape, layer, qk, v.view(B, -1), tables, positions, caches[1]).double()
        torch.cuda.synchronize()
        rel = float((got - ref).abs().max() / ref.abs().max())
        k_ref = caches[0].k[layer].double()
        k_rel = float((caches[1].k[layer].double() - k_ref).abs().max() / k_ref.abs().max())
        print(f"[decode] layer {layer} attention step rel {rel:.3e}, K write rel {k_rel:.3e}", flush=True)
        assert rel <= 2e-3, (layer, rel)
        assert torch.equal(caches[1].v[layer], caches[0].v[layer])
        assert k_rel <= 2e-3, (layer, k_rel)  # RoPE rounded once (product) against three times (elementwise)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("B,heads,kv_heads,D,pos", [(1, 32, 32, 128, 130), (2, 8, 2, 128, 0), (3, 4, 1, 64, 63),
                                                    (2, 4, 2, 128, 400)])
def test_rope_kv_write_against_torch(dtype, B, heads, kv_heads, D, pos):
    """nq_rope_kv_write against the elementwise torch rotary embedding (x * cos + rotate_half(x) *
    sin, each product and the sum rounded to the dtype, as rotary_attention runs it) and the cache
    rows torch's index_copy_ writes: bit for bit, every other cache row untouched; a position past
    the cache (pos = 400 with 384 rows) zeroes q and writes no row."""
    from nanoquant_amd import _lib
    from nanoquant_amd.decode import _rotate_half
    lib = _lib.load()
    announce("rope kv write", dtype, (B, heads, kv_heads, D, pos))
    L = 384
    gen = torch.Generator(device="cuda").manual_seed(B * 1000 + heads + pos)
    width = (heads + 2 * kv_heads) * D + 8  # a padded row
    qkv = (torch.randn(B, width, device="cuda", generator=gen) * 2).to(dtype)
    k_cache = torch.randn(B, kv_heads, L, D, device="cuda", generator=gen).to(dtype)
    v_cache = torch.randn(B, kv_heads, L, D, device="cuda", generator=gen).to(dtype)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device="cuda").float() / D))
    ang = torch.arange(L, device="cuda").float()[:, None] * inv[None, :]
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos().to(dtype).contiguous(), emb.sin().to(dtype).contiguous()
    position = torch.tensor([pos], device="cuda", dtype=torch.int64)
    q_out = torch.full((B, heads * D), 7.0, device="cuda", dtype=dtype)
    k0, v0 = k_cache.clone(), v_cache.clone()
    _lib.check(lib.nq_rope_kv_write(_lib.dtype_code(dtype), qkv.data_ptr(), width, k_cache.data_ptr(),
                                    v_cache.data_ptr(), cos.data_ptr(), sin.data_ptr(), position.data_ptr(),
                                    q_out.data_ptr(), heads * D, B, heads, kv_heads, D, L,
                                    torch.cuda.current_stream().cuda_stream), "rope")
    torch.cuda.synchronize()
    if pos >= L:
        assert torch.equal(q_out, torch.zeros_like(q_out))
        assert torch.equal(k_cache, k0) and torch.equal(v_cache, v0)
        return
    c, s_ = cos[pos], sin[pos]
    q = qkv[:, :heads * D].reshape(B, heads, D)
    k = qkv[:, heads * D:(heads + kv_heads) * D].reshape(B, kv_heads, D)
    v = qkv[:, (heads + kv_heads) * D:(heads + 2 * kv_heads) * D].reshape(B, kv_heads, D)
    q_ref = q * c + _rotate_half(q) * s_
    k_ref = k * c + _rotate_half(k) * s_
    assert torch.equal(q_out.view(B, heads, D), q_ref)
    k0[:, :, pos] = k_ref
    v0[:, :, pos] = v
    assert torch.equal(k_cache, k0)
    assert torch.equal(v_cache, v0)
