"""Greedy decode of a Llama-2-architecture model whose seven linears per layer are
``NanoQuantLinear``, with the one-token step replayed from a HIP graph.

This is the decode harness of the reference (``src/nanoquant/kernel/test_decode.py``):
one prefill forward over the prompt, then one-token steps on a static KV cache
(``make_cache`` :420-422, ``generate`` :474-693), reporting
``tokens/s = B * (new - 1) / decode wall time`` (:617, :684-685). The reference wraps
a Hugging Face ``LlamaForCausalLM`` and compiles its step with
``torch.compile(mode="reduce-overhead")`` (:385-402). Here the whole step (embedding,
every layer, final norm, lm_head, greedy argmax, the KV-cache write, the token and
position update) is recorded once into a ``torch.cuda.CUDAGraph`` (a HIP graph on
ROCm) and replayed per token: the position lives in a device tensor, so replays need
no host synchronisation and several steps can be recorded into one graph.

The layers follow Hugging Face's Llama (RMSNorm in fp32, rotate-half RoPE, SiLU-gated
MLP, grouped-query attention, untied lm_head) and keep its module names
(``model.layers.{i}.self_attn.q_proj`` ...), so the packed state dict of a converted
checkpoint maps onto this model key for key.
"""
from __future__ import annotations

import math
import time
import warnings
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from .modules.linear import NanoQuantLinear

LINEAR_NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

# The fused step's complex rotary product runs on complex32 tensors, whose first allocation makes
# torch warn that ComplexHalf support is experimental; its multiply is what the step uses, and the
# step is checked against the unfused path.
warnings.filterwarnings("ignore", message="ComplexHalf support is experimental", category=UserWarning)


@dataclass(frozen=True)
class LlamaShape:
    """Architecture sizes (defaults: Llama-2-7B)."""

    hidden: int = 4096
    layers: int = 32
    heads: int = 32
    kv_heads: int = 32
    ffn: int = 11008
    vocab: int = 32000
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    def linear_shapes(self):
        """(name, in_features, out_features) of the seven linears of one layer."""
        h, kv = self.hidden, self.kv_heads * self.head_dim
        return (("q_proj", h, h), ("k_proj", h, kv), ("v_proj", h, kv), ("o_proj", h, h),
                ("gate_proj", h, self.ffn), ("up_proj", h, self.ffn), ("down_proj", self.ffn, h))


def rank_for_bpw(out_features: int, in_features: int, bpw: float) -> int:
    """Rank whose two sign factors cost ``bpw`` bits per weight, rounded to a multiple of 32.

    r = round32(bpw * m * n / (m + n)): 1632 for 11008x4096 and 1120 for 4096x4096 at 0.55.
    """
    r = bpw * out_features * in_features / (out_features + in_features)
    return max(32, int(round(r / 32.0)) * 32)


def random_nanoquant_linear(in_features: int, out_features: int, rank: int, generator: torch.Generator,
                            device, with_mid: bool = False) -> NanoQuantLinear:
    """A NanoQuantLinear in its dense (unpacked) state with random +-1 factors.

    Scales are |N(1, 0.2)| divided by sqrt(in_features) (scale_pre) and sqrt(rank)
    (scale_post), so an input of unit RMS gives an output of about unit RMS.
    """
    # the state init_for_inference (linear.py:116-129) leaves, without its placeholder tensors
    lin = nn.Linear(in_features, out_features, bias=False, device="meta")
    lin.__class__ = NanoQuantLinear
    lin.rank, lin.do_train, lin._binarized, lin.dtype = rank, False, True, torch.float32
    del lin._parameters["weight"]
    lin.register_parameter("weight", None)
    kw = dict(device=device, generator=generator)

    def signs(rows, cols):
        return torch.randint(0, 2, (rows, cols), dtype=torch.int8, **kw).mul_(2).sub_(1).float()

    def scales(k, div):
        return (torch.randn(1, k, **kw) * 0.2 + 1.0).abs_() / div

    lin.V = nn.Parameter(signs(rank, in_features), requires_grad=False)
    lin.U = nn.Parameter(signs(out_features, rank), requires_grad=False)
    lin.scale_pre = nn.Parameter(scales(in_features, math.sqrt(in_features)), requires_grad=False)
    lin.scale_post = nn.Parameter(scales(out_features, math.sqrt(rank)), requires_grad=False)
    if with_mid:
        lin.scale_mid = nn.Parameter(scales(rank, 1.0), requires_grad=False)
    return lin


class RMSNorm(nn.Module):
    """Hugging Face LlamaRMSNorm: normalise in fp32, cast back, then scale."""

    def __init__(self, dim: int, eps: float, device=None, dtype=torch.float32):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=dtype), requires_grad=False)
        self.eps = eps

    def forward(self, x):
        # x * rsqrt(mean(x^2) + eps) in fp32 (torch's fused RMS norm: one launch instead of five on
        # the GPU, the same values), cast back, then the weight
        xf = F.rms_norm(x.float(), (x.shape[-1],), eps=self.eps)
        return self.weight * xf.to(x.dtype)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class StaticKVCache:
    """Per-layer K and V of ``batch`` sequences up to ``max_len`` positions.

    Both are [B, kv_heads, max_len, head_dim]: a position's key or value is one contiguous
    row. Mirrors ``make_cache`` (test_decode.py:420-422): preallocated once, written in
    place at the step's position.
    """

    def __init__(self, shape: LlamaShape, batch: int, max_len: int, device, dtype):
        self.batch, self.max_len = batch, max_len
        kv, d = shape.kv_heads, shape.head_dim
        self.k = [torch.zeros(batch, kv, max_len, d, device=device, dtype=dtype) for _ in range(shape.layers)]
        self.v = [torch.zeros(batch, kv, max_len, d, device=device, dtype=dtype) for _ in range(shape.layers)]
        self.key_index = torch.arange(max_len, device=device)


def rotary_attention(shape: LlamaShape, layer: int, q, k, v, cos, sin, positions, cache: StaticKVCache):
    """Rotary embedding, KV-cache write at ``positions`` and causal attention over the cache, in
    torch ops (Hugging Face's Llama attention on a static cache).

    q [B, T, H*D], k and v [B, T, KV*D] (strided views are fine), cos and sin [T, D];
    returns [B, T, H*D] in the cache dtype.
    """
    H, KV, D = shape.heads, shape.kv_heads, shape.head_dim
    B, T = q.shape[0], q.shape[1]
    G = H // KV
    q = q.reshape(B, T, H, D).transpose(1, 2)
    k = k.reshape(B, T, KV, D).transpose(1, 2)
    v = v.reshape(B, T, KV, D).transpose(1, 2)
    q = q * cos + _rotate_half(q) * sin
    k = k * cos + _rotate_half(k) * sin
    k_c, v_c = cache.k[layer], cache.v[layer]
    k_c.index_copy_(2, positions, k.to(k_c.dtype))
    v_c.index_copy_(2, positions, v.to(v_c.dtype))
    # queries of one kv head side by side, scored as K [B, KV, L, D] @ Q^T [B, KV, D, G*T]: the
    # right operand is a small contiguous copy, never a transposed view, and the cache is read
    # in place
    qg_t = q.reshape(B, KV, G * T, D).transpose(2, 3).contiguous()
    scores = torch.matmul(k_c, qg_t).transpose(2, 3).float() * (D ** -0.5)  # [B, KV, G*T, L]
    visible = cache.key_index.view(1, -1) <= positions.view(-1, 1)  # [T, L]
    scores = scores.reshape(B, KV, G, T, -1).masked_fill(~visible, float("-inf"))
    p = torch.softmax(scores, dim=-1).to(v_c.dtype).reshape(B, KV, G * T, -1)
    return torch.matmul(p, v_c).view(B, H, T, D).transpose(1, 2).reshape(B, T, H * D)


def step_constants(head_dim: int, dtype, device):
    """The fixed parts of a one-token step's tables: the identity I and the rotate-half matrix P
    (x @ P == rotate_half(x)) [D, D] in ``dtype``, and the two values of the additive causal mask
    (0, -inf) as a [2] tensor. Callers make them once and keep them (the model as buffers): tensors
    made inside a captured or compiled step would be overwritten by the graph's next run."""
    h = head_dim // 2
    eye = torch.eye(head_dim, device=device, dtype=dtype)
    rot = torch.zeros(head_dim, head_dim, device=device, dtype=dtype)
    idx = torch.arange(h, device=device)
    rot[idx + h, idx] = -1.0  # out[j < h] takes -x[j + h]
    rot[idx, idx + h] = 1.0   # out[j >= h] takes x[j - h]
    values = torch.tensor([0.0, float("-inf")], device=device, dtype=dtype)
    return eye, rot, values


def step_mask(positions, cache: StaticKVCache, values, out=None):
    """The additive causal mask of a one-token step at ``positions`` (one position, on the device):
    [1, L, 1], values[0] (0) for cache rows up to the position and values[1] (-inf) past it; written
    into ``out`` (any shape that broadcasts [1, L, 1], e.g. every layer's scores at once) when it
    is given."""
    visible = cache.key_index.view(1, -1, 1) <= positions.view(1, 1, 1)
    if out is None:
        return torch.where(visible, values[0], values[1])
    # the condition takes out's full shape, so that the result is written in place, not resized
    L = visible.shape[1]
    visible = visible.view([1] * (out.dim() - 2) + [L, 1]).expand(out.shape)
    return torch.where(visible, values[0], values[1], out=out)


def rotary_step_tables(cos, sin, positions, cache: StaticKVCache, dtype, with_mask: bool = True, consts=None):
    """What every layer of a one-token step at ``positions`` (one position, on the device) shares:
    the rotary embedding as a [D, D] matrix R (x @ R == x * cos + rotate_half(x) * sin, with cos and
    sin [1, D] of that position) and the causal mask as an additive [1, L, 1] (0 for visible cache
    rows, -inf past the position; None without ``with_mask``). R = I * cos + P * sin column by
    column: each entry is one of cos, +-sin or 0, exact in ``dtype``. ``consts``: the
    ``step_constants`` to use (made here when None)."""
    D = cos.shape[-1]
    eye, rot, values = consts if consts is not None else step_constants(D, dtype, cos.device)
    eye, rot, values = eye.to(dtype), rot.to(dtype), values.to(dtype)
    R = torch.addcmul(eye * cos.reshape(1, D).to(dtype), rot, sin.reshape(1, D).to(dtype))
    return R, (step_mask(positions, cache, values) if with_mask else None)


def attention_products_step(shape: LlamaShape, layer: int, q, madd, cache: StaticKVCache, out, scores=None):
    """The attention products of a one-token step whose rotary embedding and cache write are done
    (``nq_rope_kv_write``): the scores of each kv head's query group against the cache with the scale
    and causal mask folded into one batched product, the softmax, and the value product written into
    ``out`` [B, H * D] (directly when each kv head serves one query head, else through a copy).

    q [B, H * D] (rotated, contiguous); ``madd`` [1, L, 1]: the additive causal mask of the step's
    position (0 for visible cache rows, -inf past it). With ``scores`` [B * KV, L, G] already holding
    that mask (``nq_gemv_group_stage2_rope`` writes it), the product adds into it in place and the
    mask is not copied in first (``madd`` is then unused)."""
    H, KV, D = shape.heads, shape.kv_heads, shape.head_dim
    B, G = q.shape[0], H // KV
    k_c, v_c = cache.k[layer], cache.v[layer]
    L = k_c.shape[2]
    # K [B*KV, L, D] @ Q^T [B*KV, D, G]: the right operand contiguous (a view when G == 1)
    q_t = q.view(B * KV, G, D).transpose(1, 2)
    if G > 1:
        q_t = q_t.contiguous()
    if scores is None:
        scores = torch.baddbmm(madd, k_c.view(B * KV, L, D), q_t, alpha=D ** -0.5)  # [B*KV, L, G]
    else:
        scores.baddbmm_(k_c.view(B * KV, L, D), q_t, alpha=D ** -0.5)
    p = torch.softmax(scores, dim=1)
    vt = v_c.view(B * KV, L, D).transpose(1, 2)
    if G == 1:
        torch.bmm(vt, p, out=out.view(B * KV, D, 1))
    else:
        out.view(B, KV, G, D).copy_(torch.bmm(vt, p).view(B, KV, D, G).transpose(2, 3))
    return out


def rotary_attention_step(shape: LlamaShape, layer: int, qk, v, tables, positions, cache: StaticKVCache, out=None,
                          scores=None):
    """``rotary_attention`` for one token per sequence in seven torch launches: RoPE of q and k as one
    matrix product, the two cache writes, the scores of each kv head's query group with the scale and
    the causal mask folded into one batched product, the softmax, the value product and the copy out.

    qk [B, (H + KV) * D] (q heads then k heads, contiguous), v [B, KV * D], or None when the value
    row is already in the cache; ``tables`` from ``rotary_step_tables``; returns [B, 1, H * D],
    written into ``out`` [B, H * D] when it is given and each kv head serves one query head (the
    value product then needs no copy). With ``scores`` [B * KV, L, G] already holding the step's
    additive causal mask, the scores product adds into it in place (the mask is not copied first).
    """
    H, KV, D = shape.heads, shape.kv_heads, shape.head_dim
    R, madd = tables
    rot = torch.mm(qk.reshape(-1, D), R).view(qk.shape[0], H + KV, D)
    return attention_after_rotary(shape, layer, rot, v, positions, cache, madd, out=out, scores=scores)


def attention_after_rotary(shape: LlamaShape, layer: int, rot, v, positions, cache: StaticKVCache, madd, out=None,
                           scores=None):
    """The rest of ``rotary_attention_step`` once q and k are rotated: rot [B, H + KV, D] (q heads then
    k heads); the key and value cache writes (v None: the value row is already in the cache), the
    scores with the scale and mask folded into one batched product (``madd`` the additive mask, or
    ``scores`` already holding it), the softmax and the value product (into ``out`` when given and
    each kv head serves one query head)."""
    H, KV, D = shape.heads, shape.kv_heads, shape.head_dim
    B, G = rot.shape[0], H // KV
    k_c, v_c = cache.k[layer], cache.v[layer]
    L = k_c.shape[2]
    k_c.index_copy_(2, positions, rot[:, H:].unsqueeze(2).to(k_c.dtype))
    if v is not None:
        v_c.index_copy_(2, positions, v.reshape(B, KV, 1, D).to(v_c.dtype))
    # K [B*KV, L, D] @ Q^T [B*KV, D, G]: the right operand is a contiguous copy (free for one query per kv head)
    q_t = rot[:, :H].reshape(B * KV, G, D).transpose(1, 2).contiguous()
    if scores is None:
        scores = torch.baddbmm(madd, k_c.view(B * KV, L, D), q_t.to(k_c.dtype), alpha=D ** -0.5)  # [B*KV, L, G]
    else:
        scores.baddbmm_(k_c.view(B * KV, L, D), q_t.to(k_c.dtype), alpha=D ** -0.5)
    p = torch.softmax(scores, dim=1)
    if out is not None and G == 1:
        torch.bmm(v_c.view(B * KV, L, D).transpose(1, 2), p, out=out.view(B * KV, D, 1))
        return out.view(B, 1, H * D)
    out_t = torch.bmm(v_c.view(B * KV, L, D).transpose(1, 2), p)  # [B*KV, D, G]
    return out_t.view(B, KV, D, G).transpose(2, 3).reshape(B, 1, H * D)


class LlamaAttention(nn.Module):
    def __init__(self, shape: LlamaShape, layer: int):
        super().__init__()
        self.shape, self.layer = shape, layer

    def forward(self, x, cos, sin, positions, cache: StaticKVCache, step_tables=None):
        if step_tables is not None:  # one token per sequence
            B = x.shape[0]
            qk = torch.cat((self.q_proj(x), self.k_proj(x)), dim=-1).view(B, -1)
            out = rotary_attention_step(self.shape, self.layer, qk, self.v_proj(x).view(B, -1), step_tables,
                                        positions, cache)
        else:
            out = rotary_attention(self.shape, self.layer, self.q_proj(x), self.k_proj(x), self.v_proj(x), cos, sin,
                                   positions, cache)
        return self.o_proj(out.to(x.dtype))


class LlamaMLP(nn.Module):
    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class LlamaDecoderLayer(nn.Module):
    def __init__(self, shape: LlamaShape, layer: int, device, dtype):
        super().__init__()
        self.self_attn = LlamaAttention(shape, layer)
        self.mlp = LlamaMLP()
        self.input_layernorm = RMSNorm(shape.hidden, shape.rms_eps, device, dtype)
        self.post_attention_layernorm = RMSNorm(shape.hidden, shape.rms_eps, device, dtype)

    def forward(self, x, cos, sin, positions, cache, step_tables=None):
        x = x + self.self_attn(self.input_layernorm(x), cos, sin, positions, cache, step_tables)
        return x + self.mlp(self.post_attention_layernorm(x))


class _Body(nn.Module):
    def __init__(self, shape: LlamaShape, device, dtype):
        super().__init__()
        self.embed_tokens = nn.Embedding(shape.vocab, shape.hidden, device=device, dtype=dtype)
        self.layers = nn.ModuleList(LlamaDecoderLayer(shape, i, device, dtype) for i in range(shape.layers))
        self.norm = RMSNorm(shape.hidden, shape.rms_eps, device, dtype)


class NanoQuantLlama(nn.Module):
    """Llama-2-architecture causal LM with NanoQuantLinear projections.

    ``forward(ids [B, T], positions [T], cache)`` returns fp32 logits [B, T, vocab];
    ``positions`` is a device tensor of absolute positions, so the same call serves
    prefill (0..T-1) and a graph-captured one-token step (a position held on the device).
    """

    def __init__(self, shape: LlamaShape, device=None, dtype=torch.float32):
        super().__init__()
        self.shape = shape
        self.dtype = dtype
        self.model = _Body(shape, device, dtype)
        self.lm_head = nn.Linear(shape.hidden, shape.vocab, bias=False, device=device, dtype=dtype)
        d = shape.head_dim
        inv_freq = 1.0 / (shape.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32, device=device) / d))
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        eye, rot, values = step_constants(d, dtype, device)
        self.register_buffer("step_eye", eye, persistent=False)
        self.register_buffer("step_rot", rot, persistent=False)
        self.register_buffer("step_mask_values", values, persistent=False)

    def linears(self):
        for layer in self.model.layers:
            for name in LINEAR_NAMES:
                owner = layer.self_attn if name.endswith(("q_proj", "k_proj", "v_proj", "o_proj")) else layer.mlp
                yield getattr(owner, name)

    def rope(self, positions, dtype):
        freqs = positions.float().view(-1, 1) * self.inv_freq.view(1, -1)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(dtype), emb.sin().to(dtype)

    def forward(self, ids, positions, cache: StaticKVCache):
        x = self.model.embed_tokens(ids)
        cos, sin = self.rope(positions, x.dtype)
        consts = (self.step_eye, self.step_rot, self.step_mask_values)
        tables = rotary_step_tables(cos, sin, positions, cache, x.dtype, consts=consts) if ids.shape[1] == 1 else None
        for layer in self.model.layers:
            x = layer(x, cos, sin, positions, cache, tables)
        x = self.model.norm(x)
        return self.lm_head(x).float()

    def prepare_kernels(self, kernel_type: str = "gemv", dtype=torch.float16):
        """Pack every linear for ``kernel_type`` and cast the rest of the model to ``dtype``
        (the reference calls ``_prepare_kernel`` on each NanoQuantLinear, test_decode.py:1228-1234)."""
        for lin in self.linears():
            lin._prepare_kernel(kernel_type, dtype)
        return self.cast_non_linears(dtype)

    def cast_non_linears(self, dtype):
        self.model.embed_tokens.to(dtype)
        self.model.norm.to(dtype)
        for layer in self.model.layers:
            layer.input_layernorm.to(dtype)
            layer.post_attention_layernorm.to(dtype)
        self.lm_head.to(dtype)
        for name in ("step_eye", "step_rot", "step_mask_values"):  # the one-token step's tables
            setattr(self, name, getattr(self, name).to(dtype))
        self.dtype = dtype
        return self


def random_llama(shape: LlamaShape, bpw: float = 0.55, seed: int = 0, device="cuda", with_mid: bool = False,
                 kernel_type: str | None = None, dtype=torch.float16) -> NanoQuantLlama:
    """Random-init model: N(0, 0.02) embedding and lm_head, random NanoQuant factors of
    rank ``rank_for_bpw`` for all seven linears of every layer.

    With ``kernel_type`` None the model stays dense in fp32 (the reference path of every
    linear); otherwise each linear is packed for that kernel as soon as it is drawn (so the
    dense factors of only one linear exist at a time) and the model is cast to ``dtype``.
    """
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    model = NanoQuantLlama(shape, device=device, dtype=torch.float32)
    with torch.no_grad():
        model.model.embed_tokens.weight.normal_(0.0, 0.02, generator=gen)
        model.lm_head.weight.normal_(0.0, 0.02, generator=gen)
        for layer in model.model.layers:
            for name, n_in, n_out in shape.linear_shapes():
                owner = layer.self_attn if name in ("q_proj", "k_proj", "v_proj", "o_proj") else layer.mlp
                lin = random_nanoquant_linear(n_in, n_out, rank_for_bpw(n_out, n_in, bpw), gen, device, with_mid)
                if kernel_type is not None:
                    lin._prepare_kernel(kernel_type, dtype)
                setattr(owner, name, lin)
    if kernel_type is not None:
        model.cast_non_linears(dtype)
    return model.eval()


class GraphDecoder:
    """Greedy decoding with ``steps_per_graph`` one-token steps recorded in one HIP graph.

    Device state: ``ids`` [B, max_len] (prompt, then generated tokens) and ``pos``
    (the position of the last token so far). A step embeds ``ids[:, pos]``, runs the
    model at ``pos`` (writing K/V there), takes the argmax of the logits, stores it at
    ``ids[:, pos + 1]`` and advances ``pos``. Nothing in a step reads the host.
    """

    def __init__(self, model: NanoQuantLlama, batch: int, max_len: int, steps_per_graph: int = 1,
                 device="cuda"):
        self.model, self.batch, self.max_len = model, batch, max_len
        self.steps_per_graph = steps_per_graph
        self.device = torch.device(device)
        self.cache = StaticKVCache(model.shape, batch, max_len, self.device, model.dtype)
        self.ids = torch.zeros(batch, max_len, dtype=torch.long, device=self.device)
        self.pos = torch.zeros(1, dtype=torch.long, device=self.device)
        self.last_logits = None
        self.graph = None
        self.stream = None

    def _step(self):
        tok = self.ids.index_select(1, self.pos)  # [B, 1]
        logits = self.model(tok, self.pos, self.cache)[:, -1]  # [B, V] fp32
        nxt = logits.argmax(dim=-1, keepdim=True)
        self.pos.add_(1)
        self.ids.index_copy_(1, self.pos, nxt)
        return logits

    def _steps(self):
        logits = None
        for _ in range(self.steps_per_graph):
            logits = self._step()
        return logits

    @torch.no_grad()
    def capture(self, warmup: int = 2):
        """Warm up on the capture stream (allocates workspaces outside the graph), then record."""
        saved = self.pos.clone()
        if self.stream is None:
            self.stream = torch.cuda.Stream(self.device)
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                self.pos.zero_()
                self._steps()
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.last_logits = self._steps()
        self.pos.copy_(saved)
        torch.cuda.synchronize(self.device)
        return self

    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        """Run the prompt [B, T] at positions 0..T-1 and place its greedy next token."""
        B, T = prompt.shape
        if B != self.batch or T + 1 > self.max_len:
            raise ValueError(f"prompt {tuple(prompt.shape)} does not fit batch {self.batch}, max_len {self.max_len}")
        self.ids[:, :T].copy_(prompt)
        positions = torch.arange(T, device=self.device)
        logits = self.model(self.ids[:, :T], positions, self.cache)[:, -1]
        self.ids[:, T] = logits.argmax(dim=-1)
        self.pos.fill_(T)
        return logits

    @torch.no_grad()
    def decode(self, steps: int, use_graph: bool = True):
        """Run ``steps`` one-token steps (a multiple of ``steps_per_graph`` when graphed)."""
        if use_graph:
            if self.graph is None:
                raise RuntimeError("capture() the decode graph first")
            if steps % self.steps_per_graph:
                raise ValueError(f"steps ({steps}) must be a multiple of steps_per_graph ({self.steps_per_graph})")
            for _ in range(steps // self.steps_per_graph):
                self.graph.replay()
            return self.last_logits
        logits = None
        for _ in range(steps):
            logits = self._step()
        return logits


class FusedDecoder(GraphDecoder):
    """GraphDecoder whose one-token step runs each layer in nine launches of the HIP library:

    1. q, k, v stage 1 in one launch, with input_layernorm folded in (its weight multiplied
       into each s_in, the rsqrt(mean(x^2) + eps) factor applied to h);
    2. q, k, v stage 2 in one launch, into one [B, (heads + 2 kv_heads) * head_dim] buffer;
    3. rotary embedding, KV-cache write and attention: in torch ops (``attention="torch"``, the
       default, as the benchmark's end-to-end configuration keeps the non-linear ops in
       PyTorch; step 2 then also writes the value row into its cache,
       ``nq_gemv_group_stage2_kv``, and the step's causal mask goes into every layer's scores
       buffer in one launch per step), or the rotary embedding and cache write folded into step
       2's stores (``nq_gemv_group_stage2_rope``) and the attention products in torch
       (``attention="rope"``), or all of it in one HIP launch pair (``attention="hip"``,
       ``nq_attention_decode``);
    4, 5. o_proj, its stage 2 adding the residual;
    6. gate and up stage 1 in one launch, post_attention_layernorm folded in;
    7. gate and up stage 2 in one launch storing silu(gate) * up;
    8, 9. down_proj, its stage 2 adding the residual.
    The final norm and the lm_head run as one dense GEMV of the library (``nq_dense_gemv`` with
    its RMS-norm prologue: torch's linear reads the head's weights, cold after the layers, at a
    fraction of the bandwidth), which writes the float32 logits; the embedding lookup and argmax
    stay torch ops. The logits a step returns live in a buffer the next step overwrites. Prefill runs the unfused model (it fills the same cache
    layout). Needs the model packed for the ``gemv`` kernel in float16 or bfloat16 and head_dim 128.
    """

    def __init__(self, model: NanoQuantLlama, batch: int, max_len: int, steps_per_graph: int = 1,
                 device="cuda", attention: str = "torch"):
        super().__init__(model, batch, max_len, steps_per_graph, device)
        from . import _lib

        if attention not in ("torch", "rope", "hip"):
            raise ValueError(f"attention must be 'torch', 'rope' or 'hip', got {attention!r}")
        self.attention = attention

        self._lib = _lib
        self.lib = _lib.load()
        s = model.shape
        dt = model.dtype
        if dt not in (torch.float16, torch.bfloat16):
            raise ValueError(f"the fused decode step needs a float16 or bfloat16 model, got {dt}")
        if attention == "hip" and s.head_dim != 128:
            raise ValueError(f"the HIP attention of the fused decode step needs head_dim 128, got {s.head_dim}")
        if attention == "rope" and s.head_dim % 16:
            raise ValueError(f"the rotary store of the fused decode step needs head_dim % 16 == 0, got {s.head_dim}")
        for lin in model.linears():
            if getattr(lin, "kernel_type", None) != "gemv":
                raise ValueError("the fused decode step needs every linear prepared for the 'gemv' kernel")
        dev = self.device
        H, KV, D = s.heads, s.kv_heads, s.head_dim
        self.dcode = _lib.dtype_code(dt)
        self.qkv_width = (H + 2 * KV) * D
        self.x = torch.zeros(batch, s.hidden, device=dev, dtype=dt)
        self.h = torch.zeros(batch, s.hidden, device=dev, dtype=dt)
        self.qkv = torch.zeros(batch, self.qkv_width, device=dev, dtype=dt)
        self.attn = torch.zeros(batch, H * D, device=dev, dtype=dt)
        self.q_rot = torch.zeros(batch, H * D, device=dev, dtype=dt)
        # attention scores of the rope step [B * KV, L, G]: the q/k/v launch writes the step's causal
        # mask into it, the scores product adds into it in place
        self.scores = torch.zeros(batch * KV, max_len, H // KV, device=dev, dtype=dt)
        # the torch step's scores, one buffer per layer: the step's causal mask is copied into all of
        # them by one launch, and each layer's scores product adds into its own in place
        self.scores_all = (torch.zeros(s.layers, batch * KV, max_len, H // KV, device=dev, dtype=dt)
                           if attention == "torch" else None)
        head = model.lm_head
        if head.weight.dtype != dt or head.in_features % 8:
            raise ValueError("the fused decode step's lm_head needs the model dtype and in_features % 8 == 0")
        self.head_weight = head.weight.detach().contiguous()
        self.head_bias = None if head.bias is None else head.bias.detach()
        self.logits16 = torch.zeros(batch, head.out_features, device=dev, dtype=dt)
        self.logits = torch.zeros(batch, head.out_features, device=dev, dtype=torch.float32)
        norm = model.model.norm
        if norm.weight.dtype != dt:
            raise ValueError("the fused decode step folds the final norm into the lm_head: its weight needs the model dtype")
        self.norm_weight = norm.weight.detach().contiguous()
        self.act = torch.zeros(batch, s.ffn, device=dev, dtype=dt)
        cos, sin = model.rope(torch.arange(max_len, device=dev), dt)
        self.rope_cos, self.rope_sin = cos.contiguous(), sin.contiguous()
        self.rope_cs = torch.stack((self.rope_cos, self.rope_sin), dim=1).contiguous()  # [max_len, 2, D]
        self.tok = torch.zeros(batch, dtype=torch.long, device=dev)  # the step's input token ids
        self.step_consts = step_constants(D, dt, dev)
        # the torch step in float16 rotates q and k as one complex product: their features in pair
        # order (feature j of a head, then j + D/2, ...), the cache's keys too (dot products do not
        # change under a common reordering); bfloat16 has no complex type and keeps the [D, D] product
        self.pair_order = attention == "torch" and dt == torch.float16
        if self.pair_order:
            j = torch.arange(D, device=dev)
            self.head_order = (j // 2) + (j % 2) * (D // 2)  # position i of a head holds feature head_order[i]
            self.q_order = (torch.arange(H, device=dev)[:, None] * D + self.head_order).reshape(-1)
            self.k_order = (torch.arange(KV, device=dev)[:, None] * D + self.head_order).reshape(-1)
            half = torch.stack((self.rope_cos[:, : D // 2], self.rope_sin[:, : D // 2]), dim=-1).contiguous()
            self.rope_freqs = torch.view_as_complex(half)  # [max_len, D / 2] complex32: cos + i sin
            self.rot = torch.zeros(batch, H + KV, D, device=dev, dtype=dt)
        self._keep = []  # tensors whose addresses the item tables hold
        self.plans = [self._layer_plan(layer) for layer in model.model.layers]
        need = 0
        for plan in self.plans:
            for items, count in (plan["qkv"], plan["o"], plan["gu"], plan["down"]):
                need = max(need, self.lib.nq_gemv_group_workspace_bytes(count, items, batch))
        self.ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)
        self.attn_ws = None
        if attention == "hip":  # the partial results of the 64-position chunks
            abytes = self.lib.nq_attention_decode_workspace_bytes(batch, H, KV, D, max_len)
            if abytes == 0:
                raise ValueError("nq_attention_decode does not take this head layout")
            self.attn_ws = torch.zeros(abytes, dtype=torch.uint8, device=dev)

    def _scale_in(self, lin, norm_weight):
        s_in = lin.scale_pre
        if norm_weight is not None:
            s_in = (s_in.float() * norm_weight.float()).to(s_in.dtype)
        s_in = s_in.contiguous()
        self._keep.append(s_in)
        return s_in

    def _items(self, entries):
        """Item table of (linear, norm weight, y, offset, stride, residual[, output row order]): with a
        row order (an index tensor over the outputs), the item holds copies of U's rows and s_out in
        that order, so output j of the item is output order[j] of the linear."""
        arr = (self._lib.GemvItem * len(entries))()
        for i, entry in enumerate(entries):
            lin, norm_weight, y, y_off, y_stride, resid = entry[:6]
            order = entry[6] if len(entry) > 6 else None
            u_words, s_out = lin.U_int8, lin.scale_post
            if order is not None:
                u_words, s_out = u_words.index_select(0, order).contiguous(), s_out.index_select(0, order).contiguous()
                self._keep += [u_words, s_out]
            it = arr[i]
            it.v_bits = lin.V_int8.data_ptr()
            it.s_in = self._scale_in(lin, norm_weight).data_ptr()
            mid = getattr(lin, "scale_mid", None)
            it.s_mid = None if mid is None else mid.data_ptr()
            it.u_bits = u_words.data_ptr()
            it.s_out = s_out.data_ptr()
            it.y = y.data_ptr() + y_off * y.element_size()
            it.resid = None if resid is None else resid.data_ptr()
            it.r = lin.V_int8.shape[0]
            it.m = lin.scale_post.numel()
            it.y_stride = y_stride
        return arr, len(entries)

    def _layer_plan(self, layer):
        s = self.model.shape
        H, KV, D = s.heads, s.kv_heads, s.head_dim
        a, mlp = layer.self_attn, layer.mlp
        w1, w2 = layer.input_layernorm.weight, layer.post_attention_layernorm.weight
        W = self.qkv_width
        # in pair order (the torch step's complex rotary product) q and k come out with each head's
        # features j and j + D/2 side by side
        qo, ko = (self.q_order, self.k_order) if self.pair_order else (None, None)
        return {
            "qkv": self._items([(a.q_proj, w1, self.qkv, 0, W, None, qo), (a.k_proj, w1, self.qkv, H * D, W, None, ko),
                                (a.v_proj, w1, self.qkv, (H + KV) * D, W, None)]),
            # the same three items with q stored rotated into q_rot (k and v go to the caches)
            "qkv_rope": self._items([(a.q_proj, w1, self.q_rot, 0, H * D, None), (a.k_proj, w1, self.qkv, 0, W, None),
                                     (a.v_proj, w1, self.qkv, 0, W, None)])[0],
            "o": self._items([(a.o_proj, None, self.h, 0, s.hidden, self.x)]),
            "gu": self._items([(mlp.gate_proj, w2, self.act, 0, s.ffn, None),
                               (mlp.up_proj, w2, self.act, 0, s.ffn, None)]),
            "down": self._items([(mlp.down_proj, None, self.x, 0, s.hidden, self.h)]),
            "eps1": layer.input_layernorm.eps, "eps2": layer.post_attention_layernorm.eps,
        }

    def _check(self, status, what):
        self._lib.check(status, what)

    def _step(self):
        lib, s, B = self.lib, self.model.shape, self.batch
        H, KV, D = s.heads, s.kv_heads, s.head_dim
        dt, ws, wsb = self.dcode, self.ws.data_ptr(), self.ws.numel()
        st = self._lib.stream_of(self.device)
        torch.index_select(self.model.model.embed_tokens.weight, 0, self.tok, out=self.x)
        if self.attention == "torch":
            if self.pair_order:
                freqs = self.rope_freqs.index_select(0, self.pos)  # [1, D / 2]: cos + i sin of the position
            else:
                cs = self.rope_cs.index_select(0, self.pos)  # [1, 2, D]: cos, sin of the position
                tables = rotary_step_tables(cs[:, 0], cs[:, 1], self.pos, self.cache, self.model.dtype,
                                            with_mask=False, consts=self.step_consts)
            step_mask(self.pos, self.cache, self.step_consts[2], out=self.scores_all)
        x, h, qkv, attn, act = (t.data_ptr() for t in (self.x, self.h, self.qkv, self.attn, self.act))
        esz = self.qkv.element_size()
        for li, plan in enumerate(self.plans):
            items, n = plan["qkv"]
            self._check(lib.nq_gemv_group_stage1(dt, n, items, x, B, s.hidden, plan["eps1"], ws, wsb, st), "qkv 1")
            if self.attention == "rope":
                items_r = plan["qkv_rope"]
                self._check(lib.nq_gemv_group_stage2_rope(
                    dt, items_r, B, self.cache.k[li].data_ptr(), self.cache.v[li].data_ptr(), self.rope_cos.data_ptr(),
                    self.rope_sin.data_ptr(), self.pos.data_ptr(), D, self.max_len, self.scores.data_ptr(), ws, wsb,
                    st), "qkv 2 rope")
            elif self.attention == "torch":
                self._check(lib.nq_gemv_group_stage2_kv(dt, items, B, self.cache.v[li].data_ptr(),
                                                        self.pos.data_ptr(), D, self.max_len, ws, wsb, st), "qkv 2 kv")
            else:
                self._check(lib.nq_gemv_group_stage2(dt, n, items, B, self._lib.NQ_EPI_STORE, ws, wsb, st), "qkv 2")
            if self.attention == "hip":
                self._check(lib.nq_attention_decode(
                    dt, qkv, qkv + H * D * esz, qkv + (H + KV) * D * esz, self.qkv_width,
                    self.cache.k[li].data_ptr(), self.cache.v[li].data_ptr(), self.rope_cos.data_ptr(),
                    self.rope_sin.data_ptr(), self.pos.data_ptr(), attn, B, H, KV, D, self.max_len,
                    D ** -0.5, self.attn_ws.data_ptr(), self.attn_ws.numel(), st), "attention")
            elif self.attention == "rope":
                attention_products_step(s, li, self.q_rot, None, self.cache, self.attn, scores=self.scores)
            else:
                qk = self.qkv[:, :(H + KV) * D]
                if self.pair_order:
                    pairs = torch.view_as_complex(qk.reshape(B, H + KV, D // 2, 2))
                    torch.mul(pairs, freqs, out=torch.view_as_complex(self.rot.view(B, H + KV, D // 2, 2)))
                    out = attention_after_rotary(s, li, self.rot, None, self.pos, self.cache, None, out=self.attn,
                                                 scores=self.scores_all[li])
                else:
                    out = rotary_attention_step(s, li, qk, None, tables, self.pos, self.cache, out=self.attn,
                                                scores=self.scores_all[li])
                if out.data_ptr() != self.attn.data_ptr():
                    self.attn.copy_(out.view(B, H * D))
            items, n = plan["o"]
            self._check(lib.nq_gemv_group_stage1(dt, n, items, attn, B, H * D, -1.0, ws, wsb, st), "o 1")
            self._check(lib.nq_gemv_group_stage2(dt, n, items, B, self._lib.NQ_EPI_RESIDUAL, ws, wsb, st), "o 2")
            items, n = plan["gu"]
            self._check(lib.nq_gemv_group_stage1(dt, n, items, h, B, s.hidden, plan["eps2"], ws, wsb, st), "gu 1")
            self._check(lib.nq_gemv_group_stage2(dt, n, items, B, self._lib.NQ_EPI_GATED, ws, wsb, st), "gu 2")
            items, n = plan["down"]
            self._check(lib.nq_gemv_group_stage1(dt, n, items, act, B, s.ffn, -1.0, ws, wsb, st), "down 1")
            self._check(lib.nq_gemv_group_stage2(dt, n, items, B, self._lib.NQ_EPI_RESIDUAL, ws, wsb, st),
                        "down 2")
        # the final RMS norm folded into the lm_head launch; float32 logits straight from it (with a
        # bias, the dtype logits, the bias added in dtype, then widened, as the torch head rounds)
        norm = self.model.model.norm
        hw = self.head_weight
        out = self.logits if self.head_bias is None else self.logits16
        self._check(lib.nq_dense_gemv(dt, hw.data_ptr(), self.x.data_ptr(), self.norm_weight.data_ptr(), norm.eps,
                                      out.data_ptr(), int(self.head_bias is None), B, hw.shape[1], hw.shape[0],
                                      out.shape[1], st), "lm_head")
        logits = self.logits if self.head_bias is None else (self.logits16 + self.head_bias).float()
        self._check(lib.nq_argmax_rows(logits.data_ptr(), B, logits.shape[1], logits.stride(0), self.tok.data_ptr(),
                                       st), "argmax")
        self.pos.add_(1)
        self.ids.index_copy_(1, self.pos, self.tok.view(-1, 1))
        return logits

    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        logits = super().prefill(prompt)
        self.tok.copy_(self.ids[:, prompt.shape[1]])  # the step's input token, kept on the device
        if self.pair_order:  # the prompt's keys into the step's pair order
            for k_c in self.cache.k:
                k_c.copy_(k_c.index_select(3, self.head_order))
        return logits


@torch.no_grad()
def generate(model: NanoQuantLlama, prompt: torch.Tensor, max_new_tokens: int, steps_per_graph: int = 1,
             use_graph: bool = True, decoder: GraphDecoder | None = None, fused: bool = False,
             attention: str = "torch"):
    """Greedy generation with decode timing (test_decode.py:474-693, greedy instead of top-k sampling).

    Returns (ids [B, T + max_new_tokens], tokens_per_s, prof). Token 1 comes from the
    prefill; the timed loop produces tokens 2..max_new_tokens, and
    tokens/s = B * (max_new_tokens - 1) / decode wall time, as the reference reports it.
    """
    B, T = prompt.shape
    if decoder is None:
        if fused:
            decoder = FusedDecoder(model, B, T + max_new_tokens, steps_per_graph, device=prompt.device,
                                   attention=attention)
        else:
            decoder = GraphDecoder(model, B, T + max_new_tokens, steps_per_graph, device=prompt.device)
        if use_graph:
            decoder.capture()
    steps = max_new_tokens - 1
    torch.cuda.synchronize(prompt.device)
    t0 = time.perf_counter()
    decoder.prefill(prompt)
    torch.cuda.synchronize(prompt.device)
    t1 = time.perf_counter()
    decoder.decode(steps, use_graph=use_graph)
    torch.cuda.synchronize(prompt.device)
    t2 = time.perf_counter()
    tps = B * steps / max(t2 - t1, 1e-9)
    prof = {"prefill_time_s_wall": t1 - t0, "decode_time_s_wall": t2 - t1, "decode_tokens_total": B * steps,
            "ms_per_token": 1e3 * (t2 - t1) / max(steps, 1)}
    return decoder.ids[:, :T + max_new_tokens].clone(), tps, prof
