"""CPU checks of the decode harness: the Llama decoder and its static-cache decode loop,
in the dense (reference-path) state of every NanoQuantLinear, against Hugging Face's
``LlamaForCausalLM`` loaded with the equivalent dense weights
W = diag(s_post) U diag(s_mid) V diag(s_pre) (``linear.py:282-291``). The reference's
decode harness drives that same Hugging Face model (``test_decode.py:385-422``), so this
pins the architecture (RMSNorm, RoPE, grouped-query attention, gated MLP), the KV-cache
positions and the greedy loop independently of this package's own layer code.
"""
import numpy as np
import pytest
import torch

from nanoquant_amd.decode import GraphDecoder, LlamaShape, rank_for_bpw, random_llama

TINY = LlamaShape(hidden=128, layers=2, heads=4, kv_heads=2, ffn=320, vocab=500)


def dense_weight(lin):
    """The dense matrix a NanoQuantLinear applies (fp64), for the Hugging Face model."""
    V = lin.V.double()
    U = lin.U.double()
    s_pre = lin.scale_pre.double().reshape(-1)
    s_post = lin.scale_post.double().reshape(-1)
    mid = getattr(lin, "scale_mid", None)
    inner = U * (mid.double().reshape(1, -1) if mid is not None else 1.0)
    return s_post.view(-1, 1) * (inner @ V) * s_pre.view(1, -1)


def hf_twin(model, shape):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=shape.hidden, intermediate_size=shape.ffn, num_hidden_layers=shape.layers,
                      num_attention_heads=shape.heads, num_key_value_heads=shape.kv_heads,
                      vocab_size=shape.vocab, rms_norm_eps=shape.rms_eps, rope_theta=shape.rope_theta,
                      max_position_embeddings=256, attention_bias=False, mlp_bias=False, tie_word_embeddings=False)
    hf = LlamaForCausalLM(cfg).eval().float()
    sd = {"model.embed_tokens.weight": model.model.embed_tokens.weight, "lm_head.weight": model.lm_head.weight,
          "model.norm.weight": model.model.norm.weight}
    for i, layer in enumerate(model.model.layers):
        p = f"model.layers.{i}."
        sd[p + "input_layernorm.weight"] = layer.input_layernorm.weight
        sd[p + "post_attention_layernorm.weight"] = layer.post_attention_layernorm.weight
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            sd[p + f"self_attn.{name}.weight"] = dense_weight(getattr(layer.self_attn, name)).float()
        for name in ("gate_proj", "up_proj", "down_proj"):
            sd[p + f"mlp.{name}.weight"] = dense_weight(getattr(layer.mlp, name)).float()
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return hf


def test_rank_rule():
    # round32(bpw * m * n / (m + n)) at the Llama-2-7B shapes
    assert rank_for_bpw(11008, 4096, 0.55) == 1632
    assert rank_for_bpw(4096, 11008, 0.55) == 1632
    assert rank_for_bpw(4096, 4096, 0.55) == 1120
    assert rank_for_bpw(4096, 4096, 1.0) == 2048
    assert rank_for_bpw(11008, 4096, 1.0) == 2976


@pytest.mark.parametrize("with_mid", [False, True])
def test_dense_decoder_matches_hf_llama(with_mid):
    torch.manual_seed(0)
    model = random_llama(TINY, bpw=0.55, seed=3, device="cpu", with_mid=with_mid)
    # non-trivial norm weights so that a dropped norm scale shows
    with torch.no_grad():
        for layer in model.model.layers:
            layer.input_layernorm.weight.uniform_(0.5, 1.5)
            layer.post_attention_layernorm.weight.uniform_(0.5, 1.5)
        model.model.norm.weight.uniform_(0.5, 1.5)
    hf = hf_twin(model, TINY)

    B, T, new = 2, 11, 6
    prompt = torch.randint(0, TINY.vocab, (B, T), generator=torch.Generator().manual_seed(1))
    dec = GraphDecoder(model, B, T + new, device="cpu")
    step_logits = [dec.prefill(prompt)]
    for _ in range(new - 1):
        step_logits.append(dec.decode(1, use_graph=False))
    ids = dec.ids[:, :T + new]
    assert torch.equal(ids[:, :T], prompt)

    with torch.no_grad():
        ref = hf(ids[:, :-1]).logits.double()  # [B, T + new - 1, V]
    for j, lg in enumerate(step_logits):
        r = ref[:, T - 1 + j]
        err = (lg.double() - r).abs().max() / r.abs().max()
        assert err < 1e-5, (j, float(err))
        np.testing.assert_array_equal(ids[:, T + j].numpy(), r.argmax(-1).numpy())


def test_decoder_prefill_equals_stepwise():
    """Prefilling T tokens at once and feeding them one position at a time give the same logits."""
    model = random_llama(TINY, seed=5, device="cpu")
    B, T = 1, 7
    prompt = torch.randint(0, TINY.vocab, (B, T), generator=torch.Generator().manual_seed(2))
    a = GraphDecoder(model, B, T + 1, device="cpu")
    full = a.prefill(prompt)
    b = GraphDecoder(model, B, T + 1, device="cpu")
    b.ids[:, :T] = prompt
    for t in range(T):
        b.pos.fill_(t)
        lg = model(b.ids[:, t:t + 1], b.pos, b.cache)[:, -1]
    torch.testing.assert_close(lg, full, rtol=1e-5, atol=1e-5)


def test_linear_names_match_hf_layout():
    model = random_llama(LlamaShape(hidden=64, layers=1, heads=2, kv_heads=1, ffn=96, vocab=50), device="cpu")
    names = {k for k, _ in model.named_parameters()}
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        assert f"model.layers.0.self_attn.{name}.V" in names
    for name in ("gate_proj", "up_proj", "down_proj"):
        assert f"model.layers.0.mlp.{name}.U" in names
    assert "lm_head.weight" in names and "model.embed_tokens.weight" in names
