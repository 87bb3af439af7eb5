"""The model oracle's layer wiring against an independent implementation of the same
architecture: HF transformers' Qwen3.5 dense text model (transformers.models.qwen3_5,
the family the reference's qwen38_spec.h describes: hybrid gated-delta-net / gated
attention layers, (1 + w) RMSNorms, partial rotary, SwiGLU MLP).

oracle/model.py restates the reference's decode session (qwen_runtime.cpp:421-544)
over the oracle ops; its A4 GEMMs are pinned on their own (tests/test_oracle.py).  What
nothing else pins is the wiring between them: which norm feeds which projection, the
residual adds, the attention gate (per head, [query | gate] halves of q_proj, sigmoid
on the output), Q/K norm before the partial NeoX rotary, GQA grouping, the GDN causal
conv + SiLU, q/k L2 norms and query scale, decay exp(-exp(A_log) softplus(a + dt_bias))
and beta sigmoid(b), the gated delta rule, the gated output norm, the final norm and
head.  Here the oracle's projections are swapped for float matmuls of the same
dequantized weights, and the HF model (float32, eager attention, its chunked delta
rule) is loaded with exactly those weights; the logits of a block of tokens from an
empty state must agree to the fp16 rounding the oracle applies at its stage
boundaries.  CPU only; skipped when transformers lacks the module.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O

SEED = 1234
TOKENS = 12


def _bf16(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _dequantized(m):
    scales = O.f16_bits_to_f32(m.ws16).reshape(m.rows, m.cols // 128)
    return (m.w.astype(np.float32).reshape(m.rows, m.cols // 128, 128) * scales[:, :, None]).reshape(m.rows, m.cols)


def _hf_model(spec, oracle_model, torch):
    qwen = pytest.importorskip("transformers.models.qwen3_5")
    s = spec.as_dict()
    layer_types = ["full_attention" if (i + 1) % s["full_attention_interval"] == 0 else "linear_attention"
                   for i in range(s["layer_count"])]
    config = qwen.Qwen3_5TextConfig(
        vocab_size=s["vocabulary_size"], hidden_size=s["hidden_size"], intermediate_size=s["intermediate_size"],
        num_hidden_layers=s["layer_count"], num_attention_heads=s["attention_head_count"],
        num_key_value_heads=s["kv_head_count"], head_dim=s["attention_head_size"], rms_norm_eps=1e-6,
        linear_conv_kernel_dim=4, linear_key_head_dim=s["gdn_head_size"], linear_value_head_dim=s["gdn_head_size"],
        linear_num_key_heads=s["gdn_key_head_count"], linear_num_value_heads=s["gdn_value_head_count"],
        layer_types=layer_types, tie_word_embeddings=False,
        rope_parameters={"rope_type": "default", "rope_theta": float(s["rope_theta"]),
                         "partial_rotary_factor": s["rotary_size"] / s["attention_head_size"]})
    config._attn_implementation = "eager"
    model = qwen.Qwen3_5ForCausalLM(config).eval()
    m = oracle_model
    with torch.no_grad():
        def put(param, array):
            param.copy_(torch.from_numpy(np.ascontiguousarray(array, np.float32)).reshape(param.shape))
        put(model.model.embed_tokens.weight, _dequantized(m.embed))
        put(model.model.norm.weight, _bf16(m.final_norm))
        put(model.lm_head.weight, _dequantized(m.lm_head))
        for i, L in enumerate(m.layers):
            layer = model.model.layers[i]
            put(layer.input_layernorm.weight, _bf16(L["input_norm"]))
            put(layer.post_attention_layernorm.weight, _bf16(L["post_norm"]))
            for name in ("gate", "up", "down"):
                put(getattr(layer.mlp, name + "_proj").weight, _dequantized(L[name]))
            if L["attention"]:
                a = layer.self_attn
                for name in ("q", "k", "v", "o"):
                    put(getattr(a, name + "_proj").weight, _dequantized(L[name]))
                put(a.q_norm.weight, _bf16(L["q_norm"]))
                put(a.k_norm.weight, _bf16(L["k_norm"]))
            else:
                g = layer.linear_attn
                put(g.in_proj_qkv.weight, _dequantized(L["qkv"]))
                put(g.in_proj_z.weight, _dequantized(L["z"]))
                put(g.in_proj_a.weight, _dequantized(L["a"]))
                put(g.in_proj_b.weight, _dequantized(L["b"]))
                put(g.out_proj.weight, _dequantized(L["out"]))
                put(g.conv1d.weight, _bf16(L["conv"]))
                put(g.A_log, _bf16(L["a_log"]))
                put(g.dt_bias, _bf16(L["dt_bias"]))
                put(g.norm.weight, _bf16(L["gdn_norm"]))
    return model


BAR = 5e-3  # of the largest logit: the oracle's fp16 stage roundings give about 2e-3


def _float_oracle_logits(spec, oracle_model, monkeypatch, tokens):
    """The oracle's block_step from an empty state with every projection a float matmul
    of its dequantized weights."""
    from oracle.model import Matrix, OracleSession
    float_weights = {}

    def float_matmul(self, x16):
        key = id(self)
        if key not in float_weights:
            float_weights[key] = _dequantized(self)
        x = O.f16_bits_to_f32(np.ascontiguousarray(x16)).reshape(x16.shape)
        return (x.astype(np.float64) @ float_weights[key].astype(np.float64).T).astype(np.float32)

    monkeypatch.setattr(Matrix, "__call__", float_matmul)
    _, logits = OracleSession(oracle_model, 64).block_step(tokens)
    return logits


def _case(shape):
    torch = pytest.importorskip("torch")
    pytest.importorskip("transformers.models.qwen3_5")
    from gfxinfer_amd.runtime import reference_tiny_spec, tiny_spec
    from oracle.model import OracleModel
    spec = tiny_spec() if shape == "baseline" else reference_tiny_spec()
    oracle_model = OracleModel(spec.as_dict(), SEED)
    hf = _hf_model(spec, oracle_model, torch)
    tokens = [int(t) for t in np.random.default_rng(SEED).integers(0, spec.tokenizer_vocabulary_size, TOKENS)]
    with torch.no_grad():
        want = hf(torch.tensor([tokens])).logits[0].numpy()
    return spec, oracle_model, tokens, want


@pytest.mark.parametrize("shape", ["baseline", "reference"])
def test_oracle_wiring_matches_hf_qwen3_5(monkeypatch, shape):
    spec, oracle_model, tokens, want = _case(shape)
    logits = _float_oracle_logits(spec, oracle_model, monkeypatch, tokens)
    scale = float(np.abs(want).max())
    err = float(np.abs(logits - want).max())
    assert scale > 0.1, scale  # non-trivial logits
    assert err <= BAR * scale, (shape, err, scale)
    # the same greedy tokens wherever the float model's top-2 margin is clear
    top2 = np.sort(want, axis=1)[:, -2:]
    sure = (top2[:, 1] - top2[:, 0]) > 2e-2 * scale
    assert sure.sum() >= TOKENS // 2
    assert np.array_equal(np.argmax(logits, axis=1)[sure], np.argmax(want, axis=1)[sure])


def _swap_decay_and_beta(m):
    for L in m.layers:
        if not L["attention"]:
            L["a"], L["b"] = L["b"], L["a"]


def _post_norm_from_input_norm(m):
    for L in m.layers:
        L["post_norm"] = L["input_norm"]


def _swap_keys_and_values(m):
    for L in m.layers:
        if L["attention"]:
            L["k"], L["v"] = L["v"], L["k"]


@pytest.mark.parametrize("mistake", [_swap_decay_and_beta, _post_norm_from_input_norm, _swap_keys_and_values])
def test_planted_wiring_mistakes_fail_the_check(monkeypatch, mistake):
    """The comparison is tight enough to see plausible wiring mistakes planted in the
    oracle (a and b projections exchanged, the post-attention norm taking the input
    norm's weights, keys and values exchanged): each moves the logits past the bar."""
    spec, oracle_model, tokens, want = _case("baseline")
    mistake(oracle_model)
    logits = _float_oracle_logits(spec, oracle_model, monkeypatch, tokens)
    assert float(np.abs(logits - want).max()) > BAR * float(np.abs(want).max())
