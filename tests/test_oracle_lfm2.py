"""Pins the oracle's LFM2 forward pass (orc_lfm2_step, restating lfm2.rs:308-560)
against an independent implementation: transformers' Lfm2ForCausalLM (and
Lfm2MoeForCausalLM for the mixture-of-experts block, lfm2.rs:413-440, 691-709), the
same model code the reference's own model tests were generated from
(tools/ref_dump.py, lfm2_reference.rs:1-7).

The transformers model is built offline from a config with the tiny test
shapes, loaded with the oracle's dequantised weights, and run over the whole
prompt at once (no cache); the oracle runs the prompt token by token with its
KV cache and convolution state.  Logits and every layer's output must agree
within 1e-4 relative, the reference's float tolerance (lfm2_reference.rs:17-19).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd.lfm2 import LFM2_TINY, LFM2_TINY_F16, LFM2_TINY_MOE, Lfm2Weights

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")


def rel(got, want):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)).max()
    return d / np.abs(np.asarray(want, np.float64)).max()


def hf_model(w: Lfm2Weights):
    from transformers import Lfm2Config, Lfm2ForCausalLM, Lfm2MoeConfig, Lfm2MoeForCausalLM

    cfg = w.cfg
    moe = cfg.n_experts > 0
    # The MoE model (Lfm2MoeForCausalLM) is the one transformers implements the
    # LFM2-MoE router in: sigmoid scores, top-k of score + expert_bias,
    # weights normalised over the picks (+1e-6), scaling factor 1.
    config_cls, model_cls = (Lfm2MoeConfig, Lfm2MoeForCausalLM) if moe else (Lfm2Config, Lfm2ForCausalLM)
    extra = dict(moe_intermediate_size=cfg.n_ff_expert, num_experts=cfg.n_experts,
                 num_experts_per_tok=cfg.n_experts_used, num_dense_layers=cfg.n_dense_layers,
                 norm_topk_prob=True, routed_scaling_factor=1.0, use_expert_bias=True) if moe else \
        dict(block_auto_adjust_ff_dim=False)
    hc = config_cls(
        vocab_size=cfg.n_vocab, hidden_size=cfg.n_embd, intermediate_size=cfg.n_ff,
        num_hidden_layers=cfg.n_layers, num_attention_heads=cfg.n_heads,
        num_key_value_heads=cfg.n_kv_heads, max_position_embeddings=4096, norm_eps=cfg.norm_eps,
        conv_L_cache=cfg.conv_kernel, conv_bias=False,
        layer_types=["full_attention" if i in cfg.attention_layers else "conv" for i in range(cfg.n_layers)],
        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta}, tie_word_embeddings=True, **extra)
    hc._attn_implementation = "eager"
    model = model_cls(hc).float().eval()
    n = cfg.n_embd
    a = w.arrays

    def deq(key, fmt, rows, cols):
        return torch.from_numpy(oracle.dequantize(int(fmt), a[key], rows * cols).reshape(rows, cols))

    sd = {}
    lf = cfg.layer_format
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    for il in range(cfg.n_layers):
        p = f"model.layers.{il}."
        sd[p + "operator_norm.weight"] = torch.from_numpy(a[f"{il}.attn_norm"])
        sd[p + "ffn_norm.weight"] = torch.from_numpy(a[f"{il}.ffn_norm"])
        if il in cfg.attention_layers:
            sd[p + "self_attn.q_proj.weight"] = deq(f"{il}.wq", lf, q, n)
            sd[p + "self_attn.k_proj.weight"] = deq(f"{il}.wk", lf, kv, n)
            sd[p + "self_attn.v_proj.weight"] = deq(f"{il}.wv", lf, kv, n)
            sd[p + "self_attn.out_proj.weight"] = deq(f"{il}.wo", lf, n, q)
            sd[p + "self_attn.q_layernorm.weight"] = torch.from_numpy(a[f"{il}.q_norm"])
            sd[p + "self_attn.k_layernorm.weight"] = torch.from_numpy(a[f"{il}.k_norm"])
        else:
            sd[p + "conv.in_proj.weight"] = deq(f"{il}.in_proj", lf, 3 * n, n)
            sd[p + "conv.out_proj.weight"] = deq(f"{il}.out_proj", lf, n, n)
            sd[p + "conv.conv.weight"] = torch.from_numpy(a[f"{il}.taps"].reshape(n, 1, cfg.conv_kernel))
        if cfg.is_moe(il):
            ne, nff = cfg.n_experts, cfg.n_ff_expert
            gate = deq(f"{il}.gate_exps", lf, ne * nff, n).reshape(ne, nff, n)
            up = deq(f"{il}.up_exps", lf, ne * nff, n).reshape(ne, nff, n)
            sd[p + "feed_forward.experts.gate_up_proj"] = torch.cat([gate, up], dim=1)
            sd[p + "feed_forward.experts.down_proj"] = deq(f"{il}.down_exps", lf, ne * n, nff).reshape(ne, n, nff)
            sd[p + "feed_forward.gate.weight"] = torch.from_numpy(a[f"{il}.router"].reshape(ne, n))
            sd[p + "feed_forward.expert_bias"] = torch.from_numpy(a[f"{il}.expert_bias"])
        else:
            sd[p + "feed_forward.w1.weight"] = deq(f"{il}.gate", lf, cfg.n_ff, n)
            sd[p + "feed_forward.w3.weight"] = deq(f"{il}.up", lf, cfg.n_ff, n)
            sd[p + "feed_forward.w2.weight"] = deq(f"{il}.down", lf, n, cfg.n_ff)
    emb = deq("token_embd", cfg.embd_format, cfg.n_vocab, n)
    sd["model.embed_tokens.weight"] = emb
    sd["lm_head.weight"] = emb
    sd["model.embedding_norm.weight"] = torch.from_numpy(a["output_norm"])
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in k for k in missing), missing
    return model


@pytest.mark.parametrize("cfg", [LFM2_TINY, LFM2_TINY_F16, LFM2_TINY_MOE], ids=lambda c: c.name)
def test_oracle_step_matches_transformers(cfg):
    w = Lfm2Weights(cfg, seed=3)
    model = hf_model(w)
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, cfg.n_vocab, 12).tolist()
    with torch.no_grad():
        out = model(torch.tensor([tokens]), use_cache=False, output_hidden_states=True)
    logits = out.logits[0].numpy()
    hidden = [h[0].numpy() for h in out.hidden_states]  # embeddings, then each layer
    state = oracle.Lfm2State(w, n_ctx=32)
    for t, tok in enumerate(tokens):
        lg, (emb, layers, final) = state.step(tok, trace=True)
        assert rel(emb, hidden[0][t]) < 1e-6
        for il in range(cfg.n_layers - 1):
            assert rel(layers[il * cfg.n_embd:(il + 1) * cfg.n_embd], hidden[il + 1][t]) < 1e-4, (t, il)
        assert rel(lg, logits[t]) < 1e-4, t
        assert int(np.argmax(lg)) == int(np.argmax(logits[t]))
