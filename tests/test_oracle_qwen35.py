"""Pins the oracle's Qwen3.5 forward pass (orc_qwen35_step, restating
qwen35.rs:280-516) against an independent implementation: transformers'
Qwen3_5ForCausalLM, the model code the reference's Qwen tests were made from.

The transformers model is built offline from a config with the tiny test
shapes and loaded with the oracle's dequantised weights, mapped the way
llama.cpp's converter maps them the other way (qwen35.rs:9-11): the
zero-centred norms lose the baked-in +1, ssm_a = -exp(A_log), and the value
heads are reordered, since value head j reads key head j % n_k_heads here and
key head j // (n_v/n_k) in transformers.  It runs the whole prompt at once
(its chunked DeltaNet form); the oracle runs token by token (the recurrent
form).  Every layer's output and the logits agree within 1e-4 relative.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd.qwen35 import QWEN35_TINY, QWEN35_TINY_64, Qwen35Weights

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")


def rel(got, want):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)).max()
    return d / np.abs(np.asarray(want, np.float64)).max()


def value_order(cfg):
    """transformers' value head i is this model's head value_order[i]."""
    r = cfg.n_v_heads // cfg.n_k_heads
    return [(i % r) * cfg.n_k_heads + i // r for i in range(cfg.n_v_heads)]


def hf_model(w: Qwen35Weights):
    from transformers import Qwen3_5ForCausalLM, Qwen3_5TextConfig

    cfg = w.cfg
    hc = Qwen3_5TextConfig(
        vocab_size=cfg.n_vocab, hidden_size=cfg.n_embd, intermediate_size=cfg.n_ff,
        num_hidden_layers=cfg.n_layers, num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads,
        head_dim=cfg.head_dim, linear_num_key_heads=cfg.n_k_heads, linear_num_value_heads=cfg.n_v_heads,
        linear_key_head_dim=cfg.k_head_dim, linear_value_head_dim=cfg.v_head_dim,
        linear_conv_kernel_dim=cfg.conv_kernel, rms_norm_eps=cfg.norm_eps, tie_word_embeddings=True,
        max_position_embeddings=4096,
        layer_types=["full_attention" if cfg.is_attention(i) else "linear_attention" for i in range(cfg.n_layers)],
        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                         "partial_rotary_factor": cfg.n_rot / cfg.head_dim})
    hc._attn_implementation = "eager"
    model = Qwen3_5ForCausalLM(hc).float().eval()
    a, n, lf = w.arrays, cfg.n_embd, cfg.layer_format
    t = lambda arr: torch.from_numpy(np.ascontiguousarray(arr, np.float32))

    def deq(key, rows, cols, fmt=lf):
        return oracle.dequantize(int(fmt), a[key], rows * cols).reshape(rows, cols)

    order = value_order(cfg)
    kd, dv = cfg.key_dim, cfg.v_head_dim
    # Row permutation of value-head blocks (of `size` rows each) in a tensor.
    vperm = lambda size: np.concatenate([np.arange(h * size, (h + 1) * size) for h in order])
    sd = {}
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    for il in range(cfg.n_layers):
        p = f"model.layers.{il}."
        sd[p + "input_layernorm.weight"] = t(a[f"{il}.attn_norm"] - 1)
        sd[p + "post_attention_layernorm.weight"] = t(a[f"{il}.ffn_norm"] - 1)
        if cfg.is_attention(il):
            sd[p + "self_attn.q_proj.weight"] = t(deq(f"{il}.wq", 2 * q, n))
            sd[p + "self_attn.k_proj.weight"] = t(deq(f"{il}.wk", kv, n))
            sd[p + "self_attn.v_proj.weight"] = t(deq(f"{il}.wv", kv, n))
            sd[p + "self_attn.o_proj.weight"] = t(deq(f"{il}.wo", n, q))
            sd[p + "self_attn.q_norm.weight"] = t(a[f"{il}.q_norm"] - 1)
            sd[p + "self_attn.k_norm.weight"] = t(a[f"{il}.k_norm"] - 1)
        else:
            qkv = deq(f"{il}.qkv", cfg.conv_dim, n)
            qkv = np.concatenate([qkv[:2 * kd], qkv[2 * kd:][vperm(dv)]])
            taps = a[f"{il}.conv"].reshape(cfg.conv_dim, cfg.conv_kernel)
            taps = np.concatenate([taps[:2 * kd], taps[2 * kd:][vperm(dv)]])
            sd[p + "linear_attn.in_proj_qkv.weight"] = t(qkv)
            sd[p + "linear_attn.in_proj_z.weight"] = t(deq(f"{il}.z", cfg.value_dim, n)[vperm(dv)])
            sd[p + "linear_attn.in_proj_b.weight"] = t(deq(f"{il}.beta", cfg.n_v_heads, n)[order])
            sd[p + "linear_attn.in_proj_a.weight"] = t(deq(f"{il}.alpha", cfg.n_v_heads, n)[order])
            sd[p + "linear_attn.conv1d.weight"] = t(taps.reshape(cfg.conv_dim, 1, cfg.conv_kernel))
            sd[p + "linear_attn.dt_bias"] = t(a[f"{il}.dt_bias"][order])
            sd[p + "linear_attn.A_log"] = t(np.log(-a[f"{il}.a"])[order])
            sd[p + "linear_attn.norm.weight"] = t(a[f"{il}.ssm_norm"])
            sd[p + "linear_attn.out_proj.weight"] = t(deq(f"{il}.out", n, cfg.value_dim)[:, vperm(dv)])
        sd[p + "mlp.gate_proj.weight"] = t(deq(f"{il}.gate", cfg.n_ff, n))
        sd[p + "mlp.up_proj.weight"] = t(deq(f"{il}.up", cfg.n_ff, n))
        sd[p + "mlp.down_proj.weight"] = t(deq(f"{il}.down", n, cfg.n_ff))
    emb = t(deq("token_embd", cfg.n_vocab, n, cfg.embd_format))
    sd["model.embed_tokens.weight"] = emb
    sd["lm_head.weight"] = emb
    sd["model.norm.weight"] = t(a["output_norm"] - 1)
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in k for k in missing), missing
    return model


@pytest.mark.parametrize("cfg", [QWEN35_TINY, QWEN35_TINY_64], ids=lambda c: c.name)
def test_oracle_step_matches_transformers(cfg):
    w = Qwen35Weights(cfg, seed=3)
    model = hf_model(w)
    tokens = np.random.default_rng(4).integers(0, cfg.n_vocab, 10).tolist()
    with torch.no_grad():
        out = model(torch.tensor([tokens]), use_cache=False, output_hidden_states=True)
    logits = out.logits[0].numpy()
    hidden = [h[0].numpy() for h in out.hidden_states]
    state = oracle.Qwen35State(w, n_ctx=32)
    for t, tok in enumerate(tokens):
        lg, (emb, layers, final) = state.step(tok, trace=True)
        assert rel(emb, hidden[0][t]) < 1e-6
        for il in range(cfg.n_layers - 1):
            assert rel(layers[il * cfg.n_embd:(il + 1) * cfg.n_embd], hidden[il + 1][t]) < 1e-4, (t, il)
        assert rel(lg, logits[t]) < 1e-4, t
