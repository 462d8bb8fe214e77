"""Checkpoints (config.json + safetensors, written here at a small size)
loaded into the GPU decoder and decoded token by token, against the oracle
built from the same tensors and the converted store: Qwen3-MoE; OLMoE, with
the whole-vector QK-norm (q_norm [H*hd], k_norm [KH*hd]), no GQA and no
top-k renormalisation; and two dense families, Qwen3 (per-head QK-norm) and
Llama (no QK-norm, tied embedding), whose FFN is layer_ffn_batch's E == 0
branch."""

import json

import numpy as np
import pytest
import torch

from joule_amd.checkpoint import HipNativeDecoder
from joule_amd.decoder import rope_tables
from joule_amd.q4_store import BIN_NAME, INDEX_NAME, Q4Index
from oracle import decoder as D
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CFG = {"model_type": "qwen3_moe", "num_hidden_layers": 2, "hidden_size": 1024, "num_attention_heads": 8,
       "num_key_value_heads": 2, "head_dim": 128, "num_experts": 16, "num_experts_per_tok": 4,
       "moe_intermediate_size": 256, "vocab_size": 1000, "rope_theta": 1000000.0, "rms_norm_eps": 1e-06,
       "norm_topk_prob": True, "tie_word_embeddings": False}
OLMOE_CFG = {"model_type": "olmoe", "num_hidden_layers": 2, "hidden_size": 1024, "num_attention_heads": 8,
             "num_key_value_heads": 8, "num_experts": 16, "num_experts_per_tok": 4, "intermediate_size": 256,
             "vocab_size": 1000, "rope_theta": 10000.0, "rms_norm_eps": 1e-05, "norm_topk_prob": False,
             "clip_qkv": None, "tie_word_embeddings": False}
QWEN3_DENSE_CFG = {"model_type": "qwen3", "num_hidden_layers": 2, "hidden_size": 1024, "num_attention_heads": 8,
                   "num_key_value_heads": 2, "head_dim": 128, "intermediate_size": 3072, "vocab_size": 1000,
                   "rope_theta": 1000000.0, "rms_norm_eps": 1e-06, "tie_word_embeddings": False}
LLAMA_CFG = {"model_type": "llama", "num_hidden_layers": 2, "hidden_size": 1024, "num_attention_heads": 8,
             "num_key_value_heads": 8, "intermediate_size": 2048, "vocab_size": 1000, "rope_theta": 500000.0,
             "rms_norm_eps": 1e-05, "attention_bias": False, "tie_word_embeddings": True}
CFGS = {"qwen3_moe": CFG, "olmoe": OLMOE_CFG, "qwen3": QWEN3_DENSE_CFG, "llama": LLAMA_CFG}
QK = {"qwen3_moe": 1, "olmoe": 2, "qwen3": 1, "llama": 0}


def _dims(c):
    H = c["num_attention_heads"]
    return (c["num_hidden_layers"], c["hidden_size"], H, c["num_key_value_heads"],
            c.get("head_dim") or c["hidden_size"] // H, c.get("num_experts", 0),
            c.get("moe_intermediate_size") or c["intermediate_size"], c["vocab_size"])


def _write_checkpoint(path, c):
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(31)
    L, d, H, KH, hd, E, m, V = _dims(c)
    whole = c["model_type"] == "olmoe"
    qk = c["model_type"] in ("olmoe", "qwen3_moe", "qwen3")
    r = lambda *s, std=0.02: (torch.randn(s, generator=g) * std).to(torch.bfloat16)
    nw = lambda *s: (1.0 + 0.1 * torch.randn(s, generator=g)).to(torch.bfloat16)
    t = {"model.embed_tokens.weight": r(V, d, std=0.5), "lm_head.weight": r(V, d), "model.norm.weight": nw(d)}
    for l in range(L):
        p = f"model.layers.{l}"
        t.update({f"{p}.input_layernorm.weight": nw(d), f"{p}.post_attention_layernorm.weight": nw(d),
                  f"{p}.self_attn.q_proj.weight": r(H * hd, d), f"{p}.self_attn.k_proj.weight": r(KH * hd, d),
                  f"{p}.self_attn.v_proj.weight": r(KH * hd, d), f"{p}.self_attn.o_proj.weight": r(d, H * hd)})
        if qk:
            t.update({f"{p}.self_attn.q_norm.weight": nw(H * hd if whole else hd),
                      f"{p}.self_attn.k_norm.weight": nw(KH * hd if whole else hd)})
        if E == 0:
            t.update({f"{p}.mlp.gate_proj.weight": r(m, d), f"{p}.mlp.up_proj.weight": r(m, d),
                      f"{p}.mlp.down_proj.weight": r(d, m)})
        else:
            t[f"{p}.mlp.gate.weight"] = r(E, d)
        for e in range(E):
            t[f"{p}.mlp.experts.{e}.gate_proj.weight"] = r(m, d)
            t[f"{p}.mlp.experts.{e}.up_proj.weight"] = r(m, d)
            t[f"{p}.mlp.experts.{e}.down_proj.weight"] = r(d, m)
    path.mkdir(parents=True, exist_ok=True)
    save_file(t, str(path / "model.safetensors"))
    (path / "config.json").write_text(json.dumps(c))
    return {k: v.float().numpy() for k, v in t.items()}


@pytest.mark.parametrize("family", list(CFGS))
def test_checkpoint_decode_matches_oracle(tmp_path, family):
    c = CFGS[family]
    model = tmp_path / f"{family}-tiny"
    T = _write_checkpoint(model, c)
    print(f"[checkpoint] loading {family}", flush=True)
    nd = HipNativeDecoder(model, max_tokens=64, max_batch=4)
    L, d, H, KH, hd, E, m, _ = _dims(c)
    lay = [f"model.layers.{l}" for l in range(L)]
    w = {"norm1": np.stack([T[f"{p}.input_layernorm.weight"] for p in lay]),
         "norm2": np.stack([T[f"{p}.post_attention_layernorm.weight"] for p in lay]),
         "final_norm": T["model.norm.weight"],
         "wq": np.stack([T[f"{p}.self_attn.q_proj.weight"] for p in lay]),
         "wk": np.stack([T[f"{p}.self_attn.k_proj.weight"] for p in lay]),
         "wv": np.stack([T[f"{p}.self_attn.v_proj.weight"] for p in lay]),
         "wo": np.stack([T[f"{p}.self_attn.o_proj.weight"] for p in lay])}
    if QK[family]:
        w["qn"] = np.stack([T[f"{p}.self_attn.q_norm.weight"] for p in lay])
        w["kn"] = np.stack([T[f"{p}.self_attn.k_norm.weight"] for p in lay])
    w["cos"], w["sin"] = rope_tables(64, hd, c["rope_theta"])
    if E == 0:
        for key, n in (("w1", "gate_proj"), ("w2", "up_proj"), ("w3", "down_proj")):
            w[key] = np.stack([T[f"{p}.mlp.{n}.weight"] for p in lay])
        moe = None
    else:
        conv = model / "joule_q4"
        blob = np.fromfile(conv / BIN_NAME, dtype=np.uint8)
        offsets = Q4Index.load(conv / INDEX_NAME).offset_table(L, E)
        moe = [O.OracleMoE(d, m, E, c["num_experts_per_tok"], c["norm_topk_prob"], 64, T[f"{p}.mlp.gate.weight"],
                           blob, offsets[:, l * E:(l + 1) * E]) for l, p in enumerate(lay)]
    oracle = D.OracleDecoder(L, d, H, KH, hd, c["rms_norm_eps"], QK[family], False, w, moe)
    W_lm = T["model.embed_tokens.weight"] if c["tie_word_embeddings"] else T["lm_head.weight"]
    kv = [[(np.zeros((64, KH, hd), np.float32), np.zeros((64, KH, hd), np.float32)) for _ in range(L)]
          for _ in range(4)]
    tokens, pos = [5, 999, 0, 123], [0, 0, 0, 0]
    for step in range(4):
        print(f"[checkpoint] step {step} tokens {tokens}", flush=True)
        got = nd.decode_batch_argmax(tokens, pos)
        x = D.embed_lookup(T["model.embed_tokens.weight"], tokens)
        lg = D.lm_head(W_lm, oracle.decode_layers_batch(x, pos, kv))
        want = D.argmax_strict(lg)
        top2 = np.sort(lg, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 1e-3 * np.abs(top2[:, 1])
        assert np.array_equal(np.asarray(got)[clear], want[clear]), (got, want)
        tokens = [int(v) for v in want]          # follow the oracle's sequence
        pos = [p + 1 for p in pos]
    # the logits path (numpy argmax of the rows) agrees on the same step
    a = nd.decode_batch(tokens, pos)
    b = nd.decode_batch_argmax(tokens, pos)
    assert a == b
    nd.dec.store.close()
