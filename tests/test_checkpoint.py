"""config.json -> decoder shape, the registry mapping (registry.py:56-94), on the CPU."""

import pytest

from joule_amd.checkpoint import decoder_shape

# Qwen3-30B-A3B's published config.json values (the fields the decoder reads)
QWEN3_30B = {
    "model_type": "qwen3_moe", "num_hidden_layers": 48, "hidden_size": 2048, "num_attention_heads": 32,
    "num_key_value_heads": 4, "head_dim": 128, "num_experts": 128, "num_experts_per_tok": 8,
    "moe_intermediate_size": 768, "intermediate_size": 6144, "vocab_size": 151936, "rope_theta": 1000000.0,
    "rms_norm_eps": 1e-06, "norm_topk_prob": True, "tie_word_embeddings": False, "attention_bias": False,
}


def test_qwen3_30b_shape():
    s, naming = decoder_shape(QWEN3_30B, max_tokens=2176)
    assert naming == "qwen"
    assert (s.n_layers, s.d, s.n_heads, s.n_kv, s.hd, s.V) == (48, 2048, 32, 4, 128, 151936)
    assert (s.moe.d, s.moe.m, s.moe.E, s.moe.topk, s.moe.renorm) == (2048, 768, 128, 8, True)
    assert s.qk_norm_type == 1 and s.theta == 1e6 and s.eps == 1e-6 and s.maxT == 2176 and not s.bias_qkv
    c = s.kernel_cfg()
    assert (c.L, c.d, c.n_heads, c.n_kv, c.hd, c.E, c.topk, c.V, c.intermediate) == \
        (48, 2048, 32, 4, 128, 128, 8, 151936, 768)
    assert c.norm_topk_prob == 1 and c.qk_norm_type == 1 and c.maxT == 2176


def test_registry_defaults_and_families():
    olmoe = {"model_type": "olmoe", "num_hidden_layers": 16, "hidden_size": 2048, "num_attention_heads": 16,
             "num_experts": 64, "num_experts_per_tok": 8, "intermediate_size": 1024, "vocab_size": 50304}
    s, naming = decoder_shape(olmoe)
    # head_dim from hidden / heads, KV heads default to the query heads, eps
    # and theta defaults, no renormalisation, whole-vector QK-norm
    assert (s.hd, s.n_kv, s.eps, s.theta, s.moe.m, s.moe.renorm, s.qk_norm_type) == \
        (128, 16, 1e-5, 1e4, 1024, False, 2)
    mix = dict(olmoe, model_type="mixtral", num_key_value_heads=8)
    s, naming = decoder_shape(mix)
    assert naming == "block_sparse_moe" and s.qk_norm_type == 0 and s.n_kv == 8
    with pytest.raises(ValueError):
        decoder_shape(dict(olmoe, model_type="qwen3"))          # dense: not the MoE path
    with pytest.raises(ValueError):
        decoder_shape(dict(olmoe, model_type="deepseek", kv_lora_rank=512))   # MLA attention
