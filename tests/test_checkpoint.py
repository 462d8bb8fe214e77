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
    # dense families: no experts, the FFN of intermediate_size; qwen2's
    # attention bias by default, qwen3's per-head QK-norm
    s, _ = decoder_shape(dict(olmoe, model_type="qwen3"))
    assert (s.moe.E, s.moe.topk, s.moe.m, s.qk_norm_type, s.bias_qkv) == (0, 0, 1024, 1, False)
    s, _ = decoder_shape(dict(olmoe, model_type="qwen2"))
    assert (s.moe.E, s.qk_norm_type, s.bias_qkv) == (0, 0, True)
    s, _ = decoder_shape(dict(olmoe, model_type="llama", attention_bias=False))
    assert (s.moe.E, s.qk_norm_type, s.bias_qkv) == (0, 0, False)
    with pytest.raises(ValueError):
        decoder_shape(dict(olmoe, model_type="gemma"))          # (1 + w) norms: not taken
    with pytest.raises(ValueError):
        decoder_shape(dict(olmoe, model_type="deepseek", kv_lora_rank=512))   # MLA attention


def test_clip_qkv_and_unknown_rope_scaling_are_refused():
    # the reference keeps both fields (registry.py:76-79); the GPU decoder
    # implements llama3 scaling and refuses what it would otherwise drop
    with pytest.raises(ValueError, match="clip_qkv"):
        decoder_shape(dict(QWEN3_30B, clip_qkv=8.0))
    with pytest.raises(ValueError, match="yarn"):
        decoder_shape(dict(QWEN3_30B, rope_scaling={"rope_type": "yarn", "factor": 4.0}))
    s, _ = decoder_shape(dict(QWEN3_30B, rope_scaling={"rope_type": "default"}))
    assert s.rope_scaling == ()
    s, _ = decoder_shape(dict(QWEN3_30B, rope_parameters={"rope_type": "llama3", "factor": 8.0}))
    assert dict(s.rope_scaling)["rope_type"] == "llama3"
    # the legacy key: the reference's decoder reads rope_type only and would
    # decode unscaled, so it is refused rather than read either way
    with pytest.raises(ValueError, match="legacy key 'type'"):
        decoder_shape(dict(QWEN3_30B, rope_scaling={"type": "llama3", "factor": 8.0}))


def test_llama3_rope_tables():
    """generic_streamer.py:21-39, pinned by its three regimes: wavelengths
    below orig_max / high_freq_factor keep the base frequency, those above
    orig_max / low_freq_factor are divided by the factor, and in between the
    frequency is the linear blend with smooth = (orig_max / wavelen - low) /
    (high - low); the tables are cos/sin of pos * inv, duplicated halves."""
    import numpy as np

    from joule_amd.decoder import llama3_inv_freq, rope_tables

    hd, theta = 128, 500000.0
    sc = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_tokens": 8192}
    import torch

    # the base frequencies as the reference computes them: torch's float32
    # pow (generic_streamer.py:23; numpy's float32 pow differs in the last bit
    # for some exponents)
    base = (1.0 / (theta ** (torch.arange(0, hd, 2).float() / hd))).numpy()
    inv = llama3_inv_freq(hd, theta, sc)
    wl = 2 * np.pi / base.astype(np.float64)
    hi, lo = wl < 8192 / 4.0, wl > 8192 / 1.0
    mid = ~hi & ~lo
    assert hi.any() and lo.any() and mid.any()       # all three regimes occur at this shape
    assert np.array_equal(inv[hi], base[hi])
    np.testing.assert_allclose(inv[lo], base[lo] / 8.0, rtol=1e-7)
    smooth = (8192 / wl[mid] - 1.0) / 3.0
    np.testing.assert_allclose(inv[mid], (1 - smooth) * base[mid] / 8.0 + smooth * base[mid], rtol=1e-6)
    # blended frequencies lie between the two ends
    assert np.all(inv[mid] <= base[mid]) and np.all(inv[mid] >= base[mid] / 8.0)
    # the divided frequencies are the float64 quotient rounded to float32
    assert np.array_equal(inv[lo].view(np.uint32),
                          (base[lo].astype(np.float64) / 8.0).astype(np.float32).view(np.uint32))
    cos, sin = rope_tables(16, hd, theta, tuple(sorted(sc.items())))
    ang = (np.arange(16, dtype=np.float64)[:, None] * inv.astype(np.float64)[None, :])
    emb = np.concatenate([ang, ang], axis=1).astype(np.float32)
    assert np.array_equal(cos, np.cos(emb)) and np.array_equal(sin, np.sin(emb))
    c0, _ = rope_tables(16, hd, theta)
    assert not np.array_equal(c0, cos)
