"""A HuggingFace-layout checkpoint (MoE or dense) to a GPU decoder.

Mirrors the reference's native decoder construction
(src/jouleai/native/decoder3.py:86-135 ``NativeDecoder.__init__``,
:213-313 ``_load_fixed``, :329-367 ``_load_experts``) and its architecture
registry (src/jouleai/arch/registry.py:56-94 ``get_spec``):

* ``decoder_shape(config)`` maps config.json to the decoder shape the way
  ``get_spec`` does (head_dim, KV heads, eps, rope theta, vocabulary, QK-norm
  style by model_type, MoE sizes, top-k renormalisation);
* ``load_decoder(model_dir)`` converts the experts to the Q4 store once
  (``convert_experts_q4``, same file format), puts it in HBM, and loads the
  router, norms, attention projections, embedding and lm_head by the
  checkpoint's own tensor names into device tensors; a dense model
  (qwen2, qwen3, llama, mistral) gets a DenseFfnStore and its
  gate/up/down projections as the FFN weights (decoder3.py:251-280);
* ``HipNativeDecoder`` keeps per-sequence KV caches across calls and offers
  ``decode_batch`` / ``decode_batch_argmax`` as NativeDecoder does
  (decoder3.py:580-629).
"""

from __future__ import annotations

import dataclasses
import json
from pathlib import Path

import numpy as np
import torch

from .decoder import DecoderShape, DecoderWeights, HipDecoder, KVCacheSet
from .dense import DenseFfnStore, dense_ffn_shape
from .moe import HbmExpertStore, MoEShape
from .q4_store import BIN_NAME, INDEX_NAME, convert_experts_q4

# model_type -> (per-head QK-norm type as KernelCfg.qk_norm_type, expert naming)
# (registry.py:59-92: qwen3 families norm q/k per head, olmoe over the whole
# vector, the others not at all; mixtral/deepseek name experts block_sparse_moe)
_MOE_TYPES = {"qwen3_moe": (1, "qwen"), "olmoe": (2, "qwen"), "mixtral": (0, "block_sparse_moe"),
              "deepseek": (0, "block_sparse_moe")}
# the dense families the reference's native decoder runs through
# layer_ffn_batch's E == 0 branch (registry.py:50, decoder3.py:251-280);
# gemma's (1 + w) norms and phi / gpt_oss are not taken here
_DENSE_TYPES = {"qwen2": 0, "qwen3": 1, "llama": 0, "mistral": 0}


def decoder_shape(cfg: dict, max_tokens: int = 4096) -> tuple[DecoderShape, str]:
    """(shape, expert naming) of a config.json dict (registry.py:56-94)."""
    mt = cfg.get("model_type", "?")
    if mt not in _MOE_TYPES and mt not in _DENSE_TYPES:
        raise ValueError(f"model_type '{mt}': the GPU decoder runs {', '.join(list(_MOE_TYPES) + list(_DENSE_TYPES))}")
    dense = mt in _DENSE_TYPES
    qk, naming = (_DENSE_TYPES[mt], "qwen") if dense else _MOE_TYPES[mt]
    if cfg.get("q_lora_rank") or cfg.get("kv_lora_rank"):
        raise ValueError("MLA attention (latent KV) is not supported")
    if cfg.get("clip_qkv") is not None:
        # the reference's native decoder does not clamp q/k/v (only its
        # Python streamer does, generic_streamer.py:118-121): refuse rather
        # than decode such a checkpoint differently from either
        raise ValueError("clip_qkv is not supported by the GPU decoder")
    rs = cfg.get("rope_scaling") or (cfg.get("rope_parameters") if isinstance(cfg.get("rope_parameters"), dict)
                                     else None)
    rope_scaling: tuple = ()
    if rs:
        if "type" in rs and "rope_type" not in rs:
            # the older key: the reference's decoder reads rope_type only
            # (decoder3.py:405-410) and would decode with unscaled tables;
            # refuse rather than decode it differently from either reading
            raise ValueError("rope_scaling uses the legacy key 'type'; rename it to 'rope_type'")
        rtype = rs.get("rope_type", "default")
        if rtype == "llama3":
            rope_scaling = tuple(sorted((k, v) for k, v in rs.items() if isinstance(v, (int, float, str))))
        elif rtype != "default":
            # decoder3.py:405-410 handles llama3 only; other types would decode
            # with unscaled tables
            raise ValueError(f"rope_scaling type '{rtype}' is not supported (llama3 only)")
    heads = cfg["num_attention_heads"]
    hd = cfg.get("head_dim") or cfg["hidden_size"] // heads
    if dense:
        moe = dense_ffn_shape(cfg["hidden_size"], cfg["intermediate_size"])
    else:
        moe = MoEShape(d=cfg["hidden_size"], m=cfg.get("moe_intermediate_size") or cfg.get("intermediate_size", 0),
                       E=cfg.get("num_experts", 0), topk=cfg.get("num_experts_per_tok", 0),
                       renorm=bool(cfg.get("norm_topk_prob", False)), name=mt)
    shape = DecoderShape(n_layers=cfg["num_hidden_layers"], moe=moe, n_heads=heads,
                         n_kv=cfg.get("num_key_value_heads", heads), hd=hd,
                         eps=cfg.get("rms_norm_eps", cfg.get("layer_norm_eps", 1e-5)),
                         theta=cfg.get("rope_theta", 1e4), maxT=max_tokens, qk_norm_type=qk,
                         bias_qkv=bool(cfg.get("attention_bias", mt == "qwen2")), V=cfg["vocab_size"], name=mt,
                         rope_scaling=rope_scaling)
    return shape, naming


class _Tensors:
    """name -> tensor over every *.safetensors file of a model directory."""

    def __init__(self, model_dir: Path):
        from safetensors import safe_open

        self._open = safe_open
        self.where: dict[str, Path] = {}
        for fp in sorted(model_dir.glob("*.safetensors")):
            with safe_open(str(fp), framework="pt") as f:
                for k in f.keys():
                    self.where[k] = fp
        if not self.where:
            raise FileNotFoundError(f"no .safetensors files in {model_dir}")

    def __contains__(self, name: str) -> bool:
        return name in self.where

    def get(self, name: str) -> torch.Tensor:
        if name not in self.where:
            raise KeyError(f"tensor {name} not in the checkpoint")
        with self._open(str(self.where[name]), framework="pt") as f:
            return f.get_tensor(name)

    def stack(self, names, dtype=torch.bfloat16) -> torch.Tensor:
        return torch.stack([self.get(n).to(dtype) for n in names])


def _router_name(naming: str) -> str:
    # decoder3.py:291-296
    return "mlp.block_sparse_moe.router" if naming == "block_sparse_moe" else "mlp.gate"


def load_decoder(model_dir: str | Path, max_tokens: int = 4096, converted_dir: str | Path | None = None,
                 group: int = 64, device: str | torch.device = "cuda") -> HipDecoder:
    """The GPU decoder of a checkpoint directory (config.json + safetensors).

    The experts are converted once into ``converted_dir`` (default
    ``<model_dir>/joule_q4``) in the reference's Q4 store format, then copied
    to HBM; the dense weights are loaded by their checkpoint names.  The
    embedding and lm_head (the embedding again when tie_word_embeddings) are
    set, so the returned decoder runs decode_batch_argmax end to end."""
    model_dir = Path(model_dir)
    cfg = json.loads((model_dir / "config.json").read_text())
    shape, naming = decoder_shape(cfg, max_tokens)
    L, moe = shape.n_layers, shape.moe
    T = _Tensors(model_dir)
    lay = [f"model.layers.{l}" for l in range(L)]
    if moe.E == 0:
        store = DenseFfnStore(moe.d, moe.m, L, device=device)
    else:
        out = Path(converted_dir) if converted_dir is not None else model_dir / "joule_q4"
        if not ((out / BIN_NAME).exists() and (out / INDEX_NAME).exists()):
            convert_experts_q4(model_dir, out, L, moe.E, naming=naming, group=group)
        store = HbmExpertStore.from_dir(out, moe, n_layers=L, device=device)
        store.set_router(T.stack([f"{p}.{_router_name(naming)}.weight" for p in lay]).to(device).contiguous())
    # a qwen2-style bias flag without bias tensors runs unbiased (decoder3.py:107-114)
    if shape.bias_qkv and "model.layers.0.self_attn.q_proj.bias" not in T:
        shape = dataclasses.replace(shape, bias_qkv=False)
    t = {
        "norm1": T.stack([f"{p}.input_layernorm.weight" for p in lay]),
        "norm2": T.stack([f"{p}.post_attention_layernorm.weight" for p in lay]),
        "final_norm": T.get("model.norm.weight").to(torch.bfloat16),
        "wq": T.stack([f"{p}.self_attn.q_proj.weight" for p in lay]),
        "wk": T.stack([f"{p}.self_attn.k_proj.weight" for p in lay]),
        "wv": T.stack([f"{p}.self_attn.v_proj.weight" for p in lay]),
        "wo": T.stack([f"{p}.self_attn.o_proj.weight" for p in lay]),
        "embed": T.get("model.embed_tokens.weight").to(torch.bfloat16),
    }
    if shape.qk_norm_type != 0:
        # [hd] per head (qwen3), [H*hd] / [KH*hd] over the whole vector (olmoe)
        t["qn"] = T.stack([f"{p}.self_attn.q_norm.weight" for p in lay])
        t["kn"] = T.stack([f"{p}.self_attn.k_norm.weight" for p in lay])
    if shape.bias_qkv:
        for k, n in (("bq", "q_proj"), ("bk", "k_proj"), ("bv", "v_proj")):
            t[k] = T.stack([f"{p}.self_attn.{n}.bias" for p in lay], torch.float32)
    if moe.E == 0:
        # dense FFN: gate_proj / up_proj / down_proj (decoder3.py:276-280)
        for k, n in (("w1", "gate_proj"), ("w2", "up_proj"), ("w3", "down_proj")):
            t[k] = T.stack([f"{p}.mlp.{n}.weight" for p in lay])
    dec = HipDecoder(store, DecoderWeights(shape, device=device, **t))
    if moe.E == 0:
        store.set_weights(*(dec.weights.t[k] for k in ("w1", "w2", "w3")))
    tied = bool(cfg.get("tie_word_embeddings", False))
    lm = t["embed"] if tied else T.get("lm_head.weight").to(torch.bfloat16)
    dec.set_lm_head(lm.to(device).contiguous())
    return dec


class HipNativeDecoder:
    """NativeDecoder's batch-decode surface (decoder3.py:86, 580-629) on the
    GPU: per-sequence KV caches persist across calls, sequence b of a call
    is the reference's "seq{b}"."""

    def __init__(self, model_dir: str | Path, max_tokens: int = 4096, converted_dir: str | Path | None = None,
                 max_batch: int = 8, device: str | torch.device = "cuda"):
        self.dec = load_decoder(model_dir, max_tokens, converted_dir, device=device)
        self.shape = self.dec.shape
        self.kv = KVCacheSet(self.shape, max_batch, device=device)
        self._seq_pos: dict[str, int] = {}

    def reset(self) -> None:
        """Forget every sequence (the caches are overwritten as positions are reused)."""
        self._seq_pos = {}

    def _embed(self, tokens) -> torch.Tensor:
        tok = torch.as_tensor(np.asarray(tokens, dtype=np.int32), device=self.kv.data.device)
        return self.dec.embed(tok)

    def decode_batch_argmax(self, tokens: list[int], positions: list[int]) -> list[int]:
        """The argmax next token per sequence (decoder3.py:607-629)."""
        out = self.dec.decode_layers_batch_argmax(self._embed(tokens), positions, self.kv)
        for b, p in enumerate(positions):
            self._seq_pos[f"seq{b}"] = p + 1
        return [int(v) for v in out.cpu().tolist()]

    def decode_batch(self, tokens: list[int], positions: list[int]) -> list[int]:
        """The next token per sequence from the full logits (decoder3.py:580-605):
        numpy's argmax of each row, the first index of the maximum."""
        B = len(tokens)
        logits = torch.empty((B, self.shape.V), dtype=torch.float32, device=self.kv.data.device)
        self.dec.decode_layers_batch(self._embed(tokens), positions, self.kv, logits=logits)
        for b, p in enumerate(positions):
            self._seq_pos[f"seq{b}"] = p + 1
        lg = logits.cpu().numpy()
        return [int(lg[b].argmax()) for b in range(B)]

    def prefill(self, tokens: list[int]) -> np.ndarray:
        """NativeDecoder.prefill (decoder3.py:490-509): one prompt into seq0's
        caches; the first-token logits [V]."""
        dev = self.kv.data.device
        logits = torch.empty(self.shape.V, dtype=torch.float32, device=dev)
        self.dec.prefill_layers(torch.as_tensor(np.asarray(tokens, dtype=np.int32), device=dev), self.kv, 0, logits)
        self._seq_pos = {"seq0": len(tokens)}
        return logits.cpu().numpy()

    def prefill_batch(self, prompts: list[list[int]], chunk: int = 512) -> list[np.ndarray]:
        """NativeDecoder.prefill_batch (decoder3.py:512-571): B prompts into
        seq0..seqB-1; the logits [V] after each prompt's last token.  All
        positions of all prompts go through each layer together, in chunks of
        `chunk` tokens taken in position order, where the reference runs one
        decode_layers_batch per position."""
        dev = self.kv.data.device
        B = len(prompts)
        if B > self.kv.B:
            raise ValueError(f"{B} prompts, the cache set holds {self.kv.B} sequences")
        items = sorted(((t, b) for b in range(B) for t in range(len(prompts[b]))))   # position-major
        last = np.zeros((B, self.shape.d), np.float32)
        graph = self.dec.graph
        self.dec.set_graph(False)          # every chunk differs: run eagerly
        try:
            for c0 in range(0, len(items), chunk):
                part = items[c0:c0 + chunk]
                tok = torch.as_tensor(np.asarray([prompts[b][t] for t, b in part], np.int32), device=dev)
                x = self.dec.embed(tok)
                hid = self.dec.decode_layers_batch(x, [t for t, _ in part], self.kv, seqs=[b for _, b in part])
                rows = [i for i, (t, b) in enumerate(part) if t == len(prompts[b]) - 1]
                if rows:
                    h = hid[torch.as_tensor(rows, device=dev)].cpu().numpy()
                    for r, i in enumerate(rows):
                        last[part[i][1]] = h[r]
        finally:
            self.dec.set_graph(graph)
        logits = torch.empty((B, self.shape.V), dtype=torch.float32, device=dev)
        self.dec.lm_head(torch.from_numpy(last).to(dev), logits, None)
        self._seq_pos = {f"seq{b}": len(prompts[b]) for b in range(B)}
        lg = logits.cpu().numpy()
        return [lg[b] for b in range(B)]
