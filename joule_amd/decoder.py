"""Batch decode over all layers on the GPU: the reference's
``decode_layers_batch`` (src/jouleai/native/decode_kernel.c:1518-1556).

Host-side mirror of the reference's native decoder surface
(src/jouleai/native/decoder3.py:35-69, 402-415, 453-490):

* ``KernelW`` / ``KVCache`` are the reference's ctypes structures, filled
  with device pointers of torch tensors;
* ``rope_tables`` builds the cos/sin tables as ``NativeDecoder._rope_tables``
  does (rotate-half layout, ``emb = cat(freqs, freqs)``);
* ``KVCacheSet`` holds the bf16 caches of B sequences x L layers and the
  ``KVCache[B*L]`` array (entry b*L + l) the call takes;
* ``HipDecoder.decode_layers_batch(x, positions, kv)`` runs every layer
  (attention, then the store's MoE block) and returns the final-normed hidden
  state [B, d].  The lm_head is applied by the caller.

The arithmetic is in libjoule_amd.so; PyTorch holds device memory.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .moe import HbmExpertStore, MoEShape

_vp = ctypes.c_void_p


class KernelW(ctypes.Structure):
    """KernelW (decode_kernel.c:288-325; decoder3.py:49-69), field for field."""
    _fields_ = [
        ("embed", _vp), ("lm_head", _vp), ("final_norm", _vp),
        ("norm1", _vp), ("norm2", _vp),
        ("wq", _vp), ("wk", _vp), ("wv", _vp), ("wo", _vp),
        ("bq", _vp), ("bk", _vp), ("bv", _vp),
        ("qn", _vp), ("kn", _vp), ("gate_w", _vp),
        ("w1", _vp), ("w2", _vp), ("w3", _vp),
        ("wq_i8", _vp), ("wq_i8s", _vp), ("wk_i8", _vp), ("wk_i8s", _vp),
        ("wv_i8", _vp), ("wv_i8s", _vp), ("wo_i8", _vp), ("wo_i8s", _vp),
        ("lm_i8", _vp), ("lm_i8s", _vp),
        ("expert_pk", _vp * 3), ("expert_sc", _vp * 3),
        ("cos", _vp), ("sin", _vp),
        ("use_i8", ctypes.c_int),
    ]


class KVCache(ctypes.Structure):
    """KVCache (decode_kernel.c:328-331): one sequence's k, v of one layer."""
    _fields_ = [("k", _vp), ("v", _vp)]


@dataclass(frozen=True)
class DecoderShape:
    """Attention shape of the decoder around an MoE block."""

    n_layers: int
    moe: MoEShape
    n_heads: int
    n_kv: int
    hd: int = 128
    eps: float = 1e-6
    theta: float = 1e6
    maxT: int = 4096
    qk_norm_type: int = 1        # 1: per-head RMSNorm on q and k (Qwen3); 2: over the whole q and k vectors (OLMoE)
    bias_qkv: bool = False
    V: int = 0                   # vocabulary (embedding / lm_head rows); 0: none
    name: str = ""
    # RoPE scaling of config.json as sorted (key, value) pairs; only
    # rope_type "llama3" changes the tables (decoder3.py:405-407)
    rope_scaling: tuple = ()

    @property
    def d(self) -> int:
        return self.moe.d

    def kernel_cfg(self) -> _lib.KernelCfg:
        c = self.moe.kernel_cfg(self.n_layers)
        c.n_heads, c.n_kv, c.hd = self.n_heads, self.n_kv, self.hd
        c.eps, c.maxT = float(self.eps), int(self.maxT)
        c.qk_norm_type, c.bias_qkv = int(self.qk_norm_type), int(bool(self.bias_qkv))
        c.V = int(self.V)
        return c


def qwen3_30b_a3b(n_layers: int = 48, maxT: int = 4096, V: int = 151936) -> DecoderShape:
    """Qwen3-30B-A3B: 48 layers, d 2048, GQA 32 / 4 heads of 128, per-head
    QK-norm, RoPE theta 1e6, eps 1e-6, vocabulary 151936, and the Qwen3 MoE
    block."""
    from .moe import QWEN3
    return DecoderShape(n_layers=n_layers, moe=QWEN3, n_heads=32, n_kv=4, hd=128, eps=1e-6,
                        theta=1e6, maxT=maxT, qk_norm_type=1, V=V, name="qwen3-30b-a3b")


def llama3_inv_freq(hd: int, theta: float, scaling: dict) -> np.ndarray:
    """Inverse frequencies of rope_type "llama3" (generic_streamer.py:21-39):
    the float32 base frequencies 1 / theta^(2i/hd), unchanged above the
    high-frequency wavelength bound, divided by `factor` below the
    low-frequency one, and blended linearly in between; float32 out.  The
    base frequencies come from torch's float32 pow on the CPU, as the
    reference computes them: numpy's float32 pow differs from it in the last
    bit for some exponents."""
    inv = (1.0 / (theta ** (torch.arange(0, hd, 2).float() / hd))).numpy().astype(np.float32)
    orig_max = float(scaling.get("original_max_position_tokens", 8192))
    factor = float(scaling.get("factor", 1.0))
    low_f = float(scaling.get("low_freq_factor", 1.0))
    high_f = float(scaling.get("high_freq_factor", 4.0))
    low_w, high_w = orig_max / low_f, orig_max / high_f
    out = inv.copy()
    for i, f in enumerate(inv.tolist()):
        wavelen = 2 * 3.141592653589793 / f
        if wavelen < high_w:
            out[i] = f
        elif wavelen > low_w:
            out[i] = f / factor
        else:
            smooth = (orig_max / wavelen - low_f) / (high_f - low_f)
            out[i] = (1 - smooth) * (f / factor) + smooth * f
    return out


def rope_tables(maxT: int, hd: int, theta: float, rope_scaling=None) -> tuple[np.ndarray, np.ndarray]:
    """cos, sin [maxT, hd] float32 as NativeDecoder._rope_tables
    (decoder3.py:402-415): inv = 1 / theta^(2i/hd) in float64 (or the llama3
    frequencies when rope_scaling says rope_type "llama3"), angles pos * inv,
    emb = cat(angles, angles) rounded to float32, then cos/sin."""
    sc = dict(rope_scaling or ())
    if sc.get("rope_type") == "llama3":
        inv = llama3_inv_freq(hd, theta, sc).astype(np.float64)
    else:
        inv = 1.0 / (theta ** (np.arange(0, hd, 2).astype(np.float64) / hd))
    pos = np.arange(maxT).astype(np.float64)[:, None]
    fr = pos * inv[None, :]
    emb = np.concatenate([fr, fr], axis=-1).astype(np.float32)
    return np.cos(emb), np.sin(emb)


def _bf16_dev(t: torch.Tensor, shape, name: str, device) -> torch.Tensor:
    if t.dtype != torch.bfloat16 or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be bfloat16 {tuple(shape)}, got {t.dtype} {tuple(t.shape)}")
    return t.to(device).contiguous()


class DecoderWeights:
    """The dense (non-expert) weights of every layer, on the device.

    bf16 tensors: norm1/norm2 [L, d], final_norm [d], wq [L, H*hd, d],
    wk/wv [L, KH*hd, d], wo [L, d, H*hd], qn/kn [L, hd] (per-head QK-norm)
    or [L, H*hd] / [L, KH*hd] (whole-vector QK-norm); float32 biases
    bq [L, H*hd], bk/bv [L, KH*hd] when the shape has bias_qkv; for a
    dense model (shape.moe.E == 0) the FFN's w1/w2 [L, m, d] and w3
    [L, d, m]; optional embed [V, d] (bf16).  The rope tables are built
    from the shape.  The lm_head goes to the store (HipDecoder.set_lm_head).
    """

    def __init__(self, shape: DecoderShape, device="cuda", **t: torch.Tensor):
        L, d, H, KH, hd = shape.n_layers, shape.d, shape.n_heads, shape.n_kv, shape.hd
        self.shape = shape
        want = {"norm1": (L, d), "norm2": (L, d), "final_norm": (d,), "wq": (L, H * hd, d),
                "wk": (L, KH * hd, d), "wv": (L, KH * hd, d), "wo": (L, d, H * hd)}
        if shape.qk_norm_type == 1:
            want.update(qn=(L, hd), kn=(L, hd))
        elif shape.qk_norm_type == 2:
            # whole-vector weights, as decoder3.py:244-248 sizes them
            want.update(qn=(L, H * hd), kn=(L, KH * hd))
        if shape.moe.E == 0:
            # a dense model's FFN (decoder3.py:251-258)
            m = shape.moe.m
            want.update(w1=(L, m, d), w2=(L, m, d), w3=(L, d, m))
        self.t: dict[str, torch.Tensor] = {}
        for k, shp in want.items():
            if k not in t:
                raise ValueError(f"missing weight {k}")
            self.t[k] = _bf16_dev(t[k], shp, k, device)
        if shape.bias_qkv:
            for k, shp in (("bq", (L, H * hd)), ("bk", (L, KH * hd)), ("bv", (L, KH * hd))):
                self.t[k] = t[k].to(device=device, dtype=torch.float32).contiguous()
        if "embed" in t:
            self.t["embed"] = _bf16_dev(t["embed"], (shape.V, d), "embed", device)
        cos, sin = rope_tables(shape.maxT, hd, shape.theta, shape.rope_scaling)
        self.t["cos"] = torch.from_numpy(cos).to(device)
        self.t["sin"] = torch.from_numpy(sin).to(device)

    def kernel_w(self) -> KernelW:
        w = KernelW()
        for k, v in self.t.items():
            setattr(w, k, v.data_ptr())
        return w


class KVCacheSet:
    """Caches for B sequences x L layers: one tensor [B, L, 2, maxT, KH, hd]
    and the KVCache[B*L] array (entry b*L + l) that points into it.  bfloat16
    by default; float32 is the reference's own KVCache type
    (decode_kernel.c:328-331)."""

    def __init__(self, shape: DecoderShape, B: int, device="cuda", data: torch.Tensor | None = None,
                 dtype: torch.dtype = torch.bfloat16):
        L, KH, hd, T = shape.n_layers, shape.n_kv, shape.hd, shape.maxT
        full = (B, L, 2, T, KH, hd)
        if data is None:
            data = torch.zeros(full, dtype=dtype, device=device)
        if data.dtype not in (torch.bfloat16, torch.float32) or tuple(data.shape) != full or not data.is_contiguous():
            raise ValueError(f"cache must be a contiguous bfloat16 or float32 tensor {full}")
        self.shape, self.B, self.data = shape, B, data
        self.table = (KVCache * (B * L))()
        for b in range(B):
            for l in range(L):
                self.table[b * L + l].k = data[b, l, 0].data_ptr()
                self.table[b * L + l].v = data[b, l, 1].data_ptr()

    def k(self, b: int, l: int) -> torch.Tensor:
        return self.data[b, l, 0]

    def v(self, b: int, l: int) -> torch.Tensor:
        return self.data[b, l, 1]


class HipDecoder:
    """decode_layers_batch over an HBM expert store (or, for a dense model,
    a DenseFfnStore) and the attention weights."""

    def __init__(self, store: HbmExpertStore, weights: DecoderWeights, graph: bool = True):
        shape = weights.shape
        if store.shape != shape.moe or store.n_layers != shape.n_layers:
            raise ValueError("store and decoder shapes differ")
        self.store, self.weights, self.shape = store, weights, shape
        self._cfg = shape.kernel_cfg()
        self._w = weights.kernel_w()
        self.set_graph(graph)

    def set_graph(self, enable: bool) -> None:
        """Replay each step from a captured HIP graph (re-recorded when the
        buffers, batch size or attention split count change)."""
        _lib.check(_lib.lib().jm_store_decode_graph(self.store._h, int(bool(enable))), "jm_store_decode_graph")
        self.graph = bool(enable)

    def decode_layers_batch(self, x: torch.Tensor, positions, kv: KVCacheSet,
                            hidden: torch.Tensor | None = None, logits: torch.Tensor | None = None,
                            stream=None, seqs=None) -> torch.Tensor:
        """hidden [B, d] = final RMSNorm of the residual stream after every
        layer, for tokens x [B, d] (float32) writing cache rows positions[b];
        with logits [B, V] (float32, CUDA) also the lm_head of it.  Token b
        uses sequence b's caches, or sequence seqs[b]'s."""
        if x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous() or x.dim() != 2:
            raise ValueError("x must be a contiguous float32 CUDA tensor [B, d]")
        B = x.shape[0]
        pos = self._positions(positions, B)
        if hidden is None:
            hidden = torch.empty_like(x)
        if logits is not None and (logits.dtype != torch.float32 or tuple(logits.shape) != (B, self.shape.V)
                                   or not logits.is_contiguous()):
            raise ValueError(f"logits must be a contiguous float32 tensor [{B}, {self.shape.V}]")
        self._kv_dtype(kv)
        _lib.check(_lib.lib().jm_decode_layers_batch(
            self.store._h, ctypes.byref(self._cfg), ctypes.byref(self._w), self._table(kv, B, seqs),
            pos.ctypes.data_as(ctypes.c_void_p), _lib.ptr(x), B, _lib.ptr(logits), _lib.ptr(hidden),
            _lib.stream_handle(stream)), "jm_decode_layers_batch")
        return hidden

    def lm_head(self, x: torch.Tensor, logits: torch.Tensor | None = None,
                out_tok: torch.Tensor | None = None, stream=None):
        """The store's lm_head on x [B, d]: (logits [B, V], out_tok [B])."""
        B = x.shape[0]
        _lib.check(_lib.lib().jm_lm_head(self.store._h, _lib.ptr(x), B, _lib.ptr(logits), _lib.ptr(out_tok),
                                         _lib.stream_handle(stream)), "jm_lm_head")
        return logits, out_tok

    def set_lm_head(self, lm_head: torch.Tensor) -> None:
        """The lm_head [V, d]: bfloat16, or float32 holding bf16 values (as
        the reference widens it); the store keeps a bf16 copy."""
        V, d = self.shape.V, self.shape.d
        if tuple(lm_head.shape) != (V, d) or not lm_head.is_cuda or not lm_head.is_contiguous():
            raise ValueError(f"lm_head must be a contiguous CUDA tensor [{V}, {d}]")
        if lm_head.dtype == torch.bfloat16:
            dt = _lib.JM_DTYPE_BF16
        elif lm_head.dtype == torch.float32:
            dt = _lib.JM_DTYPE_F32
        else:
            raise ValueError("lm_head dtype must be bfloat16 or float32")
        _lib.check(_lib.lib().jm_store_set_lm_head(self.store._h, _lib.ptr(lm_head), dt, V), "jm_store_set_lm_head")

    def _kv_dtype(self, kv: KVCacheSet) -> None:
        """The store reads and appends caches of kv's element type."""
        dt = _lib.JM_DTYPE_F32 if kv.data.dtype == torch.float32 else _lib.JM_DTYPE_BF16
        if getattr(self, "_kvdt", None) != dt:
            _lib.check(_lib.lib().jm_store_set_kv_dtype(self.store._h, dt), "jm_store_set_kv_dtype")
            self._kvdt = dt

    def _positions(self, positions, B):
        pos = np.ascontiguousarray(np.asarray(positions, dtype=np.int32).reshape(-1))
        if pos.size != B:
            raise ValueError("one position per token")
        return pos

    def _table(self, kv: KVCacheSet, B: int, seqs=None):
        """The KVCache[B*L] argument: sequence b's caches for token b, or
        sequence seqs[b]'s (several tokens of one sequence in a prefill)."""
        L = self.shape.n_layers
        if seqs is not None:
            seqs = [int(q) for q in seqs]
            if len(seqs) != B or min(seqs) < 0 or max(seqs) >= kv.B:
                raise ValueError("seqs: one sequence index per token, each below the cache set's size")
            table = (KVCache * (B * L))()
            for b, q in enumerate(seqs):
                for l in range(L):
                    table[b * L + l] = kv.table[q * L + l]
            self._table_keep = table        # alive until the call has staged it
            return ctypes.cast(table, _vp)
        if kv.B < B:
            raise ValueError(f"cache set holds {kv.B} sequences, batch has {B}")
        table = kv.table if kv.B == B else (KVCache * (B * L)).from_buffer(kv.table)
        return ctypes.cast(table, _vp)

    def prefill_layers(self, tokens: torch.Tensor, kv: KVCacheSet, seq: int = 0,
                       logits: torch.Tensor | None = None, stream=None) -> torch.Tensor | None:
        """prefill_layers (decode_kernel.c:1606-1615): a prompt (int32 CUDA
        tokens [T]) through every layer into sequence seq's caches, rows
        0..T-1; returns the last position's logits [V] when given a tensor."""
        if tokens.dtype != torch.int32 or not tokens.is_cuda or not tokens.is_contiguous():
            raise ValueError("tokens must be a contiguous int32 CUDA tensor")
        L = self.shape.n_layers
        if not 0 <= seq < kv.B:
            raise ValueError("seq outside the cache set")
        table = (KVCache * L).from_buffer(kv.table, seq * L * ctypes.sizeof(KVCache))
        self._kv_dtype(kv)
        _lib.check(_lib.lib().jm_prefill_layers(
            self.store._h, ctypes.byref(self._cfg), ctypes.byref(self._w), ctypes.cast(table, _vp),
            _lib.ptr(tokens), tokens.numel(), _lib.ptr(logits), _lib.stream_handle(stream)), "jm_prefill_layers")
        return logits

    def decode_layers_batch_argmax(self, x: torch.Tensor, positions, kv: KVCacheSet,
                                   out_tok: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """out_tok [B] (int32, CUDA): the argmax token of every sequence, as
        decode_layers_batch_argmax (decode_kernel.c:1560-1590)."""
        if x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous() or x.dim() != 2:
            raise ValueError("x must be a contiguous float32 CUDA tensor [B, d]")
        B = x.shape[0]
        pos = self._positions(positions, B)
        if out_tok is None:
            out_tok = torch.empty(B, dtype=torch.int32, device=x.device)
        self._kv_dtype(kv)
        _lib.check(_lib.lib().jm_decode_layers_batch_argmax(
            self.store._h, ctypes.byref(self._cfg), ctypes.byref(self._w), self._table(kv, B),
            pos.ctypes.data_as(ctypes.c_void_p), _lib.ptr(x), B, _lib.ptr(out_tok), None,
            _lib.stream_handle(stream)), "jm_decode_layers_batch_argmax")
        return out_tok

    def embed(self, tokens: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """out [B, d] float32 = bf16 embedding rows of tokens [B] (int32, CUDA),
        as embed_lookup (decode_kernel.c:1597-1600)."""
        if tokens.dtype != torch.int32 or not tokens.is_cuda or not tokens.is_contiguous():
            raise ValueError("tokens must be a contiguous int32 CUDA tensor")
        B = tokens.numel()
        if out is None:
            out = torch.empty((B, self.shape.d), dtype=torch.float32, device=tokens.device)
        _lib.check(_lib.lib().jm_embed_lookup(ctypes.byref(self._w), ctypes.byref(self._cfg), _lib.ptr(tokens), B,
                                              _lib.ptr(out), _lib.stream_handle(stream)), "jm_embed_lookup")
        return out

    def decode_batch_argmax(self, tokens, positions, kv: KVCacheSet) -> list[int]:
        """NativeDecoder.decode_batch_argmax (decoder3.py:607-629): embed the
        tokens, run every layer, return the argmax next token per sequence."""
        dev = self.store.blob.device
        tok = torch.as_tensor(np.asarray(tokens, dtype=np.int32), device=dev)
        x = self.embed(tok)
        out = self.decode_layers_batch_argmax(x, positions, kv)
        return [int(v) for v in out.cpu().tolist()]

    def set_max_layers(self, n: int) -> None:
        """Run only layers 0 .. n-1 in later calls (n < 0: all), as the
        reference's set_max_layers (decode_kernel.c:1617)."""
        _lib.check(_lib.lib().jm_store_set_max_layers(self.store._h, int(n)), "jm_store_set_max_layers")

    def trace_topk(self, buf: torch.Tensor | None) -> None:
        """Copy each layer's selected experts into buf [L, B, topk] (int32,
        CUDA) during later calls; None stops it."""
        if buf is not None and (buf.dtype != torch.int32 or not buf.is_cuda or not buf.is_contiguous()):
            raise ValueError("trace buffer must be a contiguous int32 CUDA tensor")
        _lib.check(_lib.lib().jm_store_trace_topk(self.store._h, _lib.ptr(buf),
                                                  0 if buf is None else buf.numel() * 4),
                   "jm_store_trace_topk")

    def split_ms(self) -> dict:
        """Attention / MoE / total milliseconds of the last call made with
        profiling on (store.profile(True)); waits for it."""
        a, m, t = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        _lib.check(_lib.lib().jm_store_decode_ms(self.store._h, ctypes.byref(a), ctypes.byref(m),
                                                 ctypes.byref(t)), "jm_store_decode_ms")
        return {"attention": a.value, "moe": m.value, "total": t.value}
