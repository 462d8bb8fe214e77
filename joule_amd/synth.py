"""Seeded synthetic MoE workloads (no checkpoints are available offline).

* Expert weights: N(0, 0.02) float32, quantised to the Q4 store format.
* Router weights: N(0, 0.02) rounded to bf16 and widened back to float32,
  so the fp32 router sees exactly the values the reference's bf16 table
  (decode_kernel.c:303) would hold.
* Activations: x ~ N(0, 1) float32.
* Zipf routing (prefill-style workload): a bias beta_e = alpha * ln(z_pi(e))
  with z Zipf(1.1) over the experts is carried by a constant input feature
  x[:, 0] = c and router column w[:, 0] = beta / c, so the router stays the
  reference's plain GEMV.

Two generators produce a store: ``numpy_store`` (host, small shapes, used by
CPU tests) and ``torch_store`` (on the GPU, for full-size layers; its
quantiser follows the same arithmetic as ``q4_store.quantize`` and is checked
against it byte for byte in the GPU tests).
"""

from __future__ import annotations

import numpy as np
import torch

from .moe import MoEShape, offsets_for_layout
from .q4_store import quantize, record_sizes


def bf16_round(a: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even) -> float32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    nan = np.isnan(a)
    out = r.astype(np.uint32).view(np.float32)
    out = np.where(nan, np.float32(np.nan), out)
    return out.astype(np.float32)


def router_weights(shape: MoEShape, layer: int, seed: int = 2000, bf16: bool = True) -> np.ndarray:
    """N(0, 0.02) router table [E, d] of one layer, rounded to bf16 values
    (a bf16 checkpoint's gate) or, with bf16=False, left float32."""
    rng = np.random.default_rng(seed + layer)
    w = rng.normal(0.0, 0.02, (shape.E, shape.d)).astype(np.float32)
    return bf16_round(w) if bf16 else w


def activations(B: int, d: int, seed: int = 3000) -> np.ndarray:
    return np.random.default_rng(seed + B).standard_normal((B, d)).astype(np.float32)


def zipf_bias(E: int, s: float = 1.1, alpha: float = 1.0, seed: int = 4000) -> np.ndarray:
    r = np.arange(1, E + 1, dtype=np.float64)
    z = r ** (-s)
    z /= z.sum()
    perm = np.random.default_rng(seed).permutation(E)
    return (alpha * np.log(z[perm])).astype(np.float32)


def apply_logit_bias(gate_w: np.ndarray, x: np.ndarray, bias: np.ndarray, c: float = 4.0):
    """Return (gate_w', x') with gate_w' . x' = gate_w[:,1:] . x[:,1:] + bias
    exactly up to rounding of bias / c (column 0 carries the bias)."""
    g = gate_w.copy()
    xx = x.copy()
    g[:, 0] = bf16_round((bias / np.float32(c)).astype(np.float32))
    xx[:, 0] = np.float32(c)
    return g, xx


def expert_matrices(shape: MoEShape, layer: int, seed: int = 1000, experts=None):
    """float32 (gate, up, down) per expert from default_rng(seed + layer),
    drawn in (expert, part) order."""
    rng = np.random.default_rng(seed + layer)
    out = {}
    for e in range(shape.E):
        mats = []
        for rows, cols in ((shape.m, shape.d), (shape.m, shape.d), (shape.d, shape.m)):
            mats.append(rng.normal(0.0, 0.02, (rows, cols)).astype(np.float32))
        if experts is None or e in experts:
            out[e] = tuple(mats)
    return out


def numpy_store(shape: MoEShape, n_layers: int, group: int = 64, seed: int = 1000):
    """(blob uint8, offsets [3, L*E, 2]) built on the host with q4_store.quantize."""
    offsets, total = offsets_for_layout(shape, n_layers, group)
    blob = np.zeros(total, np.uint8)
    for l in range(n_layers):
        mats = expert_matrices(shape, l, seed)
        for e in range(shape.E):
            for p in range(3):
                sb, pb = quantize(mats[e][p], group)
                so, po = (int(v) for v in offsets[p, l * shape.E + e])
                blob[so:so + len(sb)] = np.frombuffer(sb, np.uint8)
                blob[po:po + len(pb)] = np.frombuffer(pb, np.uint8)
    return blob, offsets


# ------------------------------------------------------------------ GPU


def quantize_torch(w: torch.Tensor, group: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """Q4-quantise a float32 tensor on its device (numel % group == 0).

    Same arithmetic as q4_store.quantize: float32 absmax floored at 1e-12,
    /7 in float32, rounded to float16, float32 division, round half to even,
    clip to [-8, 7], +8, two nibbles per byte with the even element low.
    Returns (scales as int16 bits, packed uint8)."""
    flat = w.reshape(-1, group).float()
    absmax = flat.abs().amax(dim=1).clamp_min(1e-12)
    scales = (absmax / 7.0).to(torch.float16)
    q = torch.round(flat / scales.float().unsqueeze(1)).clamp_(-8, 7)
    q = torch.nan_to_num(q, nan=0.0).to(torch.int16) + 8
    q = q.to(torch.uint8).reshape(-1)
    packed = (q[0::2] & 0x0F) | (q[1::2] << 4)
    return scales.view(torch.int16), packed


def torch_store(shape: MoEShape, n_layers: int, group: int = 64, seed: int = 1000,
                device: str | torch.device = "cuda", progress=None):
    """(blob uint8 CUDA tensor, offsets) for n_layers full layers, generated
    and quantised on the GPU (seed + layer per layer)."""
    offsets, total = offsets_for_layout(shape, n_layers, group)
    blob = torch.empty(total, dtype=torch.uint8, device=device)
    dims = ((shape.m, shape.d), (shape.m, shape.d), (shape.d, shape.m))
    per_expert = int(offsets[0, 1, 0] - offsets[0, 0, 0]) if shape.E * n_layers > 1 else total
    for l in range(n_layers):
        gen = torch.Generator(device=device)
        gen.manual_seed(seed + l)
        layer = blob[l * shape.E * per_expert:(l + 1) * shape.E * per_expert].view(shape.E, per_expert)
        col = 0
        for rows, cols in dims:
            w = torch.randn((shape.E, rows * cols), generator=gen, device=device, dtype=torch.float32)
            w.mul_(0.02)
            sc, pk = quantize_torch(w, group)
            sb, pb = record_sizes(rows, cols, group)
            layer[:, col:col + sb].copy_(sc.view(torch.uint8).view(shape.E, sb))
            layer[:, col + sb:col + sb + pb].copy_(pk.view(shape.E, pb))
            col += sb + pb
            del w, sc, pk
        if progress:
            progress(l)
    return blob, offsets


# ------------------------------------------------------------ decoder


def decoder_weights(shape, seed: int = 6000, device: str | torch.device = "cuda",
                    norm_jitter: float = 0.0) -> dict:
    """Dense weights of a decoder (joule_amd.decoder.DecoderShape) as bf16
    tensors on ``device``: projections N(0, 0.02); RMSNorm / QK-norm weights
    1.0, or 1 + N(0, norm_jitter) when norm_jitter > 0 (tests use it so
    that a weight applied to the wrong element shows); float32 biases
    N(0, 0.02) when the shape has bias_qkv; a dense model's FFN weights
    w1/w2/w3 N(0, 0.02).  One torch generator seeded with ``seed`` draws
    them in a fixed order."""
    L, d, H, KH, hd = shape.n_layers, shape.d, shape.n_heads, shape.n_kv, shape.hd
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def normal(*shp, std=0.02):
        return (torch.randn(shp, generator=gen, device=device, dtype=torch.float32) * std)

    def norm_w(*shp):
        w = torch.ones(shp, device=device, dtype=torch.float32)
        if norm_jitter > 0:
            w += normal(*shp, std=norm_jitter)
        return w.to(torch.bfloat16)

    t = {
        "wq": normal(L, H * hd, d).to(torch.bfloat16),
        "wk": normal(L, KH * hd, d).to(torch.bfloat16),
        "wv": normal(L, KH * hd, d).to(torch.bfloat16),
        "wo": normal(L, d, H * hd).to(torch.bfloat16),
        "norm1": norm_w(L, d),
        "norm2": norm_w(L, d),
        "final_norm": norm_w(d),
    }
    if shape.qk_norm_type == 1:
        t["qn"] = norm_w(L, hd)
        t["kn"] = norm_w(L, hd)
    elif shape.qk_norm_type == 2:
        t["qn"] = norm_w(L, H * hd)
        t["kn"] = norm_w(L, KH * hd)
    if shape.moe.E == 0:
        m = shape.moe.m
        t["w1"] = normal(L, m, d).to(torch.bfloat16)
        t["w2"] = normal(L, m, d).to(torch.bfloat16)
        t["w3"] = normal(L, d, m).to(torch.bfloat16)
    if shape.bias_qkv:
        t["bq"] = normal(L, H * hd)
        t["bk"] = normal(L, KH * hd)
        t["bv"] = normal(L, KH * hd)
    return t


def fill_kv(data: torch.Tensor, seed: int = 5000) -> torch.Tensor:
    """Fill a cache tensor [B, L, 2, T, KH, hd] (bf16 or float32) with
    N(0, 1): one generator per layer, seeded seed + layer, drawing
    [B, 2, T, KH, hd]."""
    B, L = data.shape[0], data.shape[1]
    for l in range(L):
        gen = torch.Generator(device=data.device)
        gen.manual_seed(seed + l)
        data[:, l].copy_(torch.randn(data[:, l].shape, generator=gen, device=data.device,
                                     dtype=torch.float32).to(data.dtype))
    return data
