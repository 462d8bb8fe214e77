"""Float64 textbook MoE block (numpy), independent of the C restatement.

TEST INFRASTRUCTURE ONLY (see oracle/oracle.py).

It computes the mathematical function the reference implements
(src/jouleai/native/decode_kernel.c:1387-1508) without its rounding
choices: exact dequantised weights (q4_store.py:58-67) widened to float64,
the true exponential, a stable top-k with the lowest index winning ties,
SwiGLU and the weighted sum.  Agreement with it bounds the restatement's and
the GPU path's accumulated rounding from an independent direction.
"""

from __future__ import annotations

import numpy as np


def dequant_matrix(scales_u16: np.ndarray, packed_u8: np.ndarray, rows: int, cols: int,
                   group: int) -> np.ndarray:
    raw = np.asarray(packed_u8, np.uint8).ravel()
    q = np.empty(raw.size * 2, np.float64)
    q[0::2] = (raw & 0x0F).astype(np.float64) - 8.0
    q[1::2] = (raw >> 4).astype(np.float64) - 8.0
    s = np.asarray(scales_u16).view(np.float16).astype(np.float64)
    return (q.reshape(-1, group) * s[:, None]).reshape(rows, cols)


def topk_lowest_index(p: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest values; equal values ordered by index."""
    order = np.lexsort((np.arange(p.size), -p))
    return order[:k]


def route(gate_w: np.ndarray, x: np.ndarray, k: int, renorm: bool):
    """float64 logits -> softmax -> top-k (+ renormalisation)."""
    logits = np.asarray(x, np.float64) @ np.asarray(gate_w, np.float64).T
    z = logits - logits.max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    top = np.stack([topk_lowest_index(p[b], k) for b in range(p.shape[0])])
    w = np.take_along_axis(p, top, axis=1)
    if renorm:
        w = w / w.sum(axis=1, keepdims=True)
    return logits, p, top, w


def silu(v: np.ndarray) -> np.ndarray:
    return v / (1.0 + np.exp(-v))


def moe_block(x: np.ndarray, gate_w: np.ndarray, experts, k: int, renorm: bool,
              top: np.ndarray | None = None, w: np.ndarray | None = None):
    """out[B, d] in float64.

    ``experts(e)`` returns float64 (gate [m,d], up [m,d], down [d,m]).
    ``top``/``w`` override the routing (e.g. to reuse the bit-exact router
    result of the restatement when only the expert arithmetic is compared).
    """
    x64 = np.asarray(x, np.float64)
    if top is None or w is None:
        _, _, top, w = route(gate_w, x, k, renorm)
    B, d = x64.shape
    out = np.zeros((B, d), np.float64)
    cache = {}
    for b in range(B):
        for i in range(k):
            e = int(top[b, i])
            if e < 0:
                continue
            if e not in cache:
                cache[e] = experts(e)
            g, u, dn = cache[e]
            act = silu(g @ x64[b]) * (u @ x64[b])
            out[b] += float(w[b, i]) * (dn @ act)
    return out
