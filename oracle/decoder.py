"""CPU restatement of the reference's batch decode around the MoE block.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's checks, as the
checker.  The product path (joule_amd) never imports it.

Follows src/jouleai/native/decode_kernel.c:

  sqrtf_fast            :88-93    bit-level guess + one Newton step
  rms_norm              :224-230  x * (1 / sqrtf_fast(sum x^2 / d + eps)) * w
  matvec_f32            :234-256  out = W . x (here: float64 dot, rounded to float32)
  rope_apply            :259-266  rotate-half with the cos/sin tables
  layer_attn_batch      :1120-1234  QKV (+ bias), whole-vector QK-norm
                          (qk_norm_type 2, :1155-1167) or per-head QK-norm
                          (qk_norm_type 1, :1169-1189), RoPE at positions[b], KV append,
                          SDPA with scores / sqrtf_fast(hd) and expf_fast
                          weights normalised before P.V, o_proj
  decode_layers_batch   :1518-1556  norm1 -> attention -> residual -> norm2
                          -> MoE (OracleMoE, the C restatement of
                          layer_ffn_batch) -> residual; final norm
  dense_ffn             :1393-1422  layer_ffn_batch's E == 0 branch (dense
                          models): silu(x w1^T) * (x w2^T), then w3
  lm_head_B             :964-1000  logits = lm_head . x (float64 dot, rounded)
  lm_head_A             :1008-1062  argmax: per-worker strict-> scans from
                          (-1e30, row 0) over contiguous row ranges, merged
                          in worker order with strict >
  embed_lookup          :1597-1600  bf16 embedding row

Two deliberate differences from the reference, both matching the GPU path:
by default the KV cache holds bfloat16 values (the reference's is float32,
decode_kernel.c:328-331): the appended k and v are rounded to bf16 before
attention reads them (kv_bf16=False keeps float32 rows, the reference's
cache); and dot products / sums of squares are accumulated in float64 and
rounded once, where the reference accumulates in float32 in its own lane
order (a difference at rounding level).
"""

from __future__ import annotations

import numpy as np

from . import oracle as O

F32 = np.float32


def sqrtf_fast(x) -> np.ndarray:
    """decode_kernel.c:88-93 on float32 values (array or scalar)."""
    x = np.asarray(x, F32)
    u = x.view(np.uint32).astype(np.uint64)
    v = (((u + 0x3F800000) & 0xFFFFFFFF) >> 1).astype(np.uint32).view(F32)
    return (F32(0.5) * (v + x / v)).astype(F32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), as float32."""
    u = np.asarray(x, F32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return (r & 0xFFFFFFFF).astype(np.uint32).view(F32)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Rows of x [.., n] normalised as decode_kernel.c:224-230; w float32
    holding the bf16 weight values."""
    x = np.asarray(x, F32)
    n = x.shape[-1]
    ss = (x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True).astype(F32)
    inv = (F32(1.0) / sqrtf_fast(ss / F32(n) + F32(eps))).astype(F32)
    return ((x * inv).astype(F32) * np.asarray(w, F32)).astype(F32)


def matvec(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Rows x [B, k] times W [m, k]^T -> [B, m] float32."""
    return (np.asarray(x, np.float64) @ np.asarray(W, np.float64).T).astype(F32)


def rope(v: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE (decode_kernel.c:259-266) of heads v [.., hd] with the
    position's table rows cos/sin [hd]."""
    v = np.asarray(v, F32)
    h = v.shape[-1] // 2
    a, b = v[..., :h], v[..., h:]
    c, s = cos[:h], sin[:h]
    out = np.empty_like(v)
    out[..., :h] = (a * c).astype(F32) - (b * s).astype(F32)
    out[..., h:] = (a * s).astype(F32) + (b * c).astype(F32)
    return out


def attention(q: np.ndarray, K: np.ndarray, V: np.ndarray, sdiv: float) -> np.ndarray:
    """One query head q [hd] over T positions K, V [T, hd]: the SDPA of
    decode_kernel.c:1205-1221."""
    s = (np.asarray(K, np.float64) @ np.asarray(q, np.float64)).astype(F32) / F32(sdiv)
    p = O.expf_fast_array((s - s.max()).astype(F32))
    tot = F32(p.astype(np.float64).sum())
    return ((p / tot).astype(np.float64) @ np.asarray(V, np.float64)).astype(F32)


class OracleDecoder:
    """decode_layers_batch restated for a small model.

    ``w`` holds float32 arrays of the bf16 weight values: norm1/norm2 [L, d],
    final_norm [d], wq [L, H*hd, d], wk/wv [L, KH*hd, d], wo [L, d, H*hd],
    qn/kn [L, hd] (qk_norm_type 1) or [L, H*hd] / [L, KH*hd] (qk_norm_type
    2), bq/bk/bv (bias_qkv), cos/sin [maxT, hd].
    ``moe[l]`` is an OracleMoE for layer l; with ``moe`` None the model is
    dense and ``w`` holds w1/w2 [L, m, d] and w3 [L, d, m].  The caches are float32 arrays
    [B][L] of (k, v) [maxT, KH, hd], holding bf16 values unless kv_bf16 is
    False; they are updated in place like the reference's.
    """

    def __init__(self, L, d, H, KH, hd, eps, qk_norm_type, bias_qkv, w: dict, moe, kv_bf16: bool = True):
        self.L, self.d, self.H, self.KH, self.hd = L, d, H, KH, hd
        self.kv_bf16 = bool(kv_bf16)
        self.eps, self.qk, self.bias = float(eps), int(qk_norm_type), bool(bias_qkv)
        self.w, self.moe = w, moe
        self.sdiv = sqrtf_fast(F32(hd))

    def layer_attn(self, l: int, x: np.ndarray, positions, kv) -> np.ndarray:
        w, H, KH, hd = self.w, self.H, self.KH, self.hd
        B = x.shape[0]
        q = matvec(w["wq"][l], x)
        k = matvec(w["wk"][l], x)
        v = matvec(w["wv"][l], x)
        if self.bias:
            q = (q + w["bq"][l]).astype(F32)
            k = (k + w["bk"][l]).astype(F32)
            v = (v + w["bv"][l]).astype(F32)
        if self.qk == 2:
            # the whole q and k vectors of each token, before the head view
            # (decode_kernel.c:1155-1167)
            q = rms_norm(q, w["qn"][l], self.eps)
            k = rms_norm(k, w["kn"][l], self.eps)
        att = np.zeros((B, H * hd), F32)
        g = H // KH
        for b in range(B):
            qb = q[b].reshape(H, hd)
            kb = k[b].reshape(KH, hd)
            vb = v[b].reshape(KH, hd)
            if self.qk == 1:
                qb = rms_norm(qb, w["qn"][l], self.eps)
                kb = rms_norm(kb, w["kn"][l], self.eps)
            pos = int(positions[b])
            c, s = w["cos"][pos], w["sin"][pos]
            qb = rope(qb, c, s)
            kb = rope(kb, c, s)
            kc, vc = kv[b][l]
            kc[pos] = bf16_round(kb) if self.kv_bf16 else kb
            vc[pos] = bf16_round(vb) if self.kv_bf16 else vb
            T = pos + 1
            for h in range(H):
                kh = h // g
                att[b, h * hd:(h + 1) * hd] = attention(qb[h], kc[:T, kh], vc[:T, kh], self.sdiv)
        return matvec(w["wo"][l], att)

    def decode_layers_batch(self, x: np.ndarray, positions, kv, trace: list | None = None,
                            n_threads: int = 1, progress=None) -> np.ndarray:
        """Final-normed hidden state [B, d] after all layers.  With `trace`
        (a list), each layer appends a dict: "moe_in" (the normed input of
        its MoE block), "top" (its selected experts) and "hidden" (the final
        norm of h after this layer: what the step returns when it stops
        there, set_max_layers, decode_kernel.c:1617)."""
        w = self.w
        h = np.array(x, F32, copy=True)
        for l in range(self.L):
            t = rms_norm(h, w["norm1"][l], self.eps)
            h = (h + self.layer_attn(l, t, positions, kv)).astype(F32)
            t = rms_norm(h, w["norm2"][l], self.eps)
            if self.moe is None:                  # a dense model (E == 0)
                out, top = dense_ffn(t, w["w1"][l], w["w2"][l], w["w3"][l]), None
            else:
                out, top, _ = self.moe[l].forward(t, n_threads=n_threads)
            h = (h + out).astype(F32)
            if trace is not None:
                trace.append({"moe_in": t, "top": top, "hidden": rms_norm(h, w["final_norm"], self.eps)})
            if progress:
                progress(l)
        return rms_norm(h, w["final_norm"], self.eps)


def dense_ffn(x: np.ndarray, w1: np.ndarray, w2: np.ndarray, w3: np.ndarray) -> np.ndarray:
    """layer_ffn_batch with E == 0 (decode_kernel.c:1393-1422) on rows x
    [B, d]: g = x . w1^T and u = x . w2^T (float32 holding bf16 values;
    float64 dots rounded once), act = (g / (1 + expf_fast(-g))) * u in
    float32 as the reference writes it, out = act . w3^T."""
    g = matvec(w1, x)
    u = matvec(w2, x)
    e = O.expf_fast_array(-g).reshape(g.shape).astype(F32)
    act = ((g / (F32(1.0) + e)).astype(F32) * u).astype(F32)
    return matvec(w3, act)


def lm_head(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """logits [B, V] of rows W [V, d] (float32 holding bf16 values)."""
    return matvec(W, x)


def argmax_strict(logits: np.ndarray) -> np.ndarray:
    """Per row of logits [B, V]: the row lm_head_A picks.  Its answer is the
    first index of the largest value above -1e30 (NaN excluded), or 0 when no
    value exceeds -1e30; the worker split of the scan does not change it
    (its merge is in worker order with strict >)."""
    lg = np.asarray(logits, np.float32)
    out = np.zeros(lg.shape[0], np.int64)
    for b in range(lg.shape[0]):
        v = lg[b]
        ok = (v > np.float32(-1e30)) & ~np.isnan(v)
        if ok.any():
            m = v[ok].max()
            out[b] = int(np.flatnonzero(ok & (v == m))[0])
    return out


def embed_lookup(E: np.ndarray, tokens) -> np.ndarray:
    """Rows of the embedding E [V, d] (float32 holding bf16 values)."""
    return np.asarray(E, np.float32)[np.asarray(tokens, np.int64)].copy()
