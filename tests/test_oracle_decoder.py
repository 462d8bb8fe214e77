"""Pins of the decoder restatement (oracle/decoder.py), CPU only.

Each function is checked against what the mathematics fixes, independently
of its own formula: exact cases of the reference's square root and its error
bound, torch's bfloat16 rounding, a float64 RMSNorm, RoPE as a complex
rotation with the RoPE frequencies theta^(-2i/hd), softmax attention with
the true exponential, the GQA head mapping by construction, and the whole
decode step against a float64 textbook decoder.
"""

import math

import numpy as np
import pytest
import torch

from joule_amd.decoder import rope_tables
from joule_amd.moe import MoEShape
from joule_amd.synth import numpy_store, router_weights
from oracle import decoder as D
from oracle import oracle as O
from oracle import textbook as TB


def test_sqrtf_fast_exact_cases_and_bound():
    # powers of 4: the bit-level guess is exact and the Newton step keeps it
    for x in (0.25, 1.0, 4.0, 16.0, 1024.0, 4.0 ** -6):
        assert D.sqrtf_fast(np.float32(x)) == np.float32(math.sqrt(x))
    # 128: guess 12 (exponent halved), then 0.5 * (12 + 128 / 12)
    assert D.sqrtf_fast(np.float32(128.0)) == np.float32(0.5) * (np.float32(12.0) + np.float32(128.0) / np.float32(12.0))
    x = np.logspace(-6, 6, 20001).astype(np.float32)
    rel = np.abs(D.sqrtf_fast(x).astype(np.float64) / np.sqrt(x.astype(np.float64)) - 1.0)
    assert rel.max() < 2e-3
    assert rel.max() > 1e-3          # it is the approximation, not a true sqrt


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0,
                        # exact halfway cases between two bf16 values
                        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(D.bf16_round(x), ref)


def test_rms_norm_against_float64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 2048)).astype(np.float32) * 3.0
    w = (1.0 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    eps = 1e-6
    got = D.rms_norm(x, w, eps).astype(np.float64)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps) * w
    rel = np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)
    assert rel.max() < 2e-3          # the sqrtf_fast bound
    # mean square exactly 4 (a power of 4): the scale is exactly 1/2
    y = D.rms_norm(np.full((1, 8), 2.0, np.float32), np.ones(8, np.float32), 0.0)
    assert np.array_equal(y, np.ones((1, 8), np.float32))


def test_rope_tables_frequencies():
    hd, theta = 128, 1e6
    cos, sin = rope_tables(64, hd, theta)
    # duplicated halves, unit circle, identity at position 0
    assert np.array_equal(cos[:, :64], cos[:, 64:]) and np.array_equal(sin[:, :64], sin[:, 64:])
    assert np.allclose(cos ** 2 + sin ** 2, 1.0, atol=1e-6)
    assert np.array_equal(cos[0], np.ones(hd, np.float32)) and np.array_equal(sin[0], np.zeros(hd, np.float32))
    # pair i turns by theta^(-2i/hd) = 10^(-6 * 2i / 128) per position
    for i in (0, 1, 17, 63):
        f = 10.0 ** (-6.0 * 2 * i / 128)
        for p in (1, 5, 63):
            assert abs(cos[p, i] - math.cos(p * f)) < 1e-6 and abs(sin[p, i] - math.sin(p * f)) < 1e-6


def test_rope_is_a_complex_rotation():
    rng = np.random.default_rng(3)
    cos, sin = rope_tables(300, 128, 1e6)
    v = rng.standard_normal((4, 128)).astype(np.float32)
    for p in (0, 1, 77, 299):
        got = D.rope(v, cos[p], sin[p]).astype(np.float64)
        z = (v[:, :64] + 1j * v[:, 64:]).astype(np.complex128) * (cos[p, :64] + 1j * sin[p, :64])
        assert np.abs(got[:, :64] - z.real).max() < 1e-5
        assert np.abs(got[:, 64:] - z.imag).max() < 1e-5
    # rotations compose: p1 then p2 equals p1 + p2 (angles linear in position)
    a = D.rope(D.rope(v, cos[100], sin[100]), cos[150], sin[150])
    b = D.rope(v, cos[250], sin[250])
    assert np.abs(a - b).max() < 1e-4


def test_attention_against_softmax():
    rng = np.random.default_rng(4)
    T, hd = 300, 128
    q = rng.standard_normal(hd).astype(np.float32)
    K = D.bf16_round(rng.standard_normal((T, hd)).astype(np.float32))
    V = D.bf16_round(rng.standard_normal((T, hd)).astype(np.float32))
    sdiv = float(D.sqrtf_fast(np.float32(hd)))
    got = D.attention(q, K, V, sdiv).astype(np.float64)
    s = K.astype(np.float64) @ q.astype(np.float64) / sdiv
    p = np.exp(s - s.max())
    want = (p / p.sum()) @ V.astype(np.float64)
    assert np.abs(got - want).max() / np.abs(want).max() < 2e-5


def _tiny_model(L=2, B=3, bias=False, qk=1, seed=7, dense=False):
    """A small decoder: d 512, 4 query heads over 2 KV heads of 128, MoE with
    8 experts of 128, top-2 renormalised; weights as float32 numpy."""
    shape = MoEShape(d=512, m=128, E=8, topk=2, renorm=True, name="tiny")
    H, KH, hd, T = 4, 2, 128, 64
    rng = np.random.default_rng(seed)
    r = lambda *s: D.bf16_round((rng.standard_normal(s) * 0.02).astype(np.float32))
    nw = lambda *s: D.bf16_round((1.0 + 0.1 * rng.standard_normal(s)).astype(np.float32))
    w = {"wq": r(L, H * hd, 512), "wk": r(L, KH * hd, 512), "wv": r(L, KH * hd, 512),
         "wo": r(L, 512, H * hd), "norm1": nw(L, 512), "norm2": nw(L, 512), "final_norm": nw(512),
         "qn": nw(L, hd) if qk != 2 else nw(L, H * hd), "kn": nw(L, hd) if qk != 2 else nw(L, KH * hd)}
    if bias:
        w.update(bq=r(L, H * hd), bk=r(L, KH * hd), bv=r(L, KH * hd))
    cos, sin = rope_tables(T, hd, 1e6)
    w["cos"], w["sin"] = cos, sin
    blob, offsets = numpy_store(shape, L, 32)
    moe = [O.OracleMoE(shape.d, shape.m, shape.E, shape.topk, shape.renorm, 32, router_weights(shape, l),
                       blob, offsets[:, l * shape.E:(l + 1) * shape.E]) for l in range(L)]
    if dense:                                   # a dense FFN of 1024 instead of the MoE block
        w.update(w1=r(L, 1024, 512), w2=r(L, 1024, 512), w3=r(L, 512, 1024))
        moe = None
    kv = [[(D.bf16_round(rng.standard_normal((T, KH, hd)).astype(np.float32)),
            D.bf16_round(rng.standard_normal((T, KH, hd)).astype(np.float32))) for _ in range(L)]
          for _ in range(B)]
    dec = D.OracleDecoder(L, 512, H, KH, hd, 1e-6, qk, bias, w, moe)
    return dec, shape, blob, offsets, kv


def _textbook_decode(dec, shape, blob, offsets, kv, x, positions):
    """float64 decode: true exp, float64 sums, the textbook MoE; the
    reference's sqrtf_fast kept (its error is pinned above)."""
    w, L, H, KH, hd = dec.w, dec.L, dec.H, dec.KH, dec.hd
    sq = lambda v: float(D.sqrtf_fast(np.float32(v)))

    def norm(v, wt):
        v = np.asarray(v, np.float64)
        ss = (v ** 2).sum(axis=-1, keepdims=True) / v.shape[-1] + dec.eps
        return v * (1.0 / np.vectorize(sq)(ss)) * wt

    def rot(v, c, s):
        a, b = v[..., :hd // 2], v[..., hd // 2:]
        c, s = c[:hd // 2].astype(np.float64), s[:hd // 2].astype(np.float64)
        return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)

    h = np.asarray(x, np.float64)
    g = H // KH
    for l in range(L):
        t = norm(h, w["norm1"][l])
        q, k, v = t @ w["wq"][l].T, t @ w["wk"][l].T, t @ w["wv"][l].T
        if dec.bias:
            q, k, v = q + w["bq"][l], k + w["bk"][l], v + w["bv"][l]
        att = np.zeros((h.shape[0], H * hd))
        for b in range(h.shape[0]):
            p = positions[b]
            if dec.qk == 2:                       # over the whole vector, then the heads
                qb = norm(q[b], w["qn"][l]).reshape(H, hd)
                kb = norm(k[b], w["kn"][l]).reshape(KH, hd)
            elif dec.qk == 1:
                qb = norm(q[b].reshape(H, hd), w["qn"][l])
                kb = norm(k[b].reshape(KH, hd), w["kn"][l])
            else:
                qb, kb = q[b].reshape(H, hd), k[b].reshape(KH, hd)
            qb = rot(qb, w["cos"][p], w["sin"][p])
            kb = rot(kb, w["cos"][p], w["sin"][p])
            Kc = kv[b][l][0].astype(np.float64).copy()
            Vc = kv[b][l][1].astype(np.float64).copy()
            Kc[p], Vc[p] = D.bf16_round(kb.astype(np.float32)), D.bf16_round(v[b].reshape(KH, hd).astype(np.float32))
            for hh in range(H):
                s = Kc[:p + 1, hh // g] @ qb[hh] / sq(hd)
                e = np.exp(s - s.max())
                att[b, hh * hd:(hh + 1) * hd] = (e / e.sum()) @ Vc[:p + 1, hh // g]
        h = h + att @ w["wo"][l].T
        t = norm(h, w["norm2"][l])
        if dec.moe is None:                          # dense FFN: silu with the true exponential
            g_, u_ = t @ w["w1"][l].T, t @ w["w2"][l].T
            h = h + (g_ / (1.0 + np.exp(-g_)) * u_) @ w["w3"][l].T
            continue
        gate_w = router_weights(shape, l)

        def experts(e, l=l):
            mats = []
            for p_, (rows, cols) in enumerate(((shape.m, shape.d), (shape.m, shape.d), (shape.d, shape.m))):
                so, po = (int(vv) for vv in offsets[p_, l * shape.E + e])
                sb = rows * cols // 32 * 2
                mats.append(TB.dequant_matrix(blob[so:so + sb].view(np.uint16), blob[po:po + rows * cols // 2],
                                              rows, cols, 32))
            return tuple(mats)
        h = h + TB.moe_block(t, gate_w, experts, shape.topk, shape.renorm)
    return norm(h, w["final_norm"])


@pytest.mark.parametrize("qk,bias,dense", [(1, False, False), (2, True, False), (0, True, False), (1, False, True)])
def test_decoder_against_textbook(qk, bias, dense):
    dec, shape, blob, offsets, kv = _tiny_model(qk=qk, bias=bias, dense=dense)
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    positions = [0, 17, 63]
    want = _textbook_decode(dec, shape, blob, offsets, kv, x, positions)
    got = dec.decode_layers_batch(x, positions, kv)
    rel = np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)
    assert rel.max() < 1e-4, rel
    # the cache rows at the positions were written (bf16 values)
    for b, p in enumerate(positions):
        for l in range(dec.L):
            assert np.array_equal(kv[b][l][0][p], D.bf16_round(kv[b][l][0][p]))


def test_gqa_head_mapping():
    # KV head kh holds V = kh + 1 everywhere: query head h must read KV head
    # h // (H / KH), so its output is exactly h // g + 1
    dec, shape, blob, offsets, kv = _tiny_model(L=1, B=1)
    H, KH, hd = dec.H, dec.KH, dec.hd
    Vc = kv[0][0][1]
    for kh in range(KH):
        Vc[:, kh, :] = kh + 1.0
    dec.w["wv"][0][:] = 0.0                       # the appended v is 0 ...
    x = np.random.default_rng(9).standard_normal((1, 512)).astype(np.float32)
    t = D.rms_norm(x, dec.w["norm1"][0], dec.eps)
    dec.w["wo"][0][:] = 0.0
    for i in range(H * hd):                       # o_proj as identity on the first 512 dims
        if i < 512:
            dec.w["wo"][0][i, i] = 1.0
    out = dec.layer_attn(0, t, [0], kv)           # position 0: only the appended row
    assert np.array_equal(out, np.zeros_like(out))
    for kh in range(KH):
        Vc[:, kh, :] = kh + 1.0
    out = dec.layer_attn(0, t, [40], kv)          # rows 0..39 hold kh+1, row 40 holds 0
    o = out[0]
    for h in range(4):
        seg = o[h * hd:(h + 1) * hd]
        kh = h // (H // KH)
        assert np.all(seg > 0) and np.all(seg < kh + 1.0 + 1e-6)
        assert np.all(np.abs(seg - seg[0]) < 1e-6)
    assert o[:hd].max() < o[2 * hd:3 * hd].min()  # heads 0-1 read KV head 0, heads 2-3 KV head 1


def test_dense_ffn_against_float64():
    """layer_ffn_batch's E == 0 branch (decode_kernel.c:1393-1422) against
    silu(g) * u with the true exponential in float64 (the reference's
    expf_fast is within 1e-5 of it); zero up rows or zero gate rows give
    exactly zero (silu(0) = 0)."""
    rng = np.random.default_rng(14)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    w1, w2 = (D.bf16_round((rng.standard_normal((1536, 512)) * 0.05).astype(np.float32)) for _ in range(2))
    w3 = D.bf16_round((rng.standard_normal((512, 1536)) * 0.05).astype(np.float32))
    got = D.dense_ffn(x, w1, w2, w3).astype(np.float64)
    x64 = x.astype(np.float64)
    g, u = x64 @ w1.T.astype(np.float64), x64 @ w2.T.astype(np.float64)
    want = (g / (1.0 + np.exp(-g)) * u) @ w3.T.astype(np.float64)
    rel = np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)
    assert rel.max() < 1e-4, rel
    assert not np.any(D.dense_ffn(x, w1, np.zeros_like(w2), w3))
    assert not np.any(D.dense_ffn(x, np.zeros_like(w1), w2, w3))


def _appended_k(dec, kv, x, pos):
    """The k row layer 0 appends at pos for token x (float32 copy)."""
    t = D.rms_norm(x, dec.w["norm1"][0], dec.eps)
    dec.layer_attn(0, t, [pos], kv)
    return kv[0][0][0][pos].copy()


def test_whole_vector_qk_norm_invariants():
    """qk_norm_type 2 (decode_kernel.c:1155-1167) pinned by what it must do,
    observed through the appended k row and the attention output:
    * k over all KH * hd values has mean square 1 (unit weight, eps 0,
      position 0 where RoPE is the identity) while its heads keep their
      relative scale (a per-head norm would make each head's mean square 1);
    * the weight multiplies elementwise after the scaling;
    * the norm comes before RoPE: a weight that zeroes dimensions 64..127 of
      every head leaves a sin-rotated copy of dimensions 0..63 there;
    * q: scaling all of wq leaves the output unchanged, scaling one head's
      rows changes it (with a per-head norm it would not)."""
    dec, shape, blob, offsets, kv = _tiny_model(L=1, B=1, qk=2)
    H, KH, hd = dec.H, dec.KH, dec.hd
    dec.eps = 0.0
    x = np.random.default_rng(11).standard_normal((1, 512)).astype(np.float32)
    dec.w["kn"][0][:] = 1.0
    dec.w["wk"][0][hd:] *= 4.0                       # KV head 1 four times larger
    k0 = _appended_k(dec, kv, x, 0).astype(np.float64)
    assert abs((k0 ** 2).mean() - 1.0) < 4e-3        # sqrtf_fast and bf16 rounding
    ratio = (k0[1] ** 2).mean() / (k0[0] ** 2).mean()
    assert 8.0 < ratio < 32.0                        # not equalised per head
    wt = D.bf16_round((1.0 + 0.5 * np.random.default_rng(12).standard_normal(KH * hd)).astype(np.float32))
    dec.w["kn"][0][:] = wt
    kw = _appended_k(dec, kv, x, 0).astype(np.float64)
    rel = np.abs(kw.reshape(-1) - k0.reshape(-1) * wt) / (np.abs(k0.reshape(-1) * wt) + 1e-3)
    assert rel.max() < 2 ** -7
    half = np.tile(np.r_[np.ones(hd // 2), np.zeros(hd // 2)], KH).astype(np.float32)
    dec.w["kn"][0][:] = half
    p = 37
    kr = _appended_k(dec, kv, x, p)
    k_half = _appended_k(dec, kv, x, 0)              # position 0: the normed, weighted values
    s_ = dec.w["sin"][p][:hd // 2]
    for kh in range(KH):
        second = kr[kh, hd // 2:]
        assert np.abs(second).max() > 0.1
        want = D.bf16_round((k_half[kh, :hd // 2] * s_).astype(np.float32))
        assert np.allclose(second, want, rtol=2 ** -6, atol=1e-3)
    # q through the attention output (two positions so the scores matter)
    dec.w["kn"][0][:] = 1.0
    t = D.rms_norm(x, dec.w["norm1"][0], dec.eps)
    base = dec.layer_attn(0, t, [40], kv)
    dec.w["wq"][0] *= 3.0
    same = dec.layer_attn(0, t, [40], kv)
    # unchanged up to sqrtf_fast, whose relative error (< 2e-3) differs between ss and 9 ss
    assert np.abs(same - base).max() <= 5e-3 * np.abs(base).max()
    dec.w["wq"][0][:hd] *= 3.0                       # query head 0 only
    diff = dec.layer_attn(0, t, [40], kv)
    assert np.abs(diff - base).max() > 5e-2 * np.abs(base).max()
    dec.qk = 1                                       # per head: the same change is invisible
    dec.w["qn"], dec.w["kn"] = np.ones((1, hd), np.float32), np.ones((1, hd), np.float32)
    dec.w["wq"][0][:hd] /= 3.0
    b1 = dec.layer_attn(0, t, [40], kv)
    dec.w["wq"][0][:hd] *= 3.0
    d1 = dec.layer_attn(0, t, [40], kv)
    assert np.abs(d1 - b1).max() <= 5e-3 * np.abs(b1).max()


def _lm_head_A_scan(logits, n_workers):
    """The reference's argmax (decode_kernel.c:1008-1062) step by step:
    participants take contiguous row ranges span*id/np, each keeps its best
    from (-1e30, 0) with strict >, and the merge walks them in order with
    strict >."""
    V = len(logits)
    bv, bi = np.float32(-1e30), 0
    for w in range(n_workers):
        lo, hi = V * w // n_workers, V * (w + 1) // n_workers
        ov, oi = np.float32(-1e30), 0
        for i in range(lo, hi):
            if logits[i] > ov:
                ov, oi = logits[i], i
        if ov > bv:
            bv, bi = ov, oi
    return bi


def test_argmax_strict_matches_the_reference_scan():
    rng = np.random.default_rng(11)
    cases = []
    for _ in range(20):
        v = rng.standard_normal(997).astype(np.float32)
        top = v.max()
        for j in rng.choice(997, size=3, replace=False):   # planted ties at the max
            v[j] = top
        cases.append(v)
    v = rng.standard_normal(500).astype(np.float32)
    v[[3, 400]] = np.nan
    v[250] = 9.0
    v[499] = 9.0
    cases.append(v)                                          # NaN never wins, the lower 9.0 does
    cases.append(np.full(64, -1e30, np.float32))             # nothing beats -1e30: row 0
    cases.append(np.concatenate([np.full(10, np.nan, np.float32), np.full(5, -2e30, np.float32)]))
    cases.append(np.array([-1e30, -1e30, -0.5, -0.5], np.float32))
    for v in cases:
        want = [_lm_head_A_scan(v, n) for n in (1, 3, 9, 17)]
        assert len(set(want)) == 1                               # the worker split does not matter
        assert D.argmax_strict(v[None])[0] == want[0]
