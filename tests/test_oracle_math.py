"""The oracle's router and MoE block against closed forms and float64.

Pins for what the compiled reference cannot reach (decode_kernel.c is not
buildable here):
* expf_fast: exact cases (clamps, v = 0) and the error bound its degree-5
  Taylor polynomial implies (|f ln2|^6 / 6! / 2^f <= 3.41e-6 relative for
  |f| <= 1/2) plus the float32 rounding of v*log2(e);
* router dot: exact integer inputs (any order must give the exact sum), a
  unit-vector KAT for indexing, and a case whose answer depends on the AVX2
  horizontal-sum tree ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7));
* softmax/top-k: hand-made ties (lowest index wins), renormalisation,
  NaN scores;
* the whole block against the float64 textbook (independent arithmetic),
  plus thread-count, cost-model and batch invariances.
"""

import math

import numpy as np
import pytest

from joule_amd import q4_store as Q
from joule_amd.moe import MoEShape, offsets_for_layout
from joule_amd.synth import numpy_store, router_weights, bf16_round
from oracle import textbook as T


def test_expf_fast_closed_forms(oracle_lib):
    f = oracle_lib.expf_fast_array
    assert f(np.array([0.0]))[0] == 1.0
    assert np.all(f(np.array([-17.0001, -20.0, -1e30, -np.inf], np.float32)) == 0.0)
    assert f(np.array([-17.0], np.float32))[0] > 0.0
    big = f(np.array([88.0, 89.0, 1e30, np.inf], np.float32))
    assert np.all(big == big[0]) and np.isfinite(big[0])
    assert f(np.array([np.nan], np.float32))[0] == 0.0
    v = np.linspace(-17, 88, 200001).astype(np.float32)
    got = f(v).astype(np.float64)
    rel = np.abs(got / np.exp(v.astype(np.float64)) - 1.0)
    # polynomial truncation (|f ln2|^6/6! = 2.41e-6 absolute at |f| = 1/2,
    # relative to 2^-1/2 = 0.707 -> 3.41e-6) + rounding of y = v*log2(e)
    # (0.5 ulp of |y|, times ln 2 in the result) + the final products
    y = np.abs(v.astype(np.float64) * 1.4426950408889634)
    bound = 3.45e-6 + np.log(2) * y * 2.0**-24 + 2.0**-22
    assert np.all(rel <= bound), float((rel / bound).max())


def test_router_dot_exact_and_tree(oracle_lib):
    rng = np.random.default_rng(0)
    w = rng.integers(-8, 8, 2048).astype(np.float32)
    x = rng.integers(-8, 8, 2048).astype(np.float32)
    assert oracle_lib.router_dot(w, x) == float(np.dot(w.astype(np.int64), x.astype(np.int64)))
    for j in (0, 5, 2047):
        e = np.zeros(2048, np.float32)
        e[j] = 1.0
        assert oracle_lib.router_dot(e, x) == x[j]
    # lane partials l = [2^24, 1, 1, 1, -2^24, 1, 1, 1]: the AVX2 tree gives
    # (2^24 - 2^24) + (1 + 1) + ((1 + 1) + (1 + 1)) = 6, a sequential sum 3
    w8 = np.array([2.0**24, 1, 1, 1, -(2.0**24), 1, 1, 1], np.float32)
    assert oracle_lib.router_dot(w8, np.ones(8, np.float32)) == 6.0
    # float inputs: within the fp32 accumulation bound of the exact dot
    w = rng.normal(0, 0.02, 2048).astype(np.float32)
    x = rng.standard_normal(2048).astype(np.float32)
    exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
    bound = 2048 * 2**-24 * float(np.abs(w.astype(np.float64) * x).sum())
    assert abs(oracle_lib.router_dot(w, x) - exact) <= bound


# A router row whose dot with x = ones depends on every part of the
# reference's order (decode_kernel.c:234-256): products 2^24 at j=0, 1 at
# j=8, 16 and 9, -2^24 at j=4, zeros elsewhere.  Lanes hold j = r (mod 8),
# each an FMA chain in increasing j: lane 0 = (2^24 + 1) + 1 = 2^24 (each
# 1 lost to ties-to-even), lane 1 = 1, lane 4 = -2^24; the tree
# ((l0 + l4) + (l2 + l6)) + ((l1 + l5) + (l3 + l7)) gives 0 + 1 = 1.
ROUTER_KAT = {0: 2.0**24, 8: 1.0, 16: 1.0, 9: 1.0, 4: -(2.0**24)}


def router_kat_row(d):
    w = np.zeros(d, np.float32)
    for j, v in ROUTER_KAT.items():
        w[j] = v
    return w


def test_router_lane_grouping_kat(oracle_lib):
    """The KAT above at d = 24 and d = 2048 (zeros beyond j = 16 change no
    rounding).  Plausible mistakes give other values, computed here in
    float32 to show the KAT separates them: lanes over consecutive blocks of
    j (2), one sequential sum (3), a lane chain in decreasing j (3), and the
    j = r (mod 8) lanes summed in lane order instead of the tree (0)."""
    f32 = np.float32
    for d in (24, 2048):
        w = router_kat_row(d)
        assert oracle_lib.router_dot(w, np.ones(d, np.float32)) == 1.0
    w = router_kat_row(24)

    def tree(l):
        return f32(f32(f32(l[0] + l[4]) + f32(l[2] + l[6])) + f32(f32(l[1] + l[5]) + f32(l[3] + l[7])))

    def chain(vals):
        acc = f32(0)
        for v in vals:
            acc = f32(acc + f32(v))
        return acc

    blocked = tree([chain(w[3 * r:3 * r + 3]) for r in range(8)])
    sequential = chain(w)
    reversed_chain = tree([chain(w[r::8][::-1]) for r in range(8)])
    lane_order = chain([chain(w[r::8]) for r in range(8)])
    assert tree([chain(w[r::8]) for r in range(8)]) == 1.0       # the reference's order, restated
    assert [blocked, sequential, reversed_chain, lane_order] == [2.0, 3.0, 3.0, 0.0]


def test_softmax_topk_ties_and_renorm(oracle_lib):
    s = np.array([1.0, 3.0, 3.0, 2.0, 3.0, -5.0], np.float32)
    p, top, tw = oracle_lib.softmax_topk(s, 4, renorm=False)
    assert top.tolist() == [1, 2, 4, 3]
    assert tw[0] == tw[1] == tw[2] and tw[3] < tw[0]
    _, top2, tw2 = oracle_lib.softmax_topk(s, 4, renorm=True)
    assert top2.tolist() == [1, 2, 4, 3]
    assert abs(float(tw2.astype(np.float64).sum()) - 1.0) < 4 * 2**-23
    _, top3, _ = oracle_lib.softmax_topk(np.zeros(8, np.float32), 8, renorm=True)
    assert top3.tolist() == list(range(8))
    # a NaN score gets probability 0 (the reference's expf_fast(NaN) on x86)
    s4 = np.array([np.nan, 1.0, 2.0], np.float32)
    p4, top4, tw4 = oracle_lib.softmax_topk(s4, 3, renorm=False)
    assert p4[0] == 0.0 and top4.tolist() == [2, 1, 0]


SMALL = MoEShape(d=256, m=128, E=16, topk=4, renorm=True, name="small")
SMALL_NR = MoEShape(d=256, m=128, E=16, topk=4, renorm=False, name="small-nr")


def _block(shape, group, seed=1000):
    blob, offsets = numpy_store(shape, 1, group, seed)
    gw = router_weights(shape, 0)
    return blob, offsets, gw


def _experts64(shape, blob, offsets, group):
    def get(e):
        out = []
        for p, (r, c) in enumerate(((shape.m, shape.d), (shape.m, shape.d), (shape.d, shape.m))):
            sb, pb = Q.record_sizes(r, c, group)
            so, po = (int(v) for v in offsets[p, e])
            out.append(T.dequant_matrix(blob[so:so + sb].view(np.uint16), blob[po:po + pb], r, c, group))
        return tuple(out)
    return get


@pytest.mark.parametrize("group", [64, 32])
@pytest.mark.parametrize("shape", [SMALL, SMALL_NR])
def test_block_vs_textbook(oracle_lib, shape, group):
    blob, offsets, gw = _block(shape, group)
    moe = oracle_lib.OracleMoE(shape.d, shape.m, shape.E, shape.topk, shape.renorm, group, gw, blob, offsets[:, :shape.E])
    x = np.random.default_rng(3).standard_normal((6, shape.d)).astype(np.float32)
    out, top, tw = moe.forward(x)
    logits, p, ttop, tww = T.route(gw, x, shape.topk, shape.renorm)
    # indices agree unless two probabilities are within float32 resolution
    srt = -np.sort(-p, axis=1)
    margin = (srt[:, shape.topk - 1] - srt[:, shape.topk]) / srt[:, 0]
    for b in range(x.shape[0]):
        if margin[b] > 1e-5:
            assert sorted(top[b].tolist()) == sorted(ttop[b].tolist())
            assert top[b].tolist() == ttop[b].tolist()
    assert np.allclose(tw, tww, rtol=1e-5, atol=1e-7)
    ref = T.moe_block(x, gw, _experts64(shape, blob, offsets, group), shape.topk, shape.renorm,
                      top=top, w=tw.astype(np.float64))
    err = np.abs(out - ref).max() / np.abs(ref).max()
    assert err < 2e-6, err


def test_block_invariances(oracle_lib):
    shape, group = SMALL, 64
    blob, offsets, gw = _block(shape, group)
    moe = oracle_lib.OracleMoE(shape.d, shape.m, shape.E, shape.topk, shape.renorm, group, gw, blob, offsets[:, :shape.E])
    x = np.random.default_rng(4).standard_normal((7, shape.d)).astype(np.float32)
    a = moe.forward(x, n_threads=1)
    b = moe.forward(x, n_threads=4)
    c = moe.forward(x, n_threads=3, all_tokens=True)
    for u, v in ((a, b), (a, c)):
        for p, q in zip(u, v):
            assert np.array_equal(p.view(np.uint8), q.view(np.uint8))
    # a token alone routes identically; its output differs only by the
    # union-order rounding of the combine
    for t in (0, 4):
        o1, top1, tw1 = moe.forward(x[t:t + 1])
        assert np.array_equal(top1[0], a[1][t]) and np.array_equal(tw1[0].view(np.uint32), a[2][t].view(np.uint32))
        assert np.abs(o1[0] - a[0][t]).max() <= 1e-6 * np.abs(o1[0]).max()


def test_block_bad_shapes(oracle_lib):
    shape, group = SMALL, 64
    blob, offsets, gw = _block(shape, group)
    with pytest.raises(RuntimeError):
        oracle_lib.OracleMoE(shape.d, shape.m, shape.E, shape.E + 1, True, group, gw, blob,
                             offsets[:, :shape.E]).forward(np.zeros((1, shape.d), np.float32))
    moe = oracle_lib.OracleMoE(shape.d, shape.m, shape.E, shape.topk, True, 48, gw, blob, offsets[:, :shape.E])
    with pytest.raises(RuntimeError):
        moe.forward(np.zeros((1, shape.d), np.float32))


def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    a = np.random.default_rng(1).normal(0, 3, 100000).astype(np.float32)
    a[:4] = [0.0, -0.0, 1.00390625, 1.01171875]   # exact ties -> even
    ref = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    assert np.array_equal(bf16_round(a).view(np.uint32), ref.view(np.uint32))


def test_offsets_layout_matches_writer(tmp_path):
    shape, group = MoEShape(d=128, m=64, E=3, topk=2, renorm=False), 32
    rng = np.random.default_rng(2)
    Q.write_store(tmp_path, 2, 3, lambda l, e, p: rng.normal(0, 0.02, (64, 128) if p != "down" else (128, 64)).astype(np.float32), group)
    idx = Q.Q4Index.load(tmp_path / Q.INDEX_NAME)
    tab, total = offsets_for_layout(shape, 2, group)
    assert np.array_equal(idx.offset_table(2, 3), tab)
    assert total == (tmp_path / Q.BIN_NAME).stat().st_size
