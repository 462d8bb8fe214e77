"""The oracle's AVX2 form (the timed CPU baseline) against its scalar
statement, bit for bit: the same FMA per lane and step and the same lane
reduction, so every router dot, Q4 row dot and whole block must match
exactly, including values at the edges of float32 (large, tiny, signed
zeros, infinities and NaN in the tokens)."""

import numpy as np
import pytest

from joule_amd.moe import MoEShape
from joule_amd.q4_store import quantize
from joule_amd.synth import numpy_store, router_weights


@pytest.fixture
def simd_off(oracle_lib):
    yield oracle_lib
    oracle_lib.set_simd(False)


def _edge_vectors(rng, n, d):
    x = rng.standard_normal((n, d)).astype(np.float32)
    x[0, :7] = [3.0e38, -3.0e38, 1e-45, -0.0, 0.0, 1e-38, -2.5e-39]
    x[1] *= 1e6
    x[2] *= 1e-6
    return x


@pytest.mark.parametrize("d", [8, 64, 264, 2048, 2051])
def test_router_dot_same_bits(oracle_lib, d):
    rng = np.random.default_rng(d)
    w = rng.standard_normal((5, d)).astype(np.float32)
    x = _edge_vectors(rng, 5, d)
    for i in range(5):
        a = np.float32(oracle_lib.router_dot(w[i], x[i]))
        b = np.float32(oracle_lib.router_dot_avx2(w[i], x[i]))
        assert a.view(np.uint32) == b.view(np.uint32), (d, i, a, b)


# 5, 12 and 32 groups of 64 (and twice as many of 32): whole and partial
# sets of the four interleaved groups at B=1; B of 2, 3 and 6 tokens: token
# pairs with and without an odd token left over
@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("cols", [320, 768, 2048])
@pytest.mark.parametrize("B", [1, 2, 3, 6])
def test_q4_row_dot_same_bits(oracle_lib, group, cols, B):
    rng = np.random.default_rng(group + cols + B)
    w = rng.normal(0, 0.02, (3, cols)).astype(np.float32)
    sb, pb = quantize(w, group)
    sc = np.frombuffer(sb, np.uint16).reshape(3, cols // group)
    pk = np.frombuffer(pb, np.uint8).reshape(3, cols // 2)
    X = np.ascontiguousarray(_edge_vectors(rng, 6, cols)[np.arange(B) * 5 % 6])
    for r in range(3):
        a = oracle_lib.q4_row_dot_B(pk[r], sc[r], X, cols, group)
        b = oracle_lib.q4_row_dot_B_avx2(pk[r], sc[r], X, cols, group)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (r, a, b)
    if B < 6:
        return
    Xn = X.copy()
    Xn[3, 5] = np.nan
    Xn[4, 9] = np.inf
    a = oracle_lib.q4_row_dot_B(pk[0], sc[0], Xn, cols, group)
    b = oracle_lib.q4_row_dot_B_avx2(pk[0], sc[0], Xn, cols, group)
    assert np.array_equal(np.isnan(a), np.isnan(b))
    ok = ~np.isnan(a)
    assert np.array_equal(a[ok].view(np.uint32), b[ok].view(np.uint32))


SHAPES = [MoEShape(d=512, m=256, E=16, topk=4, renorm=True, name="s"),
          MoEShape(d=256, m=512, E=24, topk=8, renorm=False, name="s2")]


@pytest.mark.parametrize("group", [64, 32])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("B,threads,all_tokens", [(1, 1, False), (5, 4, False), (8, 3, True)])
def test_block_same_bits(simd_off, shape, group, B, threads, all_tokens):
    O = simd_off
    blob, offsets = numpy_store(shape, 1, group, 1000)
    gw = router_weights(shape, 0)
    moe = O.OracleMoE(shape.d, shape.m, shape.E, shape.topk, shape.renorm, group, gw, blob, offsets[:, :shape.E])
    x = np.random.default_rng(B + group).standard_normal((B, shape.d)).astype(np.float32)
    O.set_simd(False)
    assert not O.get_simd()
    ref = moe.forward(x, n_threads=threads, all_tokens=all_tokens)
    O.set_simd(True)
    assert O.get_simd()
    got = moe.forward(x, n_threads=threads, all_tokens=all_tokens)
    for u, v in zip(ref, got):
        assert np.array_equal(np.ascontiguousarray(u).view(np.uint8), np.ascontiguousarray(v).view(np.uint8))
