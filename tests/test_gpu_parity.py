"""GPU parity: the HIP path through the C ABI against the oracle.

Bars (tolerances written here, from the target statement):
* dequantised weights: bit-exact;
* router logits, top-k indices and routing weights: bit-exact;
* block outputs: max |gpu - oracle| / max |oracle| <= 1e-3 per token, fp32
  accumulate (measured values are printed; expected ~1e-5);
* dispatch: identical to a stable sort by expert id.
Full-size layers (OLMoE and Qwen3-30B-A3B shapes) are generated and
quantised on the GPU, copied to the host for the oracle.
"""

import ctypes

import numpy as np
import pytest
import torch

from conftest import banner
from joule_amd import _lib
from joule_amd import q4_store as Q
from joule_amd.backend import HipBackend, q4_dequant
from joule_amd.moe import OLMOE, QWEN3, HbmExpertStore, MoEShape
from joule_amd.synth import (activations, apply_logit_bias, quantize_torch, router_weights,
                             torch_store, zipf_bias)

pytestmark = pytest.mark.gpu

TOL = 1e-3
TILE = 32       # tokens per MFMA-branch tile (JM_DENSE_TILE)


class Layer:
    """A full-size synthetic store on the GPU plus its host copy and oracle."""

    def __init__(self, shape: MoEShape, group: int, n_layers: int, oracle_lib):
        banner(f"build store {shape.name} G{group} L{n_layers}")
        self.shape, self.group, self.L = shape, group, n_layers
        blob, offsets = torch_store(shape, n_layers, group)
        self.store = HbmExpertStore(shape, n_layers, blob, offsets, group)
        self.gw = np.stack([router_weights(shape, l) for l in range(n_layers)])
        self.store.set_router(torch.from_numpy(self.gw).cuda())
        self.host = blob.cpu().numpy()
        self.offsets = offsets
        self.O = oracle_lib

    def oracle(self, l: int, gw=None):
        s = self.shape
        offs = self.offsets[:, l * s.E:(l + 1) * s.E]
        return self.O.OracleMoE(s.d, s.m, s.E, s.topk, s.renorm, self.group,
                                self.gw[l] if gw is None else gw, self.host, offs)


@pytest.fixture(scope="module")
def qwen64(gpu, oracle_lib):
    return Layer(QWEN3, 64, 2, oracle_lib)


@pytest.fixture(scope="module")
def olmoe64(gpu, oracle_lib):
    return Layer(OLMOE, 64, 1, oracle_lib)


@pytest.fixture(scope="module")
def qwen32(gpu, oracle_lib):
    return Layer(QWEN3, 32, 1, oracle_lib)


def _rel(a, b):
    den = np.abs(b).max(axis=1)
    return float((np.abs(a - b).max(axis=1) / np.maximum(den, 1e-30)).max())


def _run_block(layer: Layer, l: int, x: np.ndarray):
    s = layer.shape
    B = x.shape[0]
    xd = torch.from_numpy(x).cuda()
    top = torch.empty((B, s.topk), dtype=torch.int32, device="cuda")
    tw = torch.empty((B, s.topk), dtype=torch.float32, device="cuda")
    out = layer.store.layer_ffn_batch(l, xd, topk_idx=top, topk_w=tw)
    torch.cuda.synchronize()
    return out.cpu().numpy(), top.cpu().numpy(), tw.cpu().numpy()


# ------------------------------------------------------------------ format

def test_quantize_torch_matches_numpy(gpu):
    banner("quantize_torch vs numpy")
    rng = np.random.default_rng(9)
    for group in (64, 32):
        w = rng.normal(0, 0.02, (4, 96 * 256)).astype(np.float32)
        w[0, :group] = 0.0                      # an all-zero group
        sc, pk = quantize_torch(torch.from_numpy(w).cuda(), group)
        sb, pb = Q.quantize(w, group)
        assert sc.cpu().numpy().view(np.uint16).tobytes() == sb
        assert pk.cpu().numpy().tobytes() == pb


def test_dequant_bitexact_store(qwen64):
    banner("dequant store records")
    s = qwen64.shape
    for (l, e, p) in [(0, 0, 0), (0, 77, 1), (1, 127, 2)]:
        sc, pk, numel = qwen64.store.ensure(l, e)[p]
        got = q4_dequant(pk, sc, numel, 64).cpu().numpy()
        ref = Q.dequantize(sc.cpu().numpy().view(np.uint16), pk.cpu().numpy(), numel, 64)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_all_fp16_scales(gpu):
    banner("dequant exhaustive fp16 scales")
    codes = np.arange(65536, dtype=np.uint16)
    for group in (64, 32):
        sc = torch.from_numpy(codes.view(np.int16).copy()).cuda()
        pk = torch.full((65536 * group // 2,), 0x99, dtype=torch.uint8, device="cuda")  # q - 8 = +1
        got = q4_dequant(pk, sc, 65536 * group, group).cpu().numpy().reshape(65536, group)
        assert np.all(got.view(np.uint32) == got[:, :1].view(np.uint32))
        ref = codes.view(np.float16).astype(np.float32)
        nan = np.isnan(ref)
        assert np.array_equal(got[~nan, 0].view(np.uint32), ref[~nan].view(np.uint32))
        assert np.all(np.isnan(got[nan, 0]))


# ------------------------------------------------------------------ router

def _gpu_router(gw: np.ndarray, x: np.ndarray, topk: int, renorm: bool, bf16=False):
    B, d = x.shape
    E = gw.shape[0]
    w = torch.from_numpy(gw).cuda()
    if bf16:
        w = w.to(torch.bfloat16)
    xd = torch.from_numpy(x).cuda()
    logits = torch.empty((B, E), dtype=torch.float32, device="cuda")
    top = torch.empty((B, topk), dtype=torch.int32, device="cuda")
    tw = torch.empty((B, topk), dtype=torch.float32, device="cuda")
    _lib.check(_lib.lib().jm_router(_lib.ptr(w), int(bf16), _lib.ptr(xd), B, E, d, topk, int(renorm),
                                    _lib.ptr(logits), _lib.ptr(top), _lib.ptr(tw), _lib.stream_handle()))
    torch.cuda.synchronize()
    return logits.cpu().numpy(), top.cpu().numpy(), tw.cpu().numpy()


@pytest.mark.parametrize("shape", [QWEN3, OLMOE], ids=lambda s: s.name)
@pytest.mark.parametrize("B", [1, 8, 32, 512])
def test_router_bitexact(gpu, oracle_lib, shape, B):
    banner(f"router {shape.name} B={B}")
    gw = router_weights(shape, 0)
    x = activations(B, shape.d)
    lg, top, tw = _gpu_router(gw, x, shape.topk, shape.renorm)
    rl, rtop, rtw = oracle_lib.route(gw, x, shape.topk, shape.renorm)
    assert np.array_equal(lg.view(np.uint32), rl.view(np.uint32))
    assert np.array_equal(top, rtop)
    assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    lg2, top2, tw2 = _gpu_router(gw, x, shape.topk, shape.renorm, bf16=True)
    assert np.array_equal(lg2.view(np.uint32), lg.view(np.uint32)) and np.array_equal(top2, top)


@pytest.mark.parametrize("B", [2, 160])
def test_router_lane_grouping_kat(gpu, oracle_lib, B):
    """The lane-grouping known answer of tests/test_oracle_math.py through
    the GPU router (float32 and bf16 tables, d = 512 and 2048): a row whose
    products are 2^24, 1, 1, 1, -2^24 at j = 0, 8, 16, 9, 4 scores exactly 1
    against x = ones only in the reference's chain order and sum tree.
    B = 160 takes the 4-token router, whose 4 chains per lane are interleaved;
    with E = 16 (2 expert groups) half of its waves have no chains."""
    from test_oracle_math import router_kat_row
    banner(f"router lane-grouping KAT B={B}")
    for d in (512, 2048):
        gw = router_weights(MoEShape(d=d, m=64, E=16, topk=4, renorm=True), 0)
        gw[3] = router_kat_row(d)
        x = np.ones((B, d), np.float32)
        x[1::2] = activations(B // 2, d)           # other tokens between the known answers
        for bf16 in (False, True):
            lg, _, _ = _gpu_router(gw, x, 4, True, bf16=bf16)
            assert np.all(lg[0::2, 3] == 1.0), (d, bf16, lg[0::2, 3])
            rl, _, _ = oracle_lib.route(gw, x, 4, True)
            assert np.array_equal(lg.view(np.uint32), rl.view(np.uint32))


def test_router_ties_lowest_index(gpu, oracle_lib):
    banner("router ties")
    E, d, k = 64, 256, 6
    gw = router_weights(MoEShape(d=d, m=64, E=E, topk=k, renorm=True), 0)
    gw[[3, 17, 40, 63]] = gw[50]               # four experts with identical rows
    gw[[5, 9]] = gw[60] * 0                    # zero rows tie with each other
    x = activations(5, d)
    x[:, :] = np.abs(x)                        # make row 50 likely in the top-k
    gw[50] = np.abs(gw[50]) * 3
    gw[[3, 17, 40, 63]] = gw[50]
    lg, top, tw = _gpu_router(gw, x, k, True)
    rl, rtop, rtw = oracle_lib.route(gw, x, k, True)
    assert np.array_equal(top, rtop) and np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    for b in range(5):
        sel = top[b].tolist()
        assert sel[:5] == [3, 17, 40, 50, 63]   # equal probabilities, lowest index first


# ---------------------------------------------------------------- dispatch

@pytest.mark.parametrize("B,E,k", [(1, 128, 8), (8, 128, 8), (8, 64, 8), (512, 128, 8), (3, 16, 4),
                                   # top-k widths that are not powers of two, and 1 (the token of a
                                   # slot is its index over k by a multiply-high)
                                   (300, 16, 1), (100, 40, 3), (64, 24, 5)])
def test_dispatch_stable_sort(gpu, B, E, k):
    banner(f"dispatch B={B} E={E}")
    rng = np.random.default_rng(B * 31 + E)
    top = np.stack([rng.permutation(E)[:k] for _ in range(B)]).astype(np.int32)
    if B >= 8:
        top[1, min(2, k - 1)] = -1             # a slot without an expert (NaN scores)
    t = torch.from_numpy(top.ravel()).cuda()
    outs = [torch.full((n,), -7, dtype=torch.int32, device="cuda") for n in (E + 1, B * k, E, 1, E, B * k)]
    _lib.check(_lib.lib().jm_dispatch(_lib.ptr(t), B * k, E, k, *[_lib.ptr(o) for o in outs],
                                      _lib.stream_handle()))
    torch.cuda.synchronize()
    seg_off, seg_slot, active, n_active, first_slot, comb = (o.cpu().numpy() for o in outs)
    flat = top.ravel()
    valid = np.where(flat >= 0)[0]
    order = valid[np.argsort(flat[valid], kind="stable")]
    assert np.array_equal(seg_slot[:len(order)], order)
    counts = np.bincount(flat[valid], minlength=E)
    assert np.array_equal(seg_off, np.concatenate([[0], np.cumsum(counts)]))
    act = np.where(counts > 0)[0]
    assert n_active[0] == len(act) and np.array_equal(active[:len(act)], act)
    for e in act:
        assert first_slot[e] == order[seg_off[e]]
    # union order of the reference: experts in order of first appearance over (b, i)
    first = {}
    for s_, e in enumerate(flat):
        if e >= 0 and e not in first:
            first[e] = s_
    for b in range(B):
        slots = [b * k + i for i in range(k) if flat[b * k + i] >= 0]
        want = sorted(slots, key=lambda s_: first[flat[s_]]) + [-1] * (k - len(slots))
        assert comb[b * k:(b + 1) * k].tolist() == want


# ------------------------------------------------------------------- block

CASES = [("olmoe64", 1), ("olmoe64", 8), ("qwen64", 1), ("qwen64", 8), ("qwen64", 32),
         ("qwen32", 1), ("qwen32", 8)]


@pytest.mark.parametrize("which,B", CASES)
def test_block_parity(request, which, B):
    layer = request.getfixturevalue(which)
    banner(f"block {which} B={B}")
    x = activations(B, layer.shape.d)
    out, top, tw = _run_block(layer, 0, x)
    rout, rtop, rtw = layer.oracle(0).forward(x)
    assert np.array_equal(top, rtop)
    assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    err = _rel(out, rout)
    print(f"  max rel err {which} B={B}: {err:.3e}", flush=True)
    assert err <= TOL


def _host_rec(layer: Layer, l: int, e: int, p: int):
    """(scales u16, packed u8) of one record from the host copy of the store."""
    s = layer.shape
    rows, cols = ((s.m, s.d), (s.m, s.d), (s.d, s.m))[p]
    sb, pb = Q.record_sizes(rows, cols, layer.group)
    so, po = (int(v) for v in layer.offsets[p, l * s.E + e])
    return layer.host[so:so + sb].view(np.uint16), layer.host[po:po + pb]


def _union_sum(y: np.ndarray, top: np.ndarray) -> np.ndarray:
    """Each token's y rows summed in float32 in the reference's union order:
    experts by first appearance over the slots (decode_kernel.c:1502-1507)."""
    B, k = top.shape
    first = {}
    for sl, e in enumerate(top.reshape(-1)):
        first.setdefault(int(e), sl)
    out = np.zeros((B, y.shape[1]), np.float32)
    for b in range(B):
        for i in sorted(range(k), key=lambda i: first[int(top[b, i])]):
            out[b] = out[b] + y[b * k + i]
    return out


@pytest.mark.parametrize("which,B", [("qwen64", 3), ("qwen64", 40), ("qwen32", 8), ("olmoe64", 5)])
def test_block_stages_match_oracle(request, which, B):
    """The stage entry points against the reference's expert_job per slot
    (expert_ffn.c:145-191: gate/up, SwiGLU, down times the routing weight):
    act and y within the block tolerance, the union-order combine bit-exact,
    and the three stages chained against the block."""
    layer = request.getfixturevalue(which)
    banner(f"stages {which} B={B}")
    s, l = layer.shape, layer.L - 1
    x = activations(B, s.d)
    out_blk, top, tw = _run_block(layer, l, x)
    O = layer.O
    act_ref = np.empty((B * s.topk, s.m), np.float32)
    y_ref = np.empty((B * s.topk, s.d), np.float32)
    for b in range(B):
        for i in range(s.topk):
            e = int(top[b, i])
            scr = O.expert_job(_host_rec(layer, l, e, 0), _host_rec(layer, l, e, 1), _host_rec(layer, l, e, 2),
                               s.m, s.d, layer.group, x[b], float(tw[b, i]))
            act_ref[b * s.topk + i] = scr[:s.m]
            y_ref[b * s.topk + i] = scr[s.m:]
    st = layer.store
    top_d, tw_d = torch.from_numpy(top).cuda(), torch.from_numpy(tw).cuda()
    act = st.expert_gateup(l, torch.from_numpy(x).cuda(), top_d)
    y = st.expert_down(l, torch.from_numpy(act_ref).cuda(), top_d, tw_d)
    comb = st.combine(torch.from_numpy(y_ref).cuda(), top_d)
    chained = st.combine(st.expert_down(l, act, top_d, tw_d), top_d)
    torch.cuda.synchronize()
    e_act, e_y = _rel(act.cpu().numpy(), act_ref), _rel(y.cpu().numpy(), y_ref)
    e_ch = _rel(chained.cpu().numpy(), out_blk)
    print(f"  act {e_act:.3e}  y {e_y:.3e}  chained vs block {e_ch:.3e}", flush=True)
    assert e_act <= TOL and e_y <= TOL and e_ch <= TOL
    assert np.array_equal(comb.cpu().numpy().view(np.uint32), _union_sum(y_ref, top).view(np.uint32))


def test_block_stage_errors(qwen64):
    banner("stage entry point errors")
    st, s = qwen64.store, qwen64.shape
    x = torch.zeros((2, s.d), device="cuda")
    top = torch.zeros((2, s.topk), dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.JouleError):
        _lib.check(_lib.lib().jm_expert_gateup(st._h, qwen64.L, _lib.ptr(x), _lib.ptr(top), 2, _lib.ptr(x),
                                               None), "gateup")
    with pytest.raises(ValueError):
        st.expert_down(0, torch.zeros((3, s.m), device="cuda"), top, torch.zeros((2, s.topk), device="cuda"))
    e = torch.zeros((0, s.topk), dtype=torch.int32, device="cuda")
    assert st.combine(torch.zeros((0, s.d), device="cuda"), e).shape == (0, s.d)


@pytest.mark.parametrize("which", ["qwen64", "qwen32", "olmoe64"])
def test_expert_job_matches_reference(request, which):
    """jm_expert_job (the reference's ExpertJob struct with device pointers)
    against the reference's expert_job restated in the oracle, for a few
    experts and routing weights."""
    layer = request.getfixturevalue(which)
    banner(f"expert_job {which}")
    s = layer.shape
    rng = np.random.default_rng(5)
    for e, prob in ((0, 0.125), (s.E // 2, 0.5), (s.E - 1, 1.0)):
        recs = [_host_rec(layer, 0, e, p) for p in range(3)]
        x = rng.standard_normal(s.d).astype(np.float32)
        ref = layer.O.expert_job(recs[0], recs[1], recs[2], s.m, s.d, layer.group, x, prob)
        dev = [(torch.from_numpy(sc.view(np.int16).copy()).cuda(), torch.from_numpy(pk.copy()).cuda())
               for sc, pk in recs]
        xd = torch.from_numpy(x).cuda()
        scratch = torch.empty(s.m + s.d, dtype=torch.float32, device="cuda")
        j = _lib.ExpertJob(_lib.ptr(dev[0][1]), _lib.ptr(dev[0][0]), _lib.ptr(dev[1][1]), _lib.ptr(dev[1][0]),
                           _lib.ptr(dev[2][1]), _lib.ptr(dev[2][0]), s.m, s.d, s.d, s.m, layer.group,
                           _lib.ptr(xd), _lib.ptr(scratch), prob)
        _lib.check(_lib.lib().jm_expert_job(ctypes.byref(j), _lib.stream_handle()), "jm_expert_job")
        got = scratch.cpu().numpy()
        assert _rel(got[None, :s.m], ref[None, :s.m]) <= TOL
        assert _rel(got[None, s.m:], ref[None, s.m:]) <= TOL


# Decode-path shapes beyond the two model shapes: rows of 16 lanes
# (d = 1024, m = 512), gate/up rows of two chunks per lane (d = 4096) and
# down rows of 64 lanes (m > 1024).
SHAPES = [MoEShape(1024, 512, 16, 4, True, "d1024-m512"),
          MoEShape(4096, 1536, 32, 8, False, "d4096-m1536"),
          MoEShape(1024, 2048, 8, 2, True, "d1024-m2048")]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: s.name)
@pytest.mark.parametrize("B", [1, 7])
def test_block_decode_launch_shapes(gpu, oracle_lib, shape, B):
    banner(f"block {shape.name} B={B}")
    layer = Layer(shape, 64, 1, oracle_lib)
    try:
        x = activations(B, shape.d)
        out, top, tw = _run_block(layer, 0, x)
        rout, rtop, rtw = layer.oracle(0).forward(x)
        assert np.array_equal(top, rtop)
        assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
        err = _rel(out, rout)
        print(f"  max rel err {shape.name} B={B}: {err:.3e}", flush=True)
        assert err <= TOL
    finally:
        layer.store.close()


# The dispatch path (more than 256 slots) at top-k widths 3 and 1: the
# block dispatch's token index over k, the work table and the MFMA grids
# (about 12 slots per expert).
@pytest.mark.parametrize("shape,B", [(MoEShape(1024, 1024, 24, 3, True, "d1024-E24-k3"), 100),
                                     (MoEShape(1024, 1024, 16, 1, False, "d1024-E16-k1"), 260)],
                         ids=lambda v: v.name if isinstance(v, MoEShape) else str(v))
def test_block_dispatch_path_topk_widths(gpu, oracle_lib, shape, B):
    banner(f"block {shape.name} B={B}")
    layer = Layer(shape, 64, 1, oracle_lib)
    try:
        x = activations(B, shape.d)
        out, top, tw = _run_block(layer, 0, x)
        rout, rtop, rtw = layer.oracle(0).forward(x, n_threads=8)
        assert np.array_equal(top, rtop)
        assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
        err = _rel(out, rout)
        print(f"  max rel err {shape.name} B={B}: {err:.3e}", flush=True)
        assert err <= TOL
    finally:
        layer.store.close()


def test_block_second_layer_and_determinism(qwen64):
    banner("block layer 1, determinism")
    x = activations(8, QWEN3.d)
    a = _run_block(qwen64, 1, x)
    b = _run_block(qwen64, 1, x)
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint8), v.view(np.uint8))
    rout, rtop, rtw = qwen64.oracle(1).forward(x)
    assert np.array_equal(a[1], rtop) and _rel(a[0], rout) <= TOL
    c = _run_block(qwen64, 0, x)
    assert not np.array_equal(a[1], c[1])


def test_block_fp32_router_table(qwen64):
    """A router table that is not bf16-exact is kept in float32 (the other
    chain path); results stay bit-exact against the oracle."""
    banner("block fp32 router table")
    rng = np.random.default_rng(77)
    gw = rng.normal(0, 0.02, qwen64.gw.shape).astype(np.float32)
    qwen64.store.set_router(torch.from_numpy(gw).cuda())
    try:
        assert qwen64.store.router_bytes_per_weight() == 4
        x = activations(8, QWEN3.d)
        out, top, tw = _run_block(qwen64, 1, x)
        rout, rtop, rtw = qwen64.oracle(1, gw=gw[1]).forward(x)
        assert np.array_equal(top, rtop) and np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
        assert _rel(out, rout) <= TOL
    finally:
        qwen64.store.set_router(torch.from_numpy(qwen64.gw).cuda())
    assert qwen64.store.router_bytes_per_weight() == 2


def test_block_batch_invariance(qwen64):
    banner("block batch invariance")
    x = activations(8, QWEN3.d)
    full = _run_block(qwen64, 0, x)
    for t in (0, 5):
        one = _run_block(qwen64, 0, x[t:t + 1])
        assert np.array_equal(one[1][0], full[1][t])
        assert np.array_equal(one[2][0].view(np.uint32), full[2][t].view(np.uint32))
        assert np.abs(one[0][0] - full[0][t]).max() <= 1e-6 * np.abs(one[0][0]).max()


@pytest.mark.parametrize("alpha", [1.0, 0.28])
@pytest.mark.parametrize("which", ["qwen64", "qwen32", "olmoe64"])
def test_block_zipf_large_segments(request, which, alpha):
    """512 tokens with Zipf-biased routing: segments of 0 to ~500 tokens
    (alpha 1.0) or about 5 to 200 (alpha 0.28, the mix the benchmark
    times), so the MFMA branch (32-token tiles; experts past 32 tokens take
    several) runs beside the wave-item kernels."""
    layer = request.getfixturevalue(which)
    banner(f"block zipf {which} B=512 alpha={alpha}")
    s = layer.shape
    B = 512
    gw, x = apply_logit_bias(layer.gw[0], activations(B, s.d), zipf_bias(s.E, alpha=alpha))
    w = torch.from_numpy(np.stack([gw] + [layer.gw[l] for l in range(1, layer.L)])).cuda()
    layer.store.set_router(w)
    try:
        out, top, tw = _run_block(layer, 0, x)
        tiles = layer.store.dense_tiles()
    finally:
        layer.store.set_router(torch.from_numpy(layer.gw).cuda())
    counts = np.bincount(top.ravel(), minlength=s.E)
    dense = [c for c in counts if c >= 8]                                   # the default threshold
    small = sum(1 for c in counts if 0 < c < 8)
    print(f"  segment sizes: max {counts.max()} nonzero {np.count_nonzero(counts)}, "
          f"dense tiles {tiles}, experts on the wave-item kernels {small}", flush=True)
    assert counts.max() >= 2 * TILE
    assert tiles == int(sum((c + TILE - 1) // TILE for c in dense))
    rout, rtop, rtw = layer.oracle(0, gw=gw).forward(x, n_threads=8)
    assert np.array_equal(top, rtop)
    err = _rel(out, rout)
    print(f"  max rel err zipf {which} B=512 alpha={alpha}: {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("dense_min", [1, 1 << 30])
def test_block_dispatch_path_branches(qwen64, dense_min):
    """B=64 (512 slots, the dispatch path) with every expert forced onto the
    MFMA branch (dense_min=1) or onto the wave-item GEMV kernels."""
    banner(f"block B=64 dense_min={dense_min}")
    x = activations(64, QWEN3.d)
    qwen64.store.set_dense_min(dense_min)
    try:
        out, top, tw = _run_block(qwen64, 0, x)
        tiles = qwen64.store.dense_tiles()
    finally:
        qwen64.store.set_dense_min(0)
    counts = np.bincount(top.ravel(), minlength=QWEN3.E)
    if dense_min == 1:
        assert tiles == int(sum((c + TILE - 1) // TILE for c in counts if c > 0))
    else:
        assert tiles == 0
    rout, rtop, rtw = qwen64.oracle(0).forward(x)
    assert np.array_equal(top, rtop) and np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    err = _rel(out, rout)
    print(f"  max rel err B=64 dense_min={dense_min}: {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("B,dense_min", [(40, 2), (40, 4), (64, 4)])
def test_block_small_experts_on_mfma_grid(qwen64, B, dense_min):
    """The experts under dense_min run as wave items on the MFMA kernels'
    blocks past their tiles.  With a low threshold most experts take a tile
    and the surplus blocks are few (at least row blocks x small experts),
    so each runs several virtual blocks of the small experts' items."""
    banner(f"block B={B} dense_min={dense_min}: small experts on the MFMA grids")
    x = activations(B, QWEN3.d, seed=4000 + B)
    qwen64.store.set_dense_min(dense_min)
    try:
        out, top, tw = _run_block(qwen64, 0, x)
        tiles = qwen64.store.dense_tiles()
    finally:
        qwen64.store.set_dense_min(0)
    counts = np.bincount(top.ravel(), minlength=QWEN3.E)
    small = int(sum(1 for c in counts if 0 < c < dense_min))
    assert tiles == int(sum((c + TILE - 1) // TILE for c in counts if c >= dense_min))
    assert small > 0 and tiles > 0
    rout, rtop, rtw = qwen64.oracle(0).forward(x, n_threads=8)
    assert np.array_equal(top, rtop) and np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    err = _rel(out, rout)
    print(f"  B={B} dense_min={dense_min}: {tiles} tiles, {small} small experts, max rel err {err:.3e}",
          flush=True)
    assert err <= TOL


def test_block_nan_tokens(qwen64):
    """A NaN token has NaN scores: every probability is NaN, no expert beats
    -1e30, its k slots get index -1 and it contributes nothing (the
    reference would index expert -1; here the slot is skipped)."""
    banner("block NaN tokens")
    x = activations(8, QWEN3.d)
    x[3, 100] = np.nan
    out, top, tw = _run_block(qwen64, 0, x)
    rout, rtop, rtw = qwen64.oracle(0).forward(x)
    assert np.all(top[3] == -1) and np.array_equal(top, rtop)
    assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    assert np.all(out[3] == 0.0)
    keep = [b for b in range(8) if b != 3]
    assert _rel(out[keep], rout[keep]) <= TOL
    xa = np.full((2, QWEN3.d), np.nan, np.float32)
    out2, top2, _ = _run_block(qwen64, 0, xa)
    assert np.all(top2 == -1) and np.all(out2 == 0.0)


def _shuffled_store(layer: "Layer"):
    """The same records in another order (parts and experts interleaved
    out of (layer, expert, part) order, with gaps), and its offset table:
    the kernels must then locate records through the table."""
    s = layer.shape
    host = layer.host
    offs = layer.offsets
    LE = offs.shape[1]
    recs = []
    for p in range(3):
        for key in range(LE):
            so, po = (int(v) for v in offs[p, key])
            sb, pb = po - so, Q.record_sizes(*((s.m, s.d) if p < 2 else (s.d, s.m)), layer.group)[1]
            recs.append((p, key, so, sb, pb))
    rng = np.random.default_rng(5)
    order = rng.permutation(len(recs))
    parts, new = [], np.zeros_like(offs)
    pos = 0
    for i in order:
        p, key, so, sb, pb = recs[i]
        pos += 256                                   # a gap before every record
        parts.append((pos, host[so:so + sb + pb]))
        new[p, key] = (pos, pos + sb)
        pos = (pos + sb + pb + 15) // 16 * 16
    blob = np.zeros(pos, np.uint8)
    for at, data in parts:
        blob[at:at + len(data)] = data
    st = HbmExpertStore(s, layer.L, torch.from_numpy(blob).cuda(), new, layer.group)
    st.set_router(torch.from_numpy(layer.gw).cuda())
    return st


def test_block_record_table_layout(qwen64):
    """A store whose records are not in (layer, expert, part) order gives the
    bit-identical block on the decode path, the GEMV dispatch path and the
    MFMA branch."""
    banner("block shuffled record layout")
    shuffled = _shuffled_store(qwen64)
    for B, dense_min in ((8, 0), (64, 1 << 30), (64, 1)):
        x = torch.from_numpy(activations(B, QWEN3.d)).cuda()
        outs = []
        for st in (qwen64.store, shuffled):
            st.set_dense_min(dense_min)
            outs.append(st.layer_ffn_batch(1, x).cpu().numpy())
            st.set_dense_min(0)
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), (B, dense_min)
    shuffled.close()


def test_block_empty_and_errors(qwen64):
    banner("block B=0 and argument errors")
    s = QWEN3
    x = torch.zeros((0, s.d), dtype=torch.float32, device="cuda")
    out = qwen64.store.layer_ffn_batch(0, x)
    assert out.shape == (0, s.d)
    with pytest.raises(_lib.JouleError):
        qwen64.store.layer_ffn_batch(2, torch.zeros((1, s.d), device="cuda"))
    with pytest.raises(_lib.JouleError):
        bad = torch.zeros(s.d + 1, device="cuda")[1:].view(1, s.d)
        qwen64.store.layer_ffn_batch(0, bad)


# ----------------------------------------------------------------- backend

@pytest.mark.parametrize("group", [64, 32])
@pytest.mark.parametrize("m,d,T", [(768, 2048, 1), (2048, 768, 3), (1024, 2048, 6),
                                   # from 7 tokens (the default crossover) the matrix cores (m a
                                   # multiple of 256): whole and partial 32-token tiles, one and two
                                   # 256-row passes per block
                                   (1024, 2048, 7), (768, 2048, 21),
                                   (768, 2048, 22), (768, 2048, 33), (2048, 768, 70), (8192, 512, 512),
                                   # the contraction split over 8, 2 and 4 blocks per tile and row block
                                   # (fewer than 256 blocks otherwise; 2048 x 768 above: 3), the partial
                                   # sums added afterwards
                                   (256, 2048, 30), (8192, 512, 128), (8192, 1024, 64),
                                   # shapes the matrix-core kernel does not take: the digit kernel
                                   (1000, 2048, 40), (768, 1536, 36)])
def test_hip_backend_q4_gemm(gpu, oracle_lib, group, m, d, T):
    banner(f"HipBackend q4_gemm m={m} d={d} T={T} G{group}")
    rng = np.random.default_rng(m + d + T)
    w = rng.normal(0, 0.02, (m, d)).astype(np.float32)
    sb, pb = Q.quantize(w, group)
    sc = np.frombuffer(sb, np.uint16).copy()
    pk = np.frombuffer(pb, np.uint8).copy()
    X = rng.standard_normal((T, d)).astype(np.float32)
    be = HipBackend()
    out = torch.empty((T, m), dtype=torch.float32, device="cuda")
    be.q4_gemm(out, torch.from_numpy(X).cuda(), pk, sc, m, d, group)
    ref = oracle_lib.q4_gemm_ffn(X, pk, sc, m, d, group)
    torch.cuda.synchronize()
    assert _rel(out.cpu().numpy(), ref) <= TOL
    v = be.q4_gemv(torch.from_numpy(X[0]).cuda(), pk, sc, m, d, group).cpu().numpy()
    assert _rel(v[None], ref[:1]) <= TOL


@pytest.mark.parametrize("T", [1, 5, 40])
def test_q4_gemm_min_tokens_switch(gpu, oracle_lib, T):
    """Both kernels of the plugin product forced at the same T (the switch
    the bench's crossover sweep uses) agree with the oracle; 0 restores the
    default threshold."""
    banner(f"q4_gemm kernel switch T={T}")
    L = _lib.lib()
    m, d, group = 768, 2048, 64
    rng = np.random.default_rng(90 + T)
    sb, pb = Q.quantize(rng.normal(0, 0.02, (m, d)).astype(np.float32), group)
    sc = np.frombuffer(sb, np.uint16).copy()
    pk = np.frombuffer(pb, np.uint8).copy()
    X = rng.standard_normal((T, d)).astype(np.float32)
    ref = oracle_lib.q4_gemm_ffn(X, pk, sc, m, d, group)
    be = HipBackend()
    default = L.jm_get_q4_gemm_min_tokens()
    try:
        for min_t in (1, 1 << 30):
            assert L.jm_set_q4_gemm_min_tokens(min_t) == 0
            assert L.jm_get_q4_gemm_min_tokens() == min_t
            out = torch.empty((T, m), dtype=torch.float32, device="cuda")
            be.q4_gemm(out, torch.from_numpy(X).cuda(), pk, sc, m, d, group)
            torch.cuda.synchronize()
            assert _rel(out.cpu().numpy(), ref) <= TOL, min_t
    finally:
        assert L.jm_set_q4_gemm_min_tokens(0) == 0
    assert L.jm_get_q4_gemm_min_tokens() == default
    assert L.jm_set_q4_gemm_min_tokens(-1) == -1


# ------------------------------------------------- five activation digits

def _p99(a, b):
    """99th percentile of |a - b| / |b| over the outputs with |b| at least
    1e-3 of their token's largest."""
    ref = np.abs(b).max(axis=1, keepdims=True)
    keep = np.abs(b) >= 1e-3 * ref
    return float(np.percentile((np.abs(a - b)[keep] / np.abs(b)[keep]), 99))


@pytest.mark.parametrize("which,B", [("qwen64", 1), ("qwen64", 8), ("qwen64", 40), ("olmoe64", 8), ("qwen32", 8)])
def test_block_five_digits(request, which, B):
    """With 5 digit planes per activation value (jm_store_set_act_digits) the
    GEMV kernels carry about 19 bits per group instead of 15: routing stays
    bit-exact, the normwise error drops by more than 4x against the 4-digit
    run of the same call, and the elementwise p99 is under the 1e-3 bar.
    B=40 (320 slots) takes the dispatch path's kernels."""
    layer = request.getfixturevalue(which)
    banner(f"block five digits {which} B={B}")
    st = layer.store
    x = activations(B, layer.shape.d)
    rout, rtop, rtw = layer.oracle(0).forward(x)
    assert st.act_digits == 4
    st.set_dense_min(1 << 30)                 # every expert on the GEMV kernels, also past 256 slots
    try:
        out4, _, _ = _run_block(layer, 0, x)
        st.set_act_digits(5)
        assert st.act_digits == 5
        out5, top, tw = _run_block(layer, 0, x)
    finally:
        st.set_act_digits(0)
        st.set_dense_min(0)
    assert st.act_digits == 4
    assert np.array_equal(top, rtop)
    assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    e4, e5, p5 = _rel(out4, rout), _rel(out5, rout), _p99(out5, rout)
    print(f"  normwise 4 digits {e4:.3e}, 5 digits {e5:.3e}; elementwise p99 {p5:.3e}", flush=True)
    assert e5 <= 2e-5 and e5 * 4 <= e4 and p5 <= 1e-3


def test_block_five_digits_zipf_and_stages(qwen64):
    """5 digits on the MFMA grids' small-expert items (512 Zipf-routed
    tokens) and on the stage entry points (x and act digits through the same
    encoder), against the oracle."""
    layer, s = qwen64, qwen64.shape
    banner("five digits: zipf 512 and stages")
    st = layer.store
    gw, x = apply_logit_bias(layer.gw[0], activations(512, s.d), zipf_bias(s.E, alpha=0.28))
    st.set_router(torch.from_numpy(np.stack([gw] + [layer.gw[l] for l in range(1, layer.L)])).cuda())
    try:
        st.set_act_digits(5)
        out, top, _ = _run_block(layer, 0, x)
    finally:
        st.set_act_digits(0)
        st.set_router(torch.from_numpy(layer.gw).cuda())
    rout, rtop, _ = layer.oracle(0, gw=gw).forward(x, n_threads=8)
    assert np.array_equal(top, rtop)
    err = _rel(out, rout)
    print(f"  zipf 512 five digits: {err:.3e}", flush=True)
    assert err <= TOL
    # the stages at B = 8
    B, l = 8, 0
    x8 = activations(B, s.d)
    _, top8, tw8 = _run_block(layer, l, x8)
    top_d, tw_d = torch.from_numpy(top8).cuda(), torch.from_numpy(tw8).cuda()
    O = layer.O
    act_ref = np.empty((B * s.topk, s.m), np.float32)
    for b in range(B):
        for i in range(s.topk):
            e = int(top8[b, i])
            act_ref[b * s.topk + i] = O.expert_job(_host_rec(layer, l, e, 0), _host_rec(layer, l, e, 1),
                                                   _host_rec(layer, l, e, 2), s.m, s.d, layer.group, x8[b],
                                                   1.0)[:s.m]
    errs = {}
    for nd in (4, 5):
        try:
            st.set_act_digits(nd)
            act = st.expert_gateup(l, torch.from_numpy(x8).cuda(), top_d)
            torch.cuda.synchronize()
        finally:
            st.set_act_digits(0)
        errs[nd] = _rel(act.cpu().numpy(), act_ref)
    print(f"  stage act error: 4 digits {errs[4]:.3e}, 5 digits {errs[5]:.3e}", flush=True)
    assert errs[5] <= 2e-5 and errs[5] * 4 <= errs[4]


def test_act_digits_setting_errors(qwen64):
    banner("act digits setting")
    st = qwen64.store
    for bad in (1, 3, 6, -1):
        with pytest.raises(_lib.JouleError):
            st.set_act_digits(bad)
    assert st.act_digits == 4
