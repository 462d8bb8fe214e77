"""GPU parity of the batch decode (jm_decode_layers_batch) with the CPU
restatement of decode_layers_batch (oracle/decoder.py, decode_kernel.c:1518-1556).

Each case builds a small model on the GPU (Q4 expert store, bf16 attention
weights with jittered norm weights, a bf16 KV cache filled with N(0, 1)),
runs the decode for a batch with ragged positions, and checks:
  * the final hidden state within 1e-3 max relative error per token;
  * the cache rows written at the positions against the oracle's (bf16
    values; at most one bf16 unit apart, nearly all identical);
  * a second step at the next positions, which reads the rows the first
    step appended.
"""

import ctypes

import numpy as np
import pytest
import torch

from joule_amd import _lib
from joule_amd.decoder import DecoderShape, DecoderWeights, HipDecoder, KVCacheSet, qwen3_30b_a3b
from joule_amd.moe import HbmExpertStore, MoEShape
from joule_amd.synth import activations, decoder_weights, fill_kv, router_weights, torch_store
from oracle import decoder as D
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _model(shape: DecoderShape, group: int, B: int, kv_dtype=torch.bfloat16):
    L, moe = shape.n_layers, shape.moe
    blob, offsets = torch_store(moe, L, group)
    store = HbmExpertStore(moe, L, blob, offsets, group)
    gw = np.stack([router_weights(moe, l) for l in range(L)])
    store.set_router(torch.from_numpy(gw).cuda())
    t = decoder_weights(shape, norm_jitter=0.1)
    weights = DecoderWeights(shape, **t)
    kv = KVCacheSet(shape, B, dtype=kv_dtype)
    fill_kv(kv.data)
    torch.cuda.synchronize()
    # the oracle's copies
    w = {k: v.float().cpu().numpy() for k, v in weights.t.items()}
    blob_h = blob.cpu().numpy()
    moe_o = [O.OracleMoE(moe.d, moe.m, moe.E, moe.topk, moe.renorm, group, gw[l], blob_h,
                         offsets[:, l * moe.E:(l + 1) * moe.E]) for l in range(L)]
    oracle = D.OracleDecoder(L, moe.d, shape.n_heads, shape.n_kv, shape.hd, shape.eps, shape.qk_norm_type,
                             shape.bias_qkv, w, moe_o, kv_bf16=kv_dtype == torch.bfloat16)
    return HipDecoder(store, weights), oracle, kv


def _kv_host(kv: KVCacheSet, B: int, L: int):
    d = kv.data.float().cpu().numpy()
    return [[(d[b, l, 0].copy(), d[b, l, 1].copy()) for l in range(L)] for b in range(B)]


def _check_step(dec, oracle, kv, kv_h, x, positions, label):
    B, L = x.shape[0], dec.shape.n_layers
    print(f"[decode] {label} B={B} L={L} positions={list(positions)}", flush=True)
    hid = dec.decode_layers_batch(torch.from_numpy(x).cuda(), positions, kv)
    torch.cuda.synchronize()
    got = hid.cpu().numpy()
    want = oracle.decode_layers_batch(x, positions, kv_h)
    rel = np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)
    assert np.isfinite(got).all()
    assert rel.max() <= TOL, f"{label}: per-token max rel error {rel}"
    # cache rows appended at the positions
    data = kv.data
    f32 = data.dtype == torch.float32
    n_same = n_all = 0
    for b, p in enumerate(positions):
        for l in range(L):
            for j in (0, 1):
                g = data[b, l, j, p].float().cpu().numpy()
                r = kv_h[b][l][j][p]
                # one bf16 unit (bf16 caches), plus the upstream float32
                # differences, which scale with the row (not with elements
                # near zero)
                lim = np.abs(r) * (0.0 if f32 else 2.0 ** -7) + 1e-4 * np.abs(r).max()
                bad = int((np.abs(g - r) > lim).sum())
                assert bad == 0, f"{label}: cache row b={b} l={l} {'kv'[j]}: {bad} values off by more than the bound"
                n_same += int((g == r).sum())
                n_all += g.size
    # bf16 rows are nearly all the same bf16 value; float32 rows differ in
    # their last bits
    assert f32 or n_same >= 0.98 * n_all, f"{label}: {n_all - n_same} of {n_all} cache values differ"
    return rel.max()


CASES = {
    # Qwen3-30B-A3B layers (GQA 32/4, per-head QK-norm), ragged positions
    # across split boundaries (128) and up to 2048
    "qwen3_l2_b8": (qwen3_30b_a3b(n_layers=2, maxT=2176), 64, [0, 1, 127, 128, 129, 700, 2047, 2048]),
    # no GQA, no QK-norm, QKV bias, 16 experts top-4 without renormalisation
    "mha_bias_l2_b3": (DecoderShape(n_layers=2, moe=MoEShape(d=1024, m=256, E=16, topk=4, renorm=False),
                                    n_heads=8, n_kv=8, maxT=300, qk_norm_type=0, bias_qkv=True), 64, [5, 0, 299]),
    # 4 query heads per KV head, group 32
    "gqa4_l1_b2": (DecoderShape(n_layers=1, moe=MoEShape(d=1024, m=512, E=32, topk=8, renorm=True),
                                n_heads=8, n_kv=2, maxT=520), 32, [511, 256]),
    # 2 query heads per KV head, d 2048
    "gqa2_l1_b5": (DecoderShape(n_layers=1, moe=MoEShape(d=2048, m=768, E=64, topk=4, renorm=True),
                                n_heads=16, n_kv=8, maxT=260), 64, [3, 130, 255, 64, 200]),
    # OLMoE-1B-7B layers: 16 heads without GQA, the whole-vector QK-norm
    # (qk_norm_type 2), 64 experts top-8 without renormalisation
    "olmoe_l2_b4": (DecoderShape(n_layers=2, moe=MoEShape(d=2048, m=1024, E=64, topk=8, renorm=False),
                                 n_heads=16, n_kv=16, maxT=300, qk_norm_type=2), 64, [0, 129, 255, 299]),
    # the whole-vector QK-norm after the QKV bias, with GQA
    "whole_bias_gqa2_l1_b3": (DecoderShape(n_layers=1, moe=MoEShape(d=1024, m=256, E=16, topk=4, renorm=True),
                                           n_heads=8, n_kv=4, maxT=200, qk_norm_type=2, bias_qkv=True),
                              32, [7, 150, 64]),
    # float32 caches, the reference's KVCache type: Qwen3 layers (8 query
    # heads per KV head), and OLMoE layers (one per KV head, whole-vector norm)
    "qwen3_l2_b8_f32kv": (qwen3_30b_a3b(n_layers=2, maxT=2176), 64, [0, 1, 127, 128, 129, 700, 2047, 2048],
                          torch.float32),
    "olmoe_l1_b3_f32kv": (DecoderShape(n_layers=1, moe=MoEShape(d=2048, m=1024, E=64, topk=8, renorm=False),
                                       n_heads=16, n_kv=16, maxT=300, qk_norm_type=2), 64, [31, 128, 299],
                          torch.float32),
    "gqa2_bias_l1_b2_f32kv": (DecoderShape(n_layers=1, moe=MoEShape(d=1024, m=256, E=16, topk=4, renorm=True),
                                           n_heads=8, n_kv=4, maxT=200, qk_norm_type=1, bias_qkv=True),
                              32, [0, 199], torch.float32),
    # one token: the o_proj merges the attention splits itself (17 splits
    # at position 2048, one at position 0, a split boundary at 127 -> 128)
    "qwen3_l2_b1": (qwen3_30b_a3b(n_layers=2, maxT=2176), 64, [2048]),
    "qwen3_l1_b1_p0": (qwen3_30b_a3b(n_layers=1, maxT=300), 64, [0]),
    "gqa4_l1_b1_p127": (DecoderShape(n_layers=1, moe=MoEShape(d=1024, m=512, E=32, topk=8, renorm=True),
                                     n_heads=8, n_kv=2, maxT=520), 32, [127]),
    "olmoe_l1_b1_f32kv": (DecoderShape(n_layers=1, moe=MoEShape(d=2048, m=1024, E=64, topk=8, renorm=False),
                                       n_heads=16, n_kv=16, maxT=300, qk_norm_type=2), 64, [255],
                          torch.float32),
}


@pytest.mark.parametrize("case", list(CASES))
def test_decode_layers_batch_matches_oracle(case):
    shape, group, positions = CASES[case][:3]
    kv_dtype = CASES[case][3] if len(CASES[case]) > 3 else torch.bfloat16
    B = len(positions)
    dec, oracle, kv = _model(shape, group, B, kv_dtype)
    kv_h = _kv_host(kv, B, shape.n_layers)
    x = activations(B, shape.d)
    _check_step(dec, oracle, kv, kv_h, x, positions, case)
    # next step: one position further, reading the rows just appended
    nxt = [min(p + 1, shape.maxT - 1) for p in positions]
    x2 = activations(B, shape.d, seed=3100)
    _check_step(dec, oracle, kv, kv_h, x2, nxt, case + " step 2")
    dec.store.close()


def test_decode_split_profile_and_errors():
    shape = DecoderShape(n_layers=1, moe=MoEShape(d=1024, m=256, E=16, topk=4, renorm=True),
                         n_heads=8, n_kv=2, maxT=256)
    dec, _, kv = _model(shape, 64, 2)
    x = torch.from_numpy(activations(2, shape.d)).cuda()
    L = _lib.lib()
    st = _lib.stream_handle()
    cfg, w = dec._cfg, dec._w
    pos = np.array([3, 256], np.int32)            # 256 >= maxT
    rc = L.jm_decode_layers_batch(dec.store._h, ctypes.byref(cfg), ctypes.byref(w), ctypes.cast(kv.table, ctypes.c_void_p),
                                  pos.ctypes.data_as(ctypes.c_void_p), _lib.ptr(x), 2, None, _lib.ptr(x), st)
    assert rc == -1 and b"positions" in L.jm_last_error()
    pos = np.array([3, 4], np.int32)
    rc = L.jm_decode_layers_batch(dec.store._h, ctypes.byref(cfg), ctypes.byref(w), ctypes.cast(kv.table, ctypes.c_void_p),
                                  pos.ctypes.data_as(ctypes.c_void_p), _lib.ptr(x), 2, _lib.ptr(x), _lib.ptr(x), st)
    assert rc == -1 and b"lm_head" in L.jm_last_error()
    bad = shape.kernel_cfg()
    bad.hd = 64
    rc = L.jm_decode_layers_batch(dec.store._h, ctypes.byref(bad), ctypes.byref(w), ctypes.cast(kv.table, ctypes.c_void_p),
                                  pos.ctypes.data_as(ctypes.c_void_p), _lib.ptr(x), 2, None, _lib.ptr(x), st)
    assert rc == -2
    # profiled call: attention + MoE parts within the whole
    dec.store.profile(True)
    dec.decode_layers_batch(x, [3, 4], kv)
    ms = dec.split_ms()
    assert ms["attention"] > 0 and ms["moe"] > 0 and ms["attention"] + ms["moe"] <= ms["total"] * 1.001
    dec.store.profile(False)
    dec.store.close()


@pytest.mark.parametrize("shape_name,position", [("qwen3", 2048), ("qwen3", 128), ("gqa4", 300)])
def test_decode_one_token_matches_batch(shape_name, position):
    """A one-token step (its o_proj merges the attention splits) gives the
    bits of token 0 of a two-token step (the split-merge kernel) when both
    tokens carry the same input, position and cache contents."""
    if shape_name == "qwen3":
        shape, group = qwen3_30b_a3b(n_layers=2, maxT=2176), 64
    else:
        shape, group = DecoderShape(n_layers=1, moe=MoEShape(d=1024, m=512, E=32, topk=8, renorm=True),
                                    n_heads=8, n_kv=2, maxT=520), 32
    print(f"[decode] one token vs two at position {position}, {shape_name}", flush=True)
    dec, _, kv2 = _model(shape, group, 2)
    kv2.data[1].copy_(kv2.data[0])
    kv1 = KVCacheSet(shape, 1, dtype=kv2.data.dtype)
    kv1.data.copy_(kv2.data[0:1])
    x = activations(1, shape.d)
    x2 = np.concatenate([x, x])
    for graph in (False, True):
        dec.set_graph(graph)
        one = dec.decode_layers_batch(torch.from_numpy(x).cuda(), [position], kv1).clone()
        two = dec.decode_layers_batch(torch.from_numpy(x2).cuda(), [position, position], kv2).clone()
        torch.cuda.synchronize()
        assert torch.equal(two[0], two[1])
        assert torch.equal(one[0], two[0]), f"graph={graph}: one-token step differs from the batch's token 0"
        assert torch.equal(kv1.data[0], kv2.data[0])
    dec.store.close()


@pytest.mark.parametrize("B,kv_dtype", [(4, torch.bfloat16), (40, torch.bfloat16), (4, torch.float32),
                                        (1, torch.bfloat16)])
def test_decode_graph_replays_match_eager(B, kv_dtype):
    """The step replayed from a captured HIP graph gives the eager step's bits,
    replay after replay, with eager work and synchronisation in between; new
    positions within the same split count replay the same graph, a new split
    count records a new one.  B=40 (320 slots) takes the MoE dispatch path
    (the small experts run on the MFMA kernels' last blocks); float32 caches
    take the float32 attention kernels."""
    shape = qwen3_30b_a3b(n_layers=2, maxT=400)
    dec, _, kv = _model(shape, 64, B, kv_dtype)
    x = torch.from_numpy(activations(B, shape.d)).cuda()
    hid = torch.empty_like(x)
    if B == 4:
        sets = ([10, 130, 257, 300], [11, 131, 258, 301], [11, 131, 258, 399])
    else:
        p1 = [10 + 7 * i for i in range(B)]
        sets = (p1, [p + 1 for p in p1], [p + 1 for p in p1[:-1]] + [399])
    for pos in sets:
        print(f"[decode] graph replays at positions {pos}", flush=True)
        dec.set_graph(False)
        want = dec.decode_layers_batch(x, pos, kv, torch.empty_like(x)).clone()
        torch.cuda.synchronize()
        dec.set_graph(True)
        for i in range(3):
            got = dec.decode_layers_batch(x, pos, kv, hid)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"positions {pos}: replay {i} differs from the eager step"
            # eager work in between: torch reductions and an eager decode step
            assert float((x * 2).abs().sum().item()) > 0
            dec.set_graph(False)
            again = dec.decode_layers_batch(x, pos, kv, torch.empty_like(x))
            torch.cuda.synchronize()
            assert torch.equal(again, want)
            dec.set_graph(True)
    dec.store.close()


def _lm_model(V=5003, d=2048, seed=21):
    """A one-layer Qwen3-shaped decoder with a vocabulary of V rows: embedding
    and lm_head bf16 N(0, 0.02)."""
    shape = DecoderShape(n_layers=1, moe=MoEShape(d=d, m=768, E=128, topk=8, renorm=True),
                         n_heads=16, n_kv=4, maxT=300, V=V)
    dec, oracle, kv = _model(shape, 64, 8)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    lm = (torch.randn((V, d), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    emb = (torch.randn((V, d), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    return shape, dec, oracle, kv, lm, emb


@pytest.mark.parametrize("B", [1, 3, 8])
def test_lm_head_logits_and_argmax(B):
    """jm_lm_head against float64 logits of the same bf16 rows (1e-5), and its
    argmax against lm_head_A's choice on the GPU's own logits (exact):
    duplicated rows tie and the lower one wins, NaN rows never win."""
    shape, dec, _, _, lm, _ = _lm_model()
    V, d = shape.V, shape.d
    lm = lm.clone()
    lm[4000] = lm[17] = lm[17] * 0                  # two identical rows ...
    lm[17, :8] = 1.0                                # ... made the largest for token 0
    lm[4000] = lm[17]
    lm[100] = float("nan")                          # a NaN row: NaN logits never win
    dec.set_lm_head(lm.float())                     # float32 holding bf16 values, as the reference's
    x = torch.from_numpy(activations(B, d)).cuda()
    x[0, :8] = 5.0
    logits = torch.empty((B, V), dtype=torch.float32, device="cuda")
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    print(f"[lm_head] B={B} V={V}", flush=True)
    dec.lm_head(x, logits, tok)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    want = (x.double() @ lm.double().T).cpu().numpy()
    ok = ~np.isnan(want)
    assert np.isnan(got[:, 100]).all() and np.array_equal(np.isnan(got), ~ok)
    rel = np.abs(got - want)[ok].max() / np.abs(want[ok]).max()
    assert rel < 1e-5, rel
    t = tok.cpu().numpy()
    assert np.array_equal(t, D.argmax_strict(got))
    assert t[0] == 17 and got[0, 17] == got[0, 4000]
    # argmax alone (no logits) gives the same rows
    tok2 = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    dec.lm_head(x, None, tok2)
    assert torch.equal(tok, tok2)
    dec.store.close()


def test_decode_argmax_and_embedding():
    """Tokens in, tokens out: embedding rows, one decode step with the
    lm_head, the argmax decode, against the oracle (logits within 1e-3; the
    argmax equal wherever the oracle's top two logits are apart by more than
    the tolerance), and a second step that reads the appended rows."""
    shape, dec, oracle, kv, lm, emb = _lm_model()
    t = dict(dec.weights.t)
    dec.weights.t["embed"] = emb
    dec._w = dec.weights.kernel_w()
    dec.set_lm_head(lm)
    V, B = shape.V, 8
    kv_h = _kv_host(kv, B, shape.n_layers)
    E = emb.float().cpu().numpy()
    W = lm.float().cpu().numpy()
    tokens = np.array([0, 1, 17, 4095, 5002, 777, 3, 2500], np.int32)
    pos = [0, 5, 130, 200, 250, 299, 128, 127]
    for step in range(2):
        print(f"[decode argmax] step {step} tokens {tokens.tolist()}", flush=True)
        x = dec.embed(torch.from_numpy(tokens).cuda())
        torch.cuda.synchronize()
        xh = D.embed_lookup(E, tokens)
        assert np.array_equal(x.cpu().numpy(), xh)
        got_tok = dec.decode_layers_batch_argmax(x, pos, kv).cpu().numpy()
        # the same step again with logits (the cache rows are rewritten with the same values)
        logits = torch.empty((B, V), dtype=torch.float32, device="cuda")
        dec.decode_layers_batch(x, pos, kv, logits=logits)
        torch.cuda.synchronize()
        gl = logits.cpu().numpy()
        assert np.array_equal(got_tok, D.argmax_strict(gl))
        hid = oracle.decode_layers_batch(xh, pos, kv_h)
        wl = D.lm_head(W, hid)
        rel = np.abs(gl - wl).max(axis=1) / np.abs(wl).max(axis=1)
        assert rel.max() < TOL, rel
        want_tok = D.argmax_strict(wl)
        top2 = np.sort(wl, axis=1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > TOL * np.abs(top2[:, 1])
        assert np.array_equal(got_tok[clear], want_tok[clear])
        tokens = got_tok.astype(np.int32)
        pos = [p + 1 if p + 1 < shape.maxT else p for p in pos]
    # a token outside the vocabulary embeds as NaN
    bad = dec.embed(torch.tensor([V, -1, 5], dtype=torch.int32, device="cuda")).cpu().numpy()
    assert np.isnan(bad[:2]).all() and np.array_equal(bad[2], E[5])
    dec.store.close()


def test_decode_graph_follows_router_dtype_and_max_layers():
    """A captured step is recorded again when the router copy changes element
    type (a bf16-exact table, then a float32 one, possibly at the same
    address) and when set_max_layers changes the layer count; the replays
    equal the eager steps, and the step stopped after one layer equals the
    oracle's first layer followed by the final norm."""
    shape = qwen3_30b_a3b(n_layers=2, maxT=300)
    B = 4
    dec, oracle, kv = _model(shape, 64, B)
    kv_h = _kv_host(kv, B, shape.n_layers)
    x = torch.from_numpy(activations(B, shape.d)).cuda()
    pos = [10, 20, 130, 299]
    hid = torch.empty_like(x)
    print("[decode] graph with the bf16 router copy", flush=True)
    dec.set_graph(True)
    a = dec.decode_layers_batch(x, pos, kv, hid).clone()
    rng = np.random.default_rng(31)
    gw32 = rng.normal(0, 0.02, (shape.n_layers, shape.moe.E, shape.d)).astype(np.float32)
    dec.store.set_router(torch.from_numpy(gw32).cuda())
    assert dec.store.router_bytes_per_weight() == 4
    print("[decode] graph with the float32 router copy", flush=True)
    g1 = dec.decode_layers_batch(x, pos, kv, hid).clone()
    dec.set_graph(False)
    e1 = dec.decode_layers_batch(x, pos, kv, torch.empty_like(x))
    torch.cuda.synchronize()
    assert torch.equal(g1, e1) and not torch.equal(a, g1)
    # one layer only, graph and eager, against the oracle
    gw = np.stack([router_weights(shape.moe, l) for l in range(shape.n_layers)])
    dec.store.set_router(torch.from_numpy(gw).cuda())
    print("[decode] set_max_layers(1)", flush=True)
    dec.set_max_layers(1)
    dec.set_graph(True)
    one_g = dec.decode_layers_batch(x, pos, kv, hid).clone()
    dec.set_graph(False)
    one_e = dec.decode_layers_batch(x, pos, kv, torch.empty_like(x))
    torch.cuda.synchronize()
    assert torch.equal(one_g, one_e)
    trace = []
    oracle.decode_layers_batch(x.cpu().numpy(), pos, kv_h, trace=trace)
    want = trace[0]["hidden"]
    got = one_e.cpu().numpy()
    rel = np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)
    assert rel.max() <= TOL, rel
    dec.set_max_layers(-1)
    full = dec.decode_layers_batch(x, pos, kv, torch.empty_like(x)).cpu().numpy()
    rel = np.abs(full - trace[1]["hidden"]).max(axis=1) / np.abs(trace[1]["hidden"]).max(axis=1)
    assert rel.max() <= TOL, rel
    dec.store.close()


def test_decode_five_digits_and_graph_key():
    """The decode step with 5 activation digit planes: within the tolerance
    of the oracle, graph replay equal to the eager step, and a change of the
    setting records a new graph (the 4-digit replay equals the 4-digit eager
    step, not the 5-digit one)."""
    shape = qwen3_30b_a3b(n_layers=2, maxT=2176)
    B = 4
    dec, oracle, kv = _model(shape, 64, B)
    kv_h = _kv_host(kv, B, shape.n_layers)
    x = activations(B, shape.d)
    positions = [5, 300, 1000, 2048]
    st = dec.store
    try:
        st.set_act_digits(5)
        err5 = _check_step(dec, oracle, kv, kv_h, x, positions, "five digits")
        xd = torch.from_numpy(x).cuda()
        want = {}
        for nd in (5, 4):
            st.set_act_digits(nd)
            dec.set_graph(False)
            want[nd] = dec.decode_layers_batch(xd, positions, kv, torch.empty_like(xd)).clone()
            dec.set_graph(True)
            got = dec.decode_layers_batch(xd, positions, kv, torch.empty_like(xd)).clone()
            torch.cuda.synchronize()
            assert torch.equal(got, want[nd]), f"{nd} digits: graph replay differs from the eager step"
        assert not torch.equal(want[4], want[5])
        print(f"  five-digit step error {err5:.3e}", flush=True)
    finally:
        st.set_act_digits(0)
        dec.store.close()
