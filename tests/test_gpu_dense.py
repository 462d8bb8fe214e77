"""GPU parity of the dense FFN (layer_ffn_batch's E == 0 branch,
decode_kernel.c:1393-1422) with the oracle (oracle/decoder.py dense_ffn):
the block entry point on a dense store, the decode step of a dense model
(decode_layers_batch, graph replays included) and its prefill.  Batches up
to 32 tokens take the split-K projections, from 33 the GEMM."""

import ctypes

import numpy as np
import pytest
import torch

from joule_amd import _lib
from joule_amd.decoder import DecoderShape, DecoderWeights, HipDecoder, KVCacheSet
from joule_amd.dense import DenseFfnStore, dense_ffn_shape
from joule_amd.synth import activations, decoder_weights, fill_kv
from oracle import decoder as D

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _rel(got, want):
    return (np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)).max()


@pytest.mark.parametrize("d,m,B", [(1024, 3072, 1), (2048, 5632, 8), (1024, 3072, 40), (4096, 4096, 3)])
def test_dense_block_matches_oracle(d, m, B):
    """jm_layer_ffn_batch on a dense store: intermediate sizes that are a
    multiple of 1024 and ones that are only a multiple of 512 (512-column
    slices of the down projection), the GEMM from 33 tokens."""
    L = 2
    print(f"[dense] block d={d} m={m} B={B}", flush=True)
    store = DenseFfnStore(d, m, L)
    g = torch.Generator(device="cuda")
    g.manual_seed(d + m)
    w1, w2 = ((torch.randn((L, m, d), generator=g, device="cuda") * 0.03).to(torch.bfloat16) for _ in range(2))
    w3 = (torch.randn((L, d, m), generator=g, device="cuda") * 0.03).to(torch.bfloat16)
    store.set_weights(w1, w2, w3)
    x = torch.from_numpy(activations(B, d)).cuda()
    for l in range(L):
        out = store.layer_ffn_batch(l, x)
        torch.cuda.synchronize()
        want = D.dense_ffn(x.cpu().numpy(), w1[l].float().cpu().numpy(), w2[l].float().cpu().numpy(),
                           w3[l].float().cpu().numpy())
        rel = _rel(out.cpu().numpy(), want)
        print(f"  layer {l}: max rel err {rel:.2e}", flush=True)
        assert rel <= TOL
    store.close()


def test_dense_store_refuses_expert_entry_points():
    store = DenseFfnStore(1024, 1024, 1)
    L = _lib.lib()
    gw = torch.zeros((1, 8, 1024), dtype=torch.bfloat16, device="cuda")
    assert L.jm_store_set_router(store._h, _lib.ptr(gw), _lib.JM_DTYPE_BF16) != 0
    assert b"dense store" in L.jm_last_error()
    x = torch.zeros((2, 1024), device="cuda")
    assert L.jm_layer_ffn_batch(store._h, 0, _lib.ptr(x), 2, _lib.ptr(x), None, None, None) != 0
    assert b"not set" in L.jm_last_error()          # no weights registered yet
    top = torch.zeros(2, dtype=torch.int32, device="cuda")
    store.set_weights(*(torch.zeros(s, dtype=torch.bfloat16, device="cuda")
                        for s in ((1, 1024, 1024), (1, 1024, 1024), (1, 1024, 1024))))
    assert L.jm_layer_ffn_batch(store._h, 0, _lib.ptr(x), 2, _lib.ptr(x), _lib.ptr(top), None, None) != 0
    assert b"top-k" in L.jm_last_error()
    store.close()


def _dense_model(L, d, m, H, KH, maxT, B, qk=1, bias=False, V=0):
    shape = DecoderShape(n_layers=L, moe=dense_ffn_shape(d, m), n_heads=H, n_kv=KH, maxT=maxT,
                         qk_norm_type=qk, bias_qkv=bias, V=V)
    store = DenseFfnStore(d, m, L)
    t = decoder_weights(shape, norm_jitter=0.1)
    weights = DecoderWeights(shape, **t)
    kv = KVCacheSet(shape, B)
    fill_kv(kv.data)
    torch.cuda.synchronize()
    w = {k: v.float().cpu().numpy() for k, v in weights.t.items()}
    oracle = D.OracleDecoder(L, d, H, KH, 128, shape.eps, qk, bias, w, None)
    return HipDecoder(store, weights), oracle, kv


CASES = {
    # Qwen3-dense-like layers (GQA 8/2, per-head QK-norm), m a multiple of 512 only
    "qwen3ish_l2_b4": (dict(L=2, d=1024, m=3072, H=8, KH=2, maxT=300, qk=1), [0, 5, 130, 299]),
    # Llama-like: no QK-norm, MHA, m = 5632 (11 slices of 512)
    "llamaish_l1_b3": (dict(L=1, d=2048, m=5632, H=16, KH=16, maxT=200), [7, 128, 199]),
    # qwen2-like: QKV bias
    "qwen2ish_l1_b2": (dict(L=1, d=1024, m=2048, H=8, KH=4, maxT=150, qk=0, bias=True), [3, 149]),
}


@pytest.mark.parametrize("case", list(CASES))
def test_dense_decode_matches_oracle(case):
    cfg, positions = CASES[case]
    B = len(positions)
    dec, oracle, kv = _dense_model(B=B, **cfg)
    kv_h = [[(kv.data[b, l, 0].float().cpu().numpy(), kv.data[b, l, 1].float().cpu().numpy())
             for l in range(cfg["L"])] for b in range(B)]
    for step in range(2):
        pos = [min(p + step, cfg["maxT"] - 1) for p in positions]
        x = activations(B, cfg["d"], seed=3000 + step)
        print(f"[dense] decode {case} step {step} positions {pos}", flush=True)
        hid = dec.decode_layers_batch(torch.from_numpy(x).cuda(), pos, kv)
        torch.cuda.synchronize()
        want = oracle.decode_layers_batch(x, pos, kv_h)
        rel = _rel(hid.cpu().numpy(), want)
        print(f"  max rel err {rel:.2e}", flush=True)
        assert rel <= TOL
    dec.store.close()


def test_dense_decode_graph_replays_match_eager():
    dec, _, kv = _dense_model(L=2, d=1024, m=3072, H=8, KH=2, maxT=300, B=4)
    x = torch.from_numpy(activations(4, 1024)).cuda()
    pos = [10, 130, 257, 299]
    dec.set_graph(False)
    want = dec.decode_layers_batch(x, pos, kv, torch.empty_like(x)).clone()
    torch.cuda.synchronize()
    dec.set_graph(True)
    hid = torch.empty_like(x)
    for i in range(3):
        got = dec.decode_layers_batch(x, pos, kv, hid)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i} differs from the eager step"
        assert float((x * 2).abs().sum().item()) > 0
    dec.store.close()


def test_dense_prefill_matches_per_position_decode():
    """A 100-token prompt through 2 dense layers (the GEMM projections and
    FFN) against the reference's loop of one decode step per position."""
    L, d, m, V, T = 2, 1024, 3072, 2000, 100
    dec, oracle, kv = _dense_model(L=L, d=d, m=m, H=8, KH=2, maxT=128, B=1, V=V)
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    emb = (torch.randn((V, d), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    lm = (torch.randn((V, d), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    dec.weights.t["embed"] = emb
    dec._w = dec.weights.kernel_w()
    dec.set_lm_head(lm)
    prompt = np.random.default_rng(5).integers(0, V, size=T).tolist()
    kv_seq = [(kv.data[0, l, 0].float().cpu().numpy(), kv.data[0, l, 1].float().cpu().numpy()) for l in range(L)]
    print(f"[dense] prefill T={T}", flush=True)
    logits = torch.empty(V, dtype=torch.float32, device="cuda")
    dec.prefill_layers(torch.tensor(prompt, dtype=torch.int32, device="cuda"), kv, 0, logits)
    torch.cuda.synchronize()
    E = emb.float().cpu().numpy()
    hid = None
    for t, tok in enumerate(prompt):
        hid = oracle.decode_layers_batch(D.embed_lookup(E, [tok]), [t], [kv_seq])
    want = D.lm_head(lm.float().cpu().numpy(), hid)[0]
    rel = np.abs(logits.cpu().numpy() - want).max() / np.abs(want).max()
    print(f"  last-position logits max rel err {rel:.2e}", flush=True)
    assert rel < TOL
    dec.store.close()
