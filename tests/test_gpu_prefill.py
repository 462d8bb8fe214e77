"""Multi-position prefill (jm_prefill_layers, HipNativeDecoder.prefill_batch)
against the reference's semantics: decode_layers_batch once per position
(decode_kernel.c:1606-1615, decoder3.py:512-571), restated by the oracle.
Checks the last position's logits (1e-3) and every cache row written."""

import numpy as np
import pytest
import torch

from joule_amd.decoder import DecoderShape, DecoderWeights, HipDecoder, KVCacheSet
from joule_amd.moe import HbmExpertStore, MoEShape
from joule_amd.synth import decoder_weights, fill_kv, router_weights, torch_store
from oracle import decoder as D
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _model(L, maxT, B, V=3000, seed=41, moe=None, group=64, qk=1, kv_dtype=torch.bfloat16):
    moe = moe or MoEShape(d=2048, m=768, E=128, topk=8, renorm=True)
    shape = DecoderShape(n_layers=L, moe=moe, n_heads=16, n_kv=4, maxT=maxT, V=V, qk_norm_type=qk)
    blob, offsets = torch_store(moe, L, group)
    store = HbmExpertStore(moe, L, blob, offsets, group)
    gw = np.stack([router_weights(moe, l) for l in range(L)])
    store.set_router(torch.from_numpy(gw).cuda())
    t = decoder_weights(shape, norm_jitter=0.1)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    t["embed"] = (torch.randn((V, 2048), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    lm = (torch.randn((V, 2048), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    dec = HipDecoder(store, DecoderWeights(shape, **t))
    dec.set_lm_head(lm)
    kv = KVCacheSet(shape, B, dtype=kv_dtype)
    fill_kv(kv.data)                       # rows past the prompt hold noise: never read
    torch.cuda.synchronize()
    w = {k: v.float().cpu().numpy() for k, v in dec.weights.t.items()}
    blob_h = blob.cpu().numpy()
    E = moe.E
    moe_o = [O.OracleMoE(2048, moe.m, E, moe.topk, moe.renorm, group, gw[l], blob_h, offsets[:, l * E:(l + 1) * E])
             for l in range(L)]
    oracle = D.OracleDecoder(L, 2048, 16, 4, 128, shape.eps, qk, False, w, moe_o, kv_bf16=kv_dtype == torch.bfloat16)
    return dec, oracle, kv, w, lm.float().cpu().numpy()


def _oracle_prefill(oracle, w, W_lm, prompt, kv_seq):
    """The reference's loop: one decode_layers_batch per position."""
    hid = None
    for t, tok in enumerate(prompt):
        x = D.embed_lookup(w["embed"], [tok])
        hid = oracle.decode_layers_batch(x, [t], [kv_seq])
    return D.lm_head(W_lm, hid)[0]


def _check_rows(kv, b, kv_seq, T, L, label):
    for l in range(L):
        for j in (0, 1):
            g = kv.data[b, l, j, :T].float().cpu().numpy()
            r = kv_seq[l][j][:T]
            unit = 0.0 if kv.data.dtype == torch.float32 else 2.0 ** -7     # one bf16 unit for bf16 caches
            lim = np.abs(r) * unit + 1e-4 * np.abs(r).max(axis=-1, keepdims=True)
            bad = int((np.abs(g - r) > lim).sum())
            assert bad == 0, f"{label}: layer {l} {'kv'[j]}: {bad} cache values off by more than the bound"


@pytest.mark.parametrize("L,T,kv_dtype", [(2, 200, torch.bfloat16), (1, 600, torch.bfloat16), (1, 77, torch.bfloat16),
                                          (1, 300, torch.float32)])
def test_prefill_layers_matches_per_position_decode(L, T, kv_dtype):
    dec, oracle, kv, w, W_lm = _model(L, maxT=640, B=1, kv_dtype=kv_dtype)
    rng = np.random.default_rng(T)
    prompt = rng.integers(0, 3000, size=T).tolist()
    kv_seq = [(kv.data[0, l, 0].float().cpu().numpy(), kv.data[0, l, 1].float().cpu().numpy()) for l in range(L)]
    print(f"[prefill] L={L} T={T}", flush=True)
    logits = torch.empty(3000, dtype=torch.float32, device="cuda")
    dec.prefill_layers(torch.tensor(prompt, dtype=torch.int32, device="cuda"), kv, 0, logits)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    want = _oracle_prefill(oracle, w, W_lm, prompt, kv_seq)
    rel = np.abs(got - want).max() / np.abs(want).max()
    print(f"  prefill L={L} T={T}: last-position logits max rel err {rel:.2e}", flush=True)
    assert rel < TOL, rel
    _check_rows(kv, 0, kv_seq, T, L, f"T={T}")
    dec.store.close()


@pytest.mark.parametrize("moe,group,qk", [(MoEShape(d=2048, m=1024, E=64, topk=8, renorm=False), 64, 2),
                                          (MoEShape(d=2048, m=768, E=128, topk=8, renorm=True), 32, 1)],
                         ids=["olmoe-g64", "qwen3-g32"])
def test_prefill_moe_variants(moe, group, qk):
    """The prefill with the other MoE shape (64 experts, m = 1024, no
    renormalisation, OLMoE's whole-vector QK-norm) and with Q4 group 32: the
    dispatch path, both MFMA tile shapes and the small-expert kernels at
    other sizes."""
    T = 150
    dec, oracle, kv, w, W_lm = _model(1, maxT=256, B=1, moe=moe, group=group, qk=qk)
    rng = np.random.default_rng(T + group)
    prompt = rng.integers(0, 3000, size=T).tolist()
    kv_seq = [(kv.data[0, 0, 0].float().cpu().numpy(), kv.data[0, 0, 1].float().cpu().numpy())]
    print(f"[prefill] E={moe.E} m={moe.m} G{group} T={T}", flush=True)
    logits = torch.empty(3000, dtype=torch.float32, device="cuda")
    dec.prefill_layers(torch.tensor(prompt, dtype=torch.int32, device="cuda"), kv, 0, logits)
    torch.cuda.synchronize()
    want = _oracle_prefill(oracle, w, W_lm, prompt, kv_seq)
    rel = np.abs(logits.cpu().numpy() - want).max() / np.abs(want).max()
    print(f"  prefill E={moe.E} G{group}: last-position logits max rel err {rel:.2e}", flush=True)
    assert rel < TOL, rel
    _check_rows(kv, 0, kv_seq, T, 1, f"E={moe.E} G{group}")
    dec.store.close()


def test_prefill_batch_prompts_of_different_lengths():
    from joule_amd.checkpoint import HipNativeDecoder

    dec, oracle, kv, w, W_lm = _model(2, maxT=256, B=3)
    nd = HipNativeDecoder.__new__(HipNativeDecoder)      # the host object around an existing decoder
    nd.dec, nd.shape, nd.kv, nd._seq_pos = dec, dec.shape, kv, {}
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 3000, size=n).tolist() for n in (5, 130, 64)]
    kv_o = [[(kv.data[b, l, 0].float().cpu().numpy(), kv.data[b, l, 1].float().cpu().numpy()) for l in range(2)]
            for b in range(3)]
    print("[prefill] batch of 3 prompts", flush=True)
    outs = nd.prefill_batch(prompts, chunk=96)           # chunks that split prompts
    for b, p in enumerate(prompts):
        want = _oracle_prefill(oracle, w, W_lm, p, kv_o[b])
        rel = np.abs(outs[b] - want).max() / np.abs(want).max()
        assert rel < TOL, (b, rel)
        _check_rows(kv, b, kv_o[b], len(p), 2, f"prompt {b}")
    assert nd._seq_pos == {"seq0": 5, "seq1": 130, "seq2": 64}
    # decode continues from the prefilled caches
    tok = nd.decode_batch_argmax([int(np.argmax(o)) for o in outs], [5, 130, 64])
    assert len(tok) == 3 and all(0 <= t < 3000 for t in tok)
    dec.store.close()
