"""jm_layer_ffn_batch_noalloc (the workspace in the library's fixed device
array) against jm_layer_ffn_batch (the store's own workspace), through the
C ABI: router indices, routing weights and block outputs bit-identical, on
two calls in a row, the second with fewer tokens (the array then holds the
first call's contents); a batch whose workspace exceeds the array is refused
before anything runs."""

import ctypes

import numpy as np
import pytest
import torch

from conftest import banner
from joule_amd import _lib
from joule_amd.moe import QWEN3, HbmExpertStore
from joule_amd.synth import activations, router_weights, torch_store

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def store(gpu):
    blob, offsets = torch_store(QWEN3, 2, 64)
    st = HbmExpertStore(QWEN3, 2, blob, offsets, 64)
    st.set_router(torch.from_numpy(np.stack([router_weights(QWEN3, l) for l in range(2)])).cuda())
    yield st
    st.close()


def _call(fn, st, layer, x):
    B = x.shape[0]
    out = torch.full_like(x, float("nan"))
    top = torch.full((B, QWEN3.topk), -7, dtype=torch.int32, device="cuda")
    tw = torch.full((B, QWEN3.topk), float("nan"), dtype=torch.float32, device="cuda")
    _lib.check(fn(st._h, layer, _lib.ptr(x), B, _lib.ptr(out), _lib.ptr(top), _lib.ptr(tw),
                  _lib.stream_handle()), fn.__name__)
    torch.cuda.synchronize()
    return out.cpu().numpy(), top.cpu().numpy(), tw.cpu().numpy()


@pytest.mark.parametrize("sizes", [(64, 8), (40, 1)])
def test_noalloc_matches_allocating_entry_point(store, sizes):
    L = _lib.lib()
    for i, B in enumerate(sizes):
        layer = i % 2
        banner(f"no-allocation block: call {i + 1}, B={B}, layer {layer}")
        x = torch.from_numpy(activations(B, QWEN3.d, seed=4100 + B)).cuda()
        want = _call(L.jm_layer_ffn_batch, store, layer, x)
        got = _call(L.jm_layer_ffn_batch_noalloc, store, layer, x)
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint8), w.view(np.uint8)), (B, layer)
        assert np.isfinite(got[0]).all()


def test_noalloc_refuses_batches_beyond_its_workspace(store):
    banner("no-allocation block: oversized batch refused")
    L = _lib.lib()
    B = 512                                   # ~70 MB of workspace for the Qwen3 block
    x = torch.zeros((B, QWEN3.d), dtype=torch.float32, device="cuda")
    out = torch.zeros_like(x)
    rc = L.jm_layer_ffn_batch_noalloc(store._h, 0, _lib.ptr(x), B, _lib.ptr(out), None, None, _lib.stream_handle())
    assert rc == -2 and b"workspace" in L.jm_last_error()
    rc = L.jm_layer_ffn_batch_noalloc(store._h, 0, _lib.ptr(x), 0, _lib.ptr(out), None, None, _lib.stream_handle())
    assert rc == 0
    # the refused call left the array usable
    x8 = torch.from_numpy(activations(8, QWEN3.d)).cuda()
    want = _call(L.jm_layer_ffn_batch, store, 0, x8)
    got = _call(L.jm_layer_ffn_batch_noalloc, store, 0, x8)
    assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
