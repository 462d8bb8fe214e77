"""GPU parity of the small-batch path (B * topk <= 64 slots) against the oracle.

The path is two launches: the front kernel (top-k in every block, then the
gate/up rows of the routed experts, double-buffered per wave; with the router
inside the launch in mode 2) and the down + combine kernel that requests
every routed expert's rows at once.  Mode 1 runs the router kernel first,
mode 0 the three-launch decode path, mode 3 the same three launches with the
gate/up on the matrix cores (int8 MFMA against the tokens' digit pairs).

Bars (written here):
* router indices and routing weights bit-exact against the oracle;
* block output, normwise per token: max_i |gpu - oracle| / max_i |oracle|
  <= 1e-3 (fp32 accumulate);
* modes 1 and 2 give the same bits: their token digits come from two
  different encoders (the router kernel's group encoder, the front kernel's
  8-value nibble transpose), which must agree digit for digit;
* HIP-graph replays of a mode-2 call match the eager call bit for bit (the
  router scores carry a per-call tag that a replay must advance);
* no wait for the router scores runs out of polls.
"""

import numpy as np
import pytest
import torch

from conftest import banner
from joule_amd.moe import QWEN3
from joule_amd.synth import activations
from test_gpu_parity import TOL, Layer, _rel, _run_block

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qwen64(gpu, oracle_lib):
    layer = Layer(QWEN3, 64, 2, oracle_lib)
    yield layer
    layer.store.close()


@pytest.fixture(scope="module")
def qwen32(gpu, oracle_lib):
    layer = Layer(QWEN3, 32, 1, oracle_lib)
    yield layer
    layer.store.close()


@pytest.fixture(scope="module")
def olmoe64(gpu, oracle_lib):
    from joule_amd.moe import OLMOE
    layer = Layer(OLMOE, 64, 1, oracle_lib)
    yield layer
    layer.store.close()


def _mode_block(layer, l, x, mode):
    layer.store.set_small_path(mode)
    try:
        return _run_block(layer, l, x)
    finally:
        layer.store.set_small_path(0)


def _no_timeouts(layer):
    _, timeouts = layer.store.sync_words()
    assert timeouts == 0


CASES = [("qwen64", 1), ("qwen64", 2), ("qwen64", 5), ("qwen64", 8), ("qwen32", 1), ("qwen32", 8),
         ("olmoe64", 1), ("olmoe64", 8)]


@pytest.mark.parametrize("mode", [3, 2, 1, 0])
@pytest.mark.parametrize("which,B", CASES)
def test_small_path_parity(request, which, B, mode):
    layer = request.getfixturevalue(which)
    banner(f"small path {which} B={B} mode {mode}")
    x = activations(B, layer.shape.d)
    out, top, tw = _mode_block(layer, 0, x, mode)
    rout, rtop, rtw = layer.oracle(0).forward(x)
    assert np.array_equal(top, rtop)
    assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    err = _rel(out, rout)
    print(f"  max rel err {which} B={B} mode {mode}: {err:.3e}", flush=True)
    assert err <= TOL
    _no_timeouts(layer)


@pytest.mark.parametrize("B", [8, 3])
def test_small_path_modes_same_bits(qwen64, B):
    banner(f"small path modes 1 and 2, B={B}")
    x = activations(B, QWEN3.d)
    x[0, :64] *= 1e4                         # a group of large values (its own digit scale)
    x[1 % B, 64:128] = 0.0                   # an all-zero group
    a = _mode_block(qwen64, 1, x, 1)
    b = _mode_block(qwen64, 1, x, 2)
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint8), v.view(np.uint8))
    _no_timeouts(qwen64)


def test_small_path_repeated_calls(qwen64):
    """Each mode-2 call waits for its own scores: calls alternate layers
    and tokens, so a stale score of the previous call would change the
    routing."""
    banner("small path repeated calls")
    _mode_block(qwen64, 0, activations(8, QWEN3.d), 2)
    c0, _ = qwen64.store.sync_words()
    n = 0
    for i in range(12):
        l = i % 2
        x = activations(8, QWEN3.d, seed=100 + i)
        out, top, tw = _mode_block(qwen64, l, x, 2)
        rout, rtop, rtw = qwen64.oracle(l).forward(x)
        assert np.array_equal(top, rtop), i
        assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32)), i
        assert _rel(out, rout) <= TOL, i
        n += 1
    c1, timeouts = qwen64.store.sync_words()
    assert timeouts == 0
    assert (c1 - c0) % (1 << 32) == n


def test_small_path_graph_replay(qwen64):
    """A captured mode-2 call, replayed with new token values in its input
    buffer and eager calls of another layer in between, matches the eager
    call of the same tokens bit for bit."""
    banner("small path graph replay")
    B = 8
    st = qwen64.store
    st.set_small_path(2)
    st.reserve(B)
    x_static = torch.from_numpy(activations(B, QWEN3.d, seed=7)).cuda()
    out_static = torch.empty_like(x_static)
    st.layer_ffn_batch(0, x_static, out_static)          # warm-up: per-kernel attributes set outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            st.layer_ffn_batch(0, x_static, out_static)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(5):
        xv = torch.from_numpy(activations(B, QWEN3.d, seed=200 + i)).cuda()
        st.layer_ffn_batch(1, xv)                          # eager work between the replays
        torch.cuda.synchronize()
        x_static.copy_(xv)
        g.replay()
        torch.cuda.synchronize()
        got = out_static.cpu().numpy()
        want = st.layer_ffn_batch(0, xv).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i
    _no_timeouts(qwen64)
    st.set_small_path(0)
    del g


@pytest.mark.parametrize("mode", [3, 2, 1])
def test_small_path_nan_tokens(qwen64, mode):
    banner(f"small path NaN tokens mode {mode}")
    x = activations(8, QWEN3.d)
    x[3, 100] = np.nan
    out, top, tw = _mode_block(qwen64, 0, x, mode)
    rout, rtop, rtw = qwen64.oracle(0).forward(x)
    assert np.all(top[3] == -1) and np.array_equal(top, rtop)
    assert np.array_equal(tw.view(np.uint32), rtw.view(np.uint32))
    assert np.all(out[3] == 0.0)
    keep = [b for b in range(8) if b != 3]
    assert _rel(out[keep], rout[keep]) <= TOL
    xa = np.full((2, QWEN3.d), np.nan, np.float32)
    out2, top2, _ = _mode_block(qwen64, 0, xa, mode)
    assert np.all(top2 == -1) and np.all(out2 == 0.0)
    _no_timeouts(qwen64)


def test_small_path_act_matches_dispatch_path(qwen64):
    """The front kernel's act (SiLU(gate) * up per slot, float32) against
    the three-launch path's, which tests pin to the reference's expert_job:
    both come from the same exact integer group dots."""
    banner("small path act")
    from joule_amd import _lib
    x = activations(8, QWEN3.d)
    acts = []
    for mode in (2, 0):
        _mode_block(qwen64, 0, x, mode)
        t = torch.empty((8 * QWEN3.topk, QWEN3.m), dtype=torch.float32, device="cuda")
        _lib.check(_lib.lib().jm_store_copy_workspace(qwen64.store._h, _lib.WS_ACT, _lib.ptr(t), t.numel() * 4,
                                                      _lib.stream_handle()), "copy act")
        acts.append(t.cpu().numpy())
    assert np.array_equal(acts[0].view(np.uint32), acts[1].view(np.uint32))
