"""Argument checks of the Python block wrappers (HbmExpertStore,
DenseFfnStore), reachable without a GPU: the kernels take raw pointers and
sizes, so every tensor must have exactly the shape, dtype and device the call
implies, and a mismatch must raise ValueError before any library call.  The
stores here are stand-ins built without the library (their tensors on the
CPU), so a call that passed its checks would fail at the library handle
instead of reaching a kernel."""

import pytest
import torch

from joule_amd.dense import DenseFfnStore, dense_ffn_shape
from joule_amd.moe import QWEN3, HbmExpertStore, check_tensor

D, K, M = QWEN3.d, QWEN3.topk, QWEN3.m


def test_check_tensor_cases():
    cpu = torch.device("cpu")
    good = torch.zeros((2, 8), dtype=torch.float32)
    check_tensor(good, "x", (2, 8), torch.float32, cpu)
    with pytest.raises(ValueError, match="x must be"):
        check_tensor(torch.zeros((2, 9)), "x", (2, 8), torch.float32, cpu)        # shape
    with pytest.raises(ValueError):
        check_tensor(torch.zeros((2, 8), dtype=torch.float64), "x", (2, 8), torch.float32, cpu)
    with pytest.raises(ValueError, match="not contiguous"):
        check_tensor(torch.zeros((8, 2)).t(), "x", (2, 8), torch.float32, cpu)
    with pytest.raises(ValueError):
        check_tensor(torch.zeros((2, 8), device="meta"), "x", (2, 8), torch.float32, cpu)
    with pytest.raises(ValueError, match="torch.Tensor"):
        check_tensor([[0.0] * 8] * 2, "x", (2, 8), torch.float32, cpu)


def _moe_stand_in():
    s = object.__new__(HbmExpertStore)
    s.shape = QWEN3
    s.router = object()
    s.blob = torch.empty(0, dtype=torch.uint8)
    return s


def _dense_stand_in():
    s = object.__new__(DenseFfnStore)
    s.shape = dense_ffn_shape(4096, 1024)
    s.w = (None, None, None)
    s.blob = torch.empty(0, dtype=torch.uint8)
    return s


@pytest.mark.parametrize("case", ["x_width", "x_rank", "x_dtype", "out_short", "out_width", "out_dtype",
                                  "topk_idx_shape", "topk_idx_dtype", "topk_w_shape"])
def test_moe_layer_ffn_batch_rejects(case):
    s = _moe_stand_in()
    x = torch.zeros((4, D))
    kw = {}
    if case == "x_width":
        x = torch.zeros((4, D + 1))
    elif case == "x_rank":
        x = torch.zeros(4 * D)
    elif case == "x_dtype":
        x = torch.zeros((4, D), dtype=torch.float16)
    elif case == "out_short":
        kw["out"] = torch.zeros((3, D))
    elif case == "out_width":
        kw["out"] = torch.zeros((4, D - 64))
    elif case == "out_dtype":
        kw["out"] = torch.zeros((4, D), dtype=torch.float64)
    elif case == "topk_idx_shape":
        kw["topk_idx"] = torch.zeros((4, K - 1), dtype=torch.int32)
    elif case == "topk_idx_dtype":
        kw["topk_idx"] = torch.zeros((4, K), dtype=torch.int64)
    elif case == "topk_w_shape":
        kw["topk_w"] = torch.zeros((4 * K + 1,), dtype=torch.float32)
    with pytest.raises(ValueError):
        s.layer_ffn_batch(0, x, **kw)


def test_moe_stage_wrappers_reject_shapes():
    s = _moe_stand_in()
    top = torch.zeros((4, K), dtype=torch.int32)
    with pytest.raises(ValueError):
        s.expert_gateup(0, torch.zeros((4, D + 1)), top)
    with pytest.raises(ValueError):
        s.expert_gateup(0, torch.zeros((4, D)), torch.zeros((5, K), dtype=torch.int32))
    with pytest.raises(ValueError):
        s.expert_down(0, torch.zeros((4 * K, M + 1)), top, torch.zeros((4, K)))
    with pytest.raises(ValueError):
        s.combine(torch.zeros((4 * K - 1, D)), top)


@pytest.mark.parametrize("case", ["x_width", "x_rank", "out_short", "out_dtype"])
def test_dense_layer_ffn_batch_rejects(case):
    s = _dense_stand_in()
    d = s.shape.d
    x = torch.zeros((2, d))
    kw = {}
    if case == "x_width":
        x = torch.zeros((2, d + 8))
    elif case == "x_rank":
        x = torch.zeros((2, 1, d))
    elif case == "out_short":
        kw["out"] = torch.zeros((1, d))
    elif case == "out_dtype":
        kw["out"] = torch.zeros((2, d), dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        s.layer_ffn_batch(0, x, **kw)
