"""A dense model's FFN on the GPU: the store of a model without experts.

The reference's ``layer_ffn_batch`` takes its E == 0 branch for dense
families (qwen2, qwen3, llama, mistral; src/jouleai/native/
decode_kernel.c:1393-1422, weights loaded by decoder3.py:251-280):
``silu(x W1^T) * (x W2^T)``, then ``W3``, bf16 weights shared by the batch.
``DenseFfnStore`` is the handle the decoder (``HipDecoder``) runs such a
model on: a library store created with E = 0.  The decoder passes the FFN
weights with its ``KernelW`` (w1, w2, w3); ``layer_ffn_batch`` uses the
ones given to ``set_weights``.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .moe import MoEShape, check_tensor


def dense_ffn_shape(d: int, m: int) -> MoEShape:
    """The FFN shape of a dense model (E = 0, no top-k), as DecoderShape.moe."""
    return MoEShape(d=d, m=m, E=0, topk=0, renorm=False, name="dense")


class DenseFfnStore:
    """A store with no experts (E = 0) for an n_layers-layer dense model
    of hidden d and intermediate m."""

    def __init__(self, d: int, m: int, n_layers: int, device="cuda"):
        self.shape = dense_ffn_shape(d, m)
        self.n_layers = n_layers
        self.group = 0
        self._cfg = self.shape.kernel_cfg(n_layers)
        # the device the store lives on (the decoder reads store.blob.device)
        self.blob = torch.empty(0, dtype=torch.uint8, device=device)
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.blob.device):
            _lib.check(_lib.lib().jm_store_create(ctypes.byref(self._cfg), 0, None, 0, None, ctypes.byref(handle)),
                       "jm_store_create")
        self._h = handle
        self.w: tuple | None = None

    def set_weights(self, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor) -> None:
        """w1, w2 [L, m, d] (gate_proj, up_proj) and w3 [L, d, m] (down_proj),
        bf16 CUDA tensors, for ``layer_ffn_batch``."""
        L, d, m = self.n_layers, self.shape.d, self.shape.m
        for t, shp, name in ((w1, (L, m, d), "w1"), (w2, (L, m, d), "w2"), (w3, (L, d, m), "w3")):
            if t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous() or tuple(t.shape) != shp:
                raise ValueError(f"{name} must be a contiguous bfloat16 CUDA tensor {list(shp)}")
        _lib.check(_lib.lib().jm_store_set_dense_ffn(self._h, _lib.ptr(w1), _lib.ptr(w2), _lib.ptr(w3)),
                   "jm_store_set_dense_ffn")
        self.w = (w1, w2, w3)

    def layer_ffn_batch(self, l: int, x: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """out [B, d] = the dense FFN of layer l on x [B, d] (float32, CUDA)."""
        if self.w is None:
            raise RuntimeError("FFN weights not set (set_weights)")
        d = self.shape.d
        B = x.shape[0] if isinstance(x, torch.Tensor) and x.dim() == 2 else -1
        check_tensor(x, "x", (B, d), torch.float32, self.blob.device)
        if out is None:
            out = torch.empty_like(x)
        else:
            check_tensor(out, "out", (B, d), torch.float32, self.blob.device)
        _lib.check(_lib.lib().jm_layer_ffn_batch(self._h, int(l), _lib.ptr(x), x.shape[0], _lib.ptr(out), None, None,
                                                 _lib.stream_handle(stream)), "jm_layer_ffn_batch")
        return out

    def reserve(self, max_B: int) -> None:
        _lib.check(_lib.lib().jm_store_reserve(self._h, int(max_B)), "jm_store_reserve")

    def profile(self, enable: bool = True) -> None:
        _lib.check(_lib.lib().jm_store_profile(self._h, int(bool(enable))), "jm_store_profile")

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.lib().jm_store_destroy(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover - best effort at interpreter exit
        try:
            self.close()
        except Exception:
            pass
