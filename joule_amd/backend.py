"""KernelBackend plugin API with a HIP (gfx950) implementation.

Mirrors the reference's ``KernelBackend`` (src/jouleai/native/backend.py:45-69):
a backend exposes ``q4_gemv`` and ``q4_gemm`` with the same argument order,
and ``KernelBackend.auto()`` returns the best available backend.  Adding the
GPU is "a new KernelBackend subclass, no caller changes" (backend.py:3-8).

``HipBackend`` computes on the GPU.  ``packed``/``scales`` may be CUDA
tensors (the HBM store's views from ``HbmExpertStore.ensure``) or numpy
arrays, which are uploaded for the call.  Results are float32 CUDA tensors.
There is no CPU fallback: without the HIP library ``auto()`` raises.
"""

from __future__ import annotations

from abc import ABC, abstractmethod

import numpy as np
import torch

from . import _lib


class KernelBackend(ABC):
    """Interface every kernel backend implements (backend.py:45-69)."""

    name: str = "base"

    @abstractmethod
    def q4_gemv(self, x_f32: torch.Tensor, packed, scales, m: int, d: int,
                group: int = 64) -> torch.Tensor:
        """out[m] = dequant_q4(packed, scales) @ x[d] (no dequant materialised)."""

    @abstractmethod
    def q4_gemm(self, out_f32: torch.Tensor, X_f32: torch.Tensor, packed, scales,
                m: int, d: int, group: int = 64) -> None:
        """out[T, m] (in place) = X[T, d] @ dequant(W)^T."""

    @staticmethod
    def auto() -> "KernelBackend":
        """Best available backend: the HIP backend (the only one here)."""
        return HipBackend()


def _dev(a, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        t = a if a.device == device else a.to(device)
    else:
        t = torch.from_numpy(np.ascontiguousarray(a)).to(device)
    if t.dtype != dtype:
        t = t.view(dtype) if t.element_size() == torch.empty((), dtype=dtype).element_size() else t.to(dtype)
    return t.contiguous()


class HipBackend(KernelBackend):
    """Fused Q4 GEMV/GEMM on the GPU (libjoule_amd.so)."""

    name = "hip"

    def __init__(self, device: str | torch.device | None = None):
        if not torch.cuda.is_available():
            raise RuntimeError("HipBackend needs a ROCm GPU")
        self.lib = _lib.lib()
        self.device = torch.device(device or "cuda")

    def q4_gemv(self, x_f32, packed, scales, m, d, group=64):
        x = _dev(x_f32, torch.float32, self.device)
        if x.numel() != d:
            raise ValueError(f"x has {x.numel()} elements, expected d={d}")
        pk = _dev(packed, torch.uint8, self.device)
        sc = _dev(scales, torch.int16, self.device)
        if pk.numel() != m * d // 2:
            raise ValueError("packed size does not match m * d / 2")
        out = torch.empty(m, dtype=torch.float32, device=self.device)
        _lib.check(self.lib.jm_q4_gemv_f32(_lib.ptr(out), _lib.ptr(x), _lib.ptr(pk), _lib.ptr(sc),
                                           m, d, group, _lib.stream_handle()), "jm_q4_gemv_f32")
        return out

    def q4_gemm(self, out_f32, X_f32, packed, scales, m, d, group=64):
        X = _dev(X_f32, torch.float32, self.device)
        T = X.shape[0]
        if X.numel() != T * d:
            raise ValueError("X must be [T, d]")
        if not (out_f32.is_cuda and out_f32.dtype == torch.float32 and out_f32.is_contiguous()
                and out_f32.numel() == T * m):
            raise ValueError("out must be a contiguous float32 CUDA tensor [T, m]")
        pk = _dev(packed, torch.uint8, self.device)
        sc = _dev(scales, torch.int16, self.device)
        _lib.check(self.lib.jm_q4_gemm_f32(_lib.ptr(out_f32), _lib.ptr(X), T, _lib.ptr(pk), _lib.ptr(sc),
                                           m, d, group, _lib.stream_handle()), "jm_q4_gemm_f32")


def q4_dequant(packed: torch.Tensor, scales: torch.Tensor, numel: int, group: int = 64) -> torch.Tensor:
    """Exact float32 dequantisation of one record on the GPU."""
    out = torch.empty(numel, dtype=torch.float32, device=packed.device)
    _lib.check(_lib.lib().jm_q4_dequant(_lib.ptr(out), _lib.ptr(packed), _lib.ptr(scales), numel, group,
                                        _lib.stream_handle()), "jm_q4_dequant")
    return out
