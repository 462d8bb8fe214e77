"""ctypes front end of the C restatement (oracle/moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.  The
product path (joule_amd) never imports it.

The restated functions and the reference lines they follow are listed in the
header of moe_oracle.c.  What pins each one is recorded next to its tests.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_DIR = HERE / "_ref"

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)


def build(ref: bool | None = None) -> None:
    """Compile liboracle.so (and the reference sources when they are present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    if ref is None:
        ref = Path("/root/reference/src/jouleai/native").is_dir()
    if ref:
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


class _MoE(ctypes.Structure):
    _fields_ = [("d", ctypes.c_int), ("m", ctypes.c_int), ("E", ctypes.c_int),
                ("topk", ctypes.c_int), ("renorm", ctypes.c_int), ("group", ctypes.c_int),
                ("gate_w", ctypes.c_void_p), ("pk", ctypes.c_void_p), ("sc", ctypes.c_void_p)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build(ref=False)
        L = ctypes.CDLL(str(LIB_PATH))
        L.jmo_fp16_to_f32.restype = ctypes.c_float
        L.jmo_fp16_to_f32.argtypes = [ctypes.c_uint16]
        L.jmo_bf16_to_f32.restype = ctypes.c_float
        L.jmo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.jmo_expf_fast.restype = ctypes.c_float
        L.jmo_expf_fast.argtypes = [ctypes.c_float]
        for name in ("jmo_fp16_to_f32_array", "jmo_bf16_to_f32_array"):
            f = getattr(L, name)
            f.restype = None
            f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.jmo_expf_fast_array.restype = None
        L.jmo_expf_fast_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.jmo_router_logits.restype = None
        L.jmo_router_logits.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 3 + [ctypes.c_void_p]
        L.jmo_router_dot.restype = ctypes.c_float
        L.jmo_router_dot.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        for name in ("jmo_q4_gemv_ffn", "jmo_q4_gemv_scalar"):
            f = getattr(L, name)
            f.restype = None
            f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 3
        L.jmo_q4_gemm_ffn.restype = None
        L.jmo_q4_gemm_ffn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 3
        L.jmo_q4_row_dot_B.restype = None
        L.jmo_q4_row_dot_B.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p] + [ctypes.c_int] * 3
        L.jmo_expert_job.restype = None
        L.jmo_expert_job.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 3 + \
            [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float]
        L.jmo_q4_dequant.restype = None
        L.jmo_q4_dequant.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64, ctypes.c_int]
        L.jmo_softmax_topk.restype = None
        L.jmo_softmax_topk.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 3 + [ctypes.c_void_p] * 2
        L.jmo_layer_ffn_batch.restype = ctypes.c_int
        L.jmo_layer_ffn_batch.argtypes = [ctypes.POINTER(_MoE), ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_int, ctypes.c_int]
        L.jmo_pool_init.restype = ctypes.c_int
        L.jmo_pool_init.argtypes = [ctypes.c_int]
        L.jmo_pool_shutdown.restype = None
        L.jmo_router_dot_avx2.restype = ctypes.c_float
        L.jmo_router_dot_avx2.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        L.jmo_q4_row_dot_B_avx2.restype = None
        L.jmo_q4_row_dot_B_avx2.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p] + [ctypes.c_int] * 3
        L.jmo_set_simd.restype = None
        L.jmo_set_simd.argtypes = [ctypes.c_int]
        L.jmo_get_simd.restype = ctypes.c_int
        L.jmo_get_simd.argtypes = []
        _lib = L
    return _lib


# ---------------------------------------------------------------- scalars

def fp16_to_f32(h: int) -> float:
    return lib().jmo_fp16_to_f32(h)


def expf_fast(v: float) -> float:
    return lib().jmo_expf_fast(v)


def expf_fast_array(v: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(v, np.float32).ravel()
    out = np.empty_like(a)
    lib().jmo_expf_fast_array(_ptr(a), _ptr(out), a.size)
    return out


def fp16_to_f32_array(h: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(h, np.uint16).ravel()
    out = np.empty(a.size, np.float32)
    lib().jmo_fp16_to_f32_array(_ptr(a), _ptr(out), a.size)
    return out


def bf16_to_f32_array(h: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(h, np.uint16).ravel()
    out = np.empty(a.size, np.float32)
    lib().jmo_bf16_to_f32_array(_ptr(a), _ptr(out), a.size)
    return out


def router_dot(w: np.ndarray, x: np.ndarray) -> float:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    return lib().jmo_router_dot(_ptr(w), _ptr(x), w.size)


def router_dot_avx2(w: np.ndarray, x: np.ndarray) -> float:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    return lib().jmo_router_dot_avx2(_ptr(w), _ptr(x), w.size)


def set_simd(on: bool) -> None:
    """Which form of the router and Q4 row dots the block (OracleMoE.forward)
    runs, process-wide: the AVX2 form (the same bits, the timed CPU
    baseline) or the scalar statement (the default)."""
    lib().jmo_set_simd(int(bool(on)))


def get_simd() -> bool:
    return bool(lib().jmo_get_simd())


def router_logits(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    E, d = w.shape
    B = x.shape[0]
    out = np.empty((B, E), np.float32)
    lib().jmo_router_logits(_ptr(w), _ptr(x), B, E, d, _ptr(out))
    return out


def route(w: np.ndarray, x: np.ndarray, topk: int, renorm: bool):
    """(logits, top, tw) of the reference router for a batch."""
    logits = router_logits(w, x)
    B = x.shape[0]
    top = np.empty((B, topk), np.int32)
    tw = np.empty((B, topk), np.float32)
    for b in range(B):
        _, top[b], tw[b] = softmax_topk(logits[b], topk, renorm)
    return logits, top, tw


# ------------------------------------------------------------- Q4 kernels

def q4_gemv_ffn(x, packed, scales, m, d, group=64) -> np.ndarray:
    out = np.empty(m, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lib().jmo_q4_gemv_ffn(_ptr(out), _ptr(x), _ptr(packed), _ptr(scales), m, d, group)
    return out


def q4_gemm_ffn(X, packed, scales, m, d, group=64) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    T = X.shape[0]
    out = np.empty((T, m), np.float32)
    lib().jmo_q4_gemm_ffn(_ptr(out), _ptr(X), T, _ptr(packed), _ptr(scales), m, d, group)
    return out


def q4_gemv_scalar(x, packed, scales, m, d, group=64) -> np.ndarray:
    out = np.empty(m, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lib().jmo_q4_gemv_scalar(_ptr(out), _ptr(x), _ptr(packed), _ptr(scales), m, d, group)
    return out


def q4_row_dot_B(row, sc, X, cols, group=64) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    B = X.shape[0]
    acc = np.empty(B, np.float32)
    lib().jmo_q4_row_dot_B(_ptr(row), _ptr(sc), _ptr(X), B, _ptr(acc), cols, group, X.shape[1])
    return acc


def q4_row_dot_B_avx2(row, sc, X, cols, group=64) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    B = X.shape[0]
    acc = np.empty(B, np.float32)
    lib().jmo_q4_row_dot_B_avx2(_ptr(row), _ptr(sc), _ptr(X), B, _ptr(acc), cols, group, X.shape[1])
    return acc


def expert_job(rec_g, rec_u, rec_d, m, d, group, x, prob) -> np.ndarray:
    """rec_* = (scales u16, packed u8).  Returns scratch [m + d]."""
    x = np.ascontiguousarray(x, np.float32)
    scratch = np.zeros(m + d, np.float32)
    lib().jmo_expert_job(_ptr(rec_g[1]), _ptr(rec_g[0]), _ptr(rec_u[1]), _ptr(rec_u[0]),
                         _ptr(rec_d[1]), _ptr(rec_d[0]), m, d, group, _ptr(x), _ptr(scratch),
                         float(prob))
    return scratch


def q4_dequant(packed, scales, numel, group=64) -> np.ndarray:
    out = np.empty(numel, np.float32)
    lib().jmo_q4_dequant(_ptr(out), _ptr(packed), _ptr(scales), numel, group)
    return out


def softmax_topk(scores: np.ndarray, topk: int, renorm: bool):
    """Returns (probs, top int32, tw float32) for one token's router scores."""
    p = np.array(scores, np.float32, copy=True)
    top = np.empty(topk, np.int32)
    tw = np.empty(topk, np.float32)
    lib().jmo_softmax_topk(_ptr(p), p.size, topk, int(bool(renorm)), _ptr(top), _ptr(tw))
    return p, top, tw


# ------------------------------------------------------------ MoE block

class OracleMoE:
    """layer_ffn_batch restated on the CPU for one layer of a Q4 store.

    ``blob`` is the store bytes (uint8), ``offsets`` the [3, E, 2] table of
    (scales offset, packed offset) for this layer, ``gate_w`` the [E, d]
    router weights (bf16 values held as float32).
    """

    def __init__(self, d, m, E, topk, renorm, group, gate_w, blob, offsets):
        self.d, self.m, self.E, self.topk = d, m, E, topk
        self.renorm, self.group = bool(renorm), group
        self.gate_w = np.ascontiguousarray(gate_w, np.float32)
        assert self.gate_w.shape == (E, d)
        self.blob = blob
        base = blob.ctypes.data
        offs = np.asarray(offsets, np.uint64).reshape(3, E, 2)
        self._pk = (ctypes.c_void_p * (3 * E))(*[base + int(offs[p, e, 1]) for p in range(3) for e in range(E)])
        self._sc = (ctypes.c_void_p * (3 * E))(*[base + int(offs[p, e, 0]) for p in range(3) for e in range(E)])
        self._cfg = _MoE(d, m, E, topk, int(self.renorm), group,
                         self.gate_w.ctypes.data,
                         ctypes.cast(self._pk, ctypes.c_void_p).value,
                         ctypes.cast(self._sc, ctypes.c_void_p).value)

    def forward(self, x: np.ndarray, n_threads: int = 1, all_tokens: bool = False):
        x = np.ascontiguousarray(x, np.float32)
        B = x.shape[0]
        out = np.empty((B, self.d), np.float32)
        top = np.empty((B, self.topk), np.int32)
        tw = np.empty((B, self.topk), np.float32)
        rc = lib().jmo_layer_ffn_batch(ctypes.byref(self._cfg), _ptr(x), B, _ptr(out), _ptr(top),
                                       _ptr(tw), int(n_threads), int(bool(all_tokens)))
        if rc != 0:
            raise RuntimeError(f"oracle layer_ffn_batch failed with code {rc}")
        return out, top, tw


# ----------------------------------------------------- reference library

def ref_lib(name: str) -> ctypes.CDLL | None:
    """The reference's own source compiled into oracle/_ref (None if absent)."""
    p = REF_DIR / f"libref_{name}.so"
    if not p.exists():
        return None
    L = ctypes.CDLL(str(p))
    L.q4_gemv_f32.restype = None
    L.q4_gemv_f32.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 3
    if name == "expert_ffn":
        L.q4_gemm_f32.restype = None
        L.q4_gemm_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                  ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 3
        L.expert_job.restype = None
        L.expert_job.argtypes = [ctypes.c_void_p]
    return L


class RefExpertJob(ctypes.Structure):
    """Layout of ExpertJob (expert_ffn.c:145-157) for calling the reference build."""
    _fields_ = [("pk_g", ctypes.c_void_p), ("sc_g", ctypes.c_void_p),
                ("pk_u", ctypes.c_void_p), ("sc_u", ctypes.c_void_p),
                ("pk_d", ctypes.c_void_p), ("sc_d", ctypes.c_void_p),
                ("m_gg", ctypes.c_int), ("d_in", ctypes.c_int),
                ("m_d", ctypes.c_int), ("d_m", ctypes.c_int),
                ("group", ctypes.c_int),
                ("x", ctypes.c_void_p), ("scratch", ctypes.c_void_p),
                ("prob", ctypes.c_float)]


def cpu_count() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
