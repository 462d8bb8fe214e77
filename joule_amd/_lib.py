"""ctypes binding of libjoule_amd.so (include/joule_amd.h).

Plays the role of the reference's DLL cache ``get_dll``
(src/jouleai/native/backend.py:32-42): one handle per process, loaded from
the package directory.  There is no fallback: if the library is missing the
import of anything that needs it fails with an error saying how to build it.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libjoule_amd.so"

JM_DTYPE_F32 = 0
JM_DTYPE_BF16 = 1

# Every function declared in include/joule_amd.h, with its argument types.
_c = ctypes
_vp, _i, _u64, _i64 = _c.c_void_p, _c.c_int, _c.c_uint64, _c.c_int64
SIGNATURES = {
    "jm_version": ([], _i),
    "jm_last_error": ([], _c.c_char_p),
    "jm_abi_sizes": ([_vp, _vp, _vp], _i),
    "jm_store_create": ([_vp, _i, _vp, _u64, _vp, _vp], _i),
    "jm_store_destroy": ([_vp], _i),
    "jm_store_set_router": ([_vp, _vp, _i], _i),
    "jm_store_reserve": ([_vp, _i], _i),
    "jm_store_info": ([_vp] + [_vp] * 6, _i),
    "jm_store_set_dense_min": ([_vp, _i], _i),
    "jm_store_set_act_digits": ([_vp, _i], _i),
    "jm_store_act_digits": ([_vp], _i),
    "jm_store_router_dtype": ([_vp, _vp], _i),
    "jm_layer_ffn_batch": ([_vp, _i, _vp, _i, _vp, _vp, _vp, _vp], _i),
    "jm_layer_ffn_batch_noalloc": ([_vp, _i, _vp, _i, _vp, _vp, _vp, _vp], _i),
    "jm_store_copy_workspace": ([_vp, _i, _vp, _u64, _vp], _i),
    "jm_store_profile": ([_vp, _i], _i),
    "jm_store_stage_ms": ([_vp, _vp, _i], _i),
    "jm_decode_layers_batch": ([_vp] * 6 + [_i, _vp, _vp, _vp], _i),
    "jm_store_decode_ms": ([_vp] * 4, _i),
    "jm_store_trace_topk": ([_vp, _vp, _u64], _i),
    "jm_store_set_max_layers": ([_vp, _i], _i),
    "jm_store_set_kv_dtype": ([_vp, _i], _i),
    "jm_store_set_dense_ffn": ([_vp, _vp, _vp, _vp], _i),
    "jm_store_decode_graph": ([_vp, _i], _i),
    "jm_decode_layers_batch_argmax": ([_vp] * 6 + [_i, _vp, _vp, _vp], _i),
    "jm_store_set_lm_head": ([_vp, _vp, _i, _i], _i),
    "jm_lm_head": ([_vp, _vp, _i, _vp, _vp, _vp], _i),
    "jm_embed_lookup": ([_vp, _vp, _vp, _i, _vp, _vp], _i),
    "jm_prefill_layers": ([_vp] * 5 + [_i, _vp, _vp], _i),
    "jm_router": ([_vp, _i, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp], _i),
    "jm_dispatch": ([_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "jm_expert_gateup": ([_vp, _i, _vp, _vp, _i, _vp, _vp], _i),
    "jm_expert_down": ([_vp, _i, _vp, _vp, _vp, _i, _vp, _vp], _i),
    "jm_combine": ([_vp, _vp, _vp, _i, _vp, _vp], _i),
    "jm_q4_dequant": ([_vp, _vp, _vp, _i64, _i, _vp], _i),
    "jm_expert_job": ([_vp, _vp], _i),
    "jm_q4_gemv_f32": ([_vp, _vp, _vp, _vp, _i, _i, _i, _vp], _i),
    "jm_q4_gemm_f32": ([_vp, _vp, _i, _vp, _vp, _i, _i, _i, _vp], _i),
    "jm_set_q4_gemm_min_tokens": ([_i], _i),
    "jm_get_q4_gemm_min_tokens": ([], _i),
}


class KernelCfg(ctypes.Structure):
    """The reference's KernelCfg (decode_kernel.c:269-286, decoder3.py:35-46)."""
    _fields_ = [("L", _i), ("d", _i), ("n_heads", _i), ("n_kv", _i), ("hd", _i),
                ("E", _i), ("topk", _i), ("V", _i), ("eps", _c.c_float), ("maxT", _i),
                ("intermediate", _i), ("qk_norm_type", _i), ("bias_qkv", _i),
                ("norm_topk_prob", _i), ("expert_i8", _i), ("expert_bf16", _i)]


class ExpertJob(ctypes.Structure):
    """The reference's ExpertJob (expert_ffn.c:145-157, moe.py:32-42), here
    with device pointers: jm_expert_job_t."""
    _fields_ = [("pk_g", _vp), ("sc_g", _vp), ("pk_u", _vp), ("sc_u", _vp), ("pk_d", _vp), ("sc_d", _vp),
                ("m_gg", _i), ("d_in", _i), ("m_d", _i), ("d_m", _i), ("group", _i),
                ("x", _vp), ("scratch", _vp), ("prob", _c.c_float)]


STAGES = ("route", "gateup", "down")

# jm_store_copy_workspace fields
(WS_LOGITS, WS_SEG_OFF, WS_SEG_SLOT, WS_ACTIVE, WS_N_ACTIVE, WS_FIRST_SLOT, WS_ACT, WS_Y,
 WS_N_DENSE_TILES) = range(9)


class JouleError(RuntimeError):
    """A libjoule_amd call returned a non-zero status."""


_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load libjoule_amd.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m joule_amd.build` "
                "(hipcc, gfx950). There is no CPU fallback.")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().jm_last_error().decode(errors="replace")
        raise JouleError(f"{what or 'libjoule_amd'} failed ({rc}): {msg}")


def ptr(t) -> ctypes.c_void_p:
    """Device (or host) address of a torch tensor / numpy array, None -> NULL."""
    if t is None:
        return ctypes.c_void_p(0)
    if hasattr(t, "data_ptr"):
        return ctypes.c_void_p(t.data_ptr())
    return ctypes.c_void_p(t.ctypes.data)


def stream_handle(stream=None) -> ctypes.c_void_p:
    """hipStream_t of a torch stream (default: torch's current stream)."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)
