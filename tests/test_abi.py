"""The C ABI library loads and exports what include/joule_amd.h declares.

CPU-only: no call here launches GPU work.  Argument and shape errors are
checked before any HIP call, so they are exercised here as well.
"""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from joule_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "joule_amd.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jm_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_header_symbols():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libjoule_amd.so not built (run python -m joule_amd.build)")
    syms = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                          text=True, check=True).stdout
    exported = set(re.findall(r"\bT (jm_[a-z0-9_]+)", syms))
    declared = _declared()
    assert declared, "no declarations parsed"
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    # the ctypes table covers every declared function
    assert set(declared) == set(_lib.SIGNATURES)
    L = _lib.lib()
    for name in declared:
        assert hasattr(L, name)


def test_probe_library_exports_header_symbols():
    """libjoule_probe.so (bench.py --probe) exports what joule_probe.h declares."""
    from joule_amd.build import PROBE_OUT

    if not PROBE_OUT.exists():
        pytest.skip("libjoule_probe.so not built (run python -m joule_amd.build)")
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "joule_probe.h").read_text(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(jmp_[a-z0-9_]+)\s*\(", text)))
    assert declared == ["jmp_handoff", "jmp_last_error", "jmp_launch_chain", "jmp_stream"]
    syms = subprocess.run(["nm", "-D", "--defined-only", str(PROBE_OUT)], capture_output=True,
                          text=True, check=True).stdout
    exported = set(re.findall(r"\bT (jmp_[a-z0-9_]+)", syms))
    assert set(declared) <= exported
    P = ctypes.CDLL(str(PROBE_OUT))
    f = ctypes.c_float()
    assert P.jmp_launch_chain(0, 0, 1, ctypes.byref(f)) == -1      # argument check, no GPU work
    assert P.jmp_handoff(0, 1, 0, 1, ctypes.byref(f), None) == -1
    P.jmp_stream.argtypes = [ctypes.c_ulonglong, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                             ctypes.POINTER(ctypes.c_float)]
    assert P.jmp_stream(1000, 16384, 1, 1, ctypes.byref(f)) == -1


def test_kernel_cfg_layout():
    # KernelCfg of decode_kernel.c:269-286: 15 ints and one float, 64 bytes,
    # eps at byte 32 and norm_topk_prob at byte 52 (decoder3.py:35-46)
    assert ctypes.sizeof(_lib.KernelCfg) == 64
    assert _lib.KernelCfg.eps.offset == 32
    assert _lib.KernelCfg.intermediate.offset == 40
    assert _lib.KernelCfg.norm_topk_prob.offset == 52
    assert _lib.KernelCfg.expert_bf16.offset == 60
    if _lib.LIB_PATH.exists():
        n, ndig, nt = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        assert _lib.lib().jm_abi_sizes(ctypes.byref(n), ctypes.byref(ndig), ctypes.byref(nt)) == 0
        assert n.value == 64 and 3 <= ndig.value <= 5 and nt.value >= 1
        assert _lib.lib().jm_version() == 1


def _cfg(**kw):
    c = _lib.KernelCfg()
    c.L, c.d, c.E, c.topk, c.intermediate, c.norm_topk_prob = 2, 2048, 128, 8, 768, 1
    for k, v in kw.items():
        setattr(c, k, v)
    return c


@pytest.mark.parametrize("kw,group,code", [
    (dict(topk=0), 64, -2), (dict(topk=129), 64, -2), (dict(E=0), 64, -2),
    (dict(E=513), 64, -2), (dict(d=2000), 64, -2), (dict(intermediate=700), 64, -2),
    (dict(d=8192), 64, -2), (dict(expert_i8=1), 64, -2), ({}, 48, -2),
])
def test_store_create_rejects_bad_shapes(kw, group, code):
    if not _lib.LIB_PATH.exists():
        pytest.skip("libjoule_amd.so not built")
    L = _lib.lib()
    cfg = _cfg(**kw)
    offs = np.zeros(16, np.uint64)
    h = ctypes.c_void_p()
    rc = L.jm_store_create(ctypes.byref(cfg), group, ctypes.c_void_p(4096), 1 << 20,
                           offs.ctypes.data, ctypes.byref(h))
    assert rc == code
    assert L.jm_last_error()
    assert h.value is None


def test_expert_job_layout():
    # ExpertJob of expert_ffn.c:145-157 / moe.py:32-42 on x86-64: six
    # pointers, five ints, two pointers, one float
    J = _lib.ExpertJob
    assert J.m_gg.offset == 48 and J.group.offset == 64 and J.x.offset == 72
    assert J.scratch.offset == 80 and J.prob.offset == 88 and ctypes.sizeof(J) == 96


def test_null_arguments_are_errors():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libjoule_amd.so not built")
    L = _lib.lib()
    assert L.jm_store_create(None, 64, None, 0, None, None) == -1
    assert L.jm_layer_ffn_batch(None, 0, None, 1, None, None, None, None) == -1
    assert L.jm_q4_gemm_f32(None, None, 1, None, None, 1, 64, 64, None) == -1
    assert L.jm_expert_gateup(None, 0, None, None, 1, None, None) == -1
    assert L.jm_expert_down(None, 0, None, None, None, 1, None, None) == -1
    assert L.jm_combine(None, None, None, 1, None, None) == -1
    assert L.jm_expert_job(None, None) == -1
    j = _lib.ExpertJob()
    assert L.jm_expert_job(ctypes.byref(j), None) == -1
    assert L.jm_store_destroy(None) == 0
    with pytest.raises(_lib.JouleError):
        _lib.check(L.jm_store_reserve(None, 4), "reserve")


def test_ctypes_argument_counts_match_the_header():
    """Each ctypes signature has as many arguments as the C prototype."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    protos = dict(re.findall(r"\b(jm_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S))
    assert set(protos) == set(_lib.SIGNATURES)
    for name, params in protos.items():
        params = params.strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert n == len(_lib.SIGNATURES[name][0]), (name, n, len(_lib.SIGNATURES[name][0]))


def test_act_digits_setting_null_store():
    """The digit-plane setting refuses a NULL store and reports -1 for it.
    No GPU work."""
    if not _lib.LIB_PATH.exists():
        pytest.skip("libjoule_amd.so not built")
    L = _lib.lib()
    assert L.jm_store_set_act_digits(None, 5) < 0
    assert L.jm_store_act_digits(None) == -1


def test_q4_gemm_min_tokens_setting():
    """The plugin product's kernel threshold: process-wide, 0 restores the
    default (the measured crossover, 7 tokens), negative is an error.  No
    GPU work."""
    if not _lib.LIB_PATH.exists():
        pytest.skip("libjoule_amd.so not built")
    L = _lib.lib()
    assert L.jm_get_q4_gemm_min_tokens() == 7
    try:
        assert L.jm_set_q4_gemm_min_tokens(-1) == -1
        assert L.jm_get_q4_gemm_min_tokens() == 7
        assert L.jm_set_q4_gemm_min_tokens(5) == 0
        assert L.jm_get_q4_gemm_min_tokens() == 5
    finally:
        assert L.jm_set_q4_gemm_min_tokens(0) == 0
    assert L.jm_get_q4_gemm_min_tokens() == 7
