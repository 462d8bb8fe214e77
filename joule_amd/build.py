"""Build the HIP shared library (gfx950) in-tree.

    python -m joule_amd.build

compiles joule_amd/csrc/*.hip (objects under joule_amd/_build/) into
joule_amd/libjoule_amd.so with hipcc, and joule_amd/csrc/probe/jm_probe.hip
into joule_amd/libjoule_probe.so (launch and hand-off cost probes that
bench.py --probe runs; not part of the MoE block).
Flags: -ffp-contract=off (fused multiply-adds are written explicitly where
the reference arithmetic has them) and packed FP32 instructions disabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = sorted((PKG / "csrc").glob("*.hip"))
OUT = PKG / "libjoule_amd.so"
PROBE_SRC = PKG / "csrc" / "probe" / "jm_probe.hip"
PROBE_OUT = PKG / "libjoule_probe.so"
ARCH = os.environ.get("JM_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature; drop that line
    noise = [ln for ln in res.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(noise))
    if noise and verbose:
        print("\n".join(noise), file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile each source to an object in parallel (one process per file),
    then link the shared library."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objs = [objdir / (src.stem + ".o") for src in SRC]
    jobs = [[hipcc(), *compile_flags, "-c", str(src), "-o", str(obj)] for src, obj in zip(SRC, objs)]
    probe_tmp = PROBE_OUT.with_suffix(".so.tmp")
    jobs.append([hipcc(), *FLAGS, str(PROBE_SRC), "-o", str(probe_tmp)])
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for fut in [ex.submit(_run, cmd, verbose) for cmd in jobs]:
            fut.result()
    tmp = OUT.with_suffix(".so.tmp")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, OUT)
    os.replace(probe_tmp, PROBE_OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
