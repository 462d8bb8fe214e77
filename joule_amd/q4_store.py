"""Q4 expert store: the on-disk format the HBM-resident store keeps byte for byte.

Format (reference: src/jouleai/storage/q4_store.py:1-9, 23-67, 125-166):

* A tensor is flattened in row-major order and cut into groups of ``group``
  values (64 in the reference's store, 32 also supported here).
* Per group one IEEE fp16 scale ``fp16(max(absmax, 1e-12) / 7)``.
* Values ``q = clip(round_half_even(v / fp32(scale)), -8, 7) + 8`` are packed
  two per byte, the even element in the low nibble.
* A tensor record is ``[all fp16 scales][all packed bytes]``; records follow
  each other in (layer, expert, part) order with part in (gate, up, down).
* ``experts_q4.json`` maps ``"l.e.part"`` to ``{offset, numel, scales_bytes,
  packed_bytes, shape}`` (same keys as the reference index).

Dequantisation ``(q - 8) * fp32(scale)`` is exact in fp32: a 4-bit integer
times an 11-bit significand needs at most 15 significant bits.

This module is offline tooling (conversion and inspection).  It runs on the
host with numpy and is not part of the per-token decode path.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Callable, Iterable, Iterator

import numpy as np

GROUP = 64
PARTS = ("gate", "up", "down")
BIN_NAME = "experts_q4.bin"
INDEX_NAME = "experts_q4.json"


def expert_tensor_name(l: int, e: int, part: str, naming: str = "qwen") -> str:
    """Checkpoint tensor name of one expert matrix (q4_store.py:26-37)."""
    if part not in PARTS:
        raise ValueError(f"unknown expert part {part!r}")
    if naming == "block_sparse_moe":
        w = {"gate": "w1", "up": "w2", "down": "w3"}[part]
        return f"model.layers.{l}.mlp.block_sparse_moe.experts.{e}.{w}.weight"
    if naming != "qwen":
        raise ValueError(f"unknown expert naming {naming!r}")
    return f"model.layers.{l}.mlp.experts.{e}.{part}_proj.weight"


def quantize(x: np.ndarray, group: int = GROUP) -> tuple[bytes, bytes]:
    """Quantise a tensor to ``(scales_bytes, packed_bytes)`` (q4_store.py:40-55).

    The arithmetic is numpy float32 throughout, as in the reference: the
    scale is computed in float32 and rounded to float16 (round to nearest
    even), the division is float32 and ``np.round`` rounds half to even.
    An all-zero group gets scale 0; its 0/0 quotients become NaN, which the
    int8 cast turns into 0, so those values are stored as nibble 8.
    A tail shorter than a group is padded for the scale computation and its
    padding nibbles are stored as 0.
    """
    if group not in (32, 64):
        raise ValueError(f"group must be 32 or 64, got {group}")
    flat = np.asarray(x).astype(np.float32).ravel()
    n = flat.size
    pad = (-n) % group
    padded = np.concatenate([flat, np.zeros(pad, np.float32)]) if pad else flat
    blocks = padded.reshape(-1, group)
    absmax = np.maximum(np.abs(blocks).max(axis=1), np.float32(1e-12))
    scales = (absmax / np.float32(7.0)).astype(np.float16)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = blocks / scales.astype(np.float32)[:, None]
        q = np.clip(np.round(ratio), -8, 7).astype(np.int8)
    nib = (q + 8).astype(np.uint8).ravel()[:n]
    if pad:
        nib = np.concatenate([nib, np.zeros(pad, np.uint8)])
    packed = (nib[0::2] & 0x0F) | (nib[1::2] << 4)
    return scales.tobytes(), packed.astype(np.uint8).tobytes()


def dequantize(scales_b: bytes | np.ndarray, packed_b: bytes | np.ndarray,
               numel: int, group: int = GROUP) -> np.ndarray:
    """Exact float32 dequantisation of one record (q4_store.py:58-67)."""
    raw = np.frombuffer(bytes(packed_b), dtype=np.uint8) if not isinstance(packed_b, np.ndarray) \
        else packed_b.view(np.uint8).ravel()
    sc = np.frombuffer(bytes(scales_b), dtype=np.float16) if not isinstance(scales_b, np.ndarray) \
        else scales_b.view(np.float16).ravel()
    q = np.empty(raw.size * 2, dtype=np.float32)
    q[0::2] = (raw & 0x0F).astype(np.float32) - 8.0
    q[1::2] = (raw >> 4).astype(np.float32) - 8.0
    w = q.reshape(-1, group) * sc.astype(np.float32)[:, None]
    return w.ravel()[:numel]


def record_sizes(rows: int, cols: int, group: int = GROUP) -> tuple[int, int]:
    """(scales_bytes, packed_bytes) of one [rows, cols] tensor record."""
    numel = rows * cols
    ngroups = -(-numel // group)
    return 2 * ngroups, (ngroups * group) // 2


def expert_bytes(d: int, m: int, group: int = GROUP) -> int:
    """Bytes of one expert (gate [m,d] + up [m,d] + down [d,m])."""
    return sum(sum(record_sizes(r, c, group)) for r, c in ((m, d), (m, d), (d, m)))


@dataclass
class Q4Index:
    """Parsed ``experts_q4.json``: offsets of every (layer, expert, part)."""

    records: dict
    group: int = GROUP

    @classmethod
    def load(cls, path: str | Path, group: int | None = None) -> "Q4Index":
        data = json.loads(Path(path).read_text())
        g = group
        if g is None:
            g = int(data.pop("__group__", GROUP)) if "__group__" in data else GROUP
        else:
            data.pop("__group__", None)
        return cls(data, g)

    def rec(self, l: int, e: int, part: str) -> dict:
        return self.records[f"{l}.{e}.{part}"]

    def dims(self) -> tuple[int, int, int]:
        """(n_layers, n_experts, max offset end) scanned from the keys."""
        L = E = 0
        end = 0
        for k, r in self.records.items():
            l, e, _ = k.split(".")
            L = max(L, int(l) + 1)
            E = max(E, int(e) + 1)
            end = max(end, r["offset"] + r["scales_bytes"] + r["packed_bytes"])
        return L, E, end

    def offset_table(self, n_layers: int, n_experts: int) -> np.ndarray:
        """uint64 [3, L*E, 2] of (scales offset, packed offset) in blob bytes."""
        tab = np.zeros((3, n_layers * n_experts, 2), dtype=np.uint64)
        for p_i, part in enumerate(PARTS):
            for l in range(n_layers):
                for e in range(n_experts):
                    r = self.rec(l, e, part)
                    tab[p_i, l * n_experts + e, 0] = r["offset"]
                    tab[p_i, l * n_experts + e, 1] = r["offset"] + r["scales_bytes"]
        return tab


def write_store(out_dir: str | Path, n_layers: int, n_experts: int,
                get_tensor: Callable[[int, int, str], np.ndarray],
                group: int = GROUP, progress_every: int = 0) -> Path:
    """Write ``experts_q4.bin`` + ``experts_q4.json`` from a tensor source.

    ``get_tensor(l, e, part)`` returns the float matrix of one expert part in
    checkpoint orientation (gate/up ``[m, d]``, down ``[d, m]``).  Records
    are appended in (layer, expert, part) order, as the reference converter
    does (q4_store.py:143-163).  A group other than 64 is recorded in the
    index under ``"__group__"`` (the reference index has no such key because
    its group is fixed).
    """
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    bin_path, idx_path = out_dir / BIN_NAME, out_dir / INDEX_NAME
    index: dict = {}
    offset = 0
    written = 0
    with open(bin_path, "wb") as f:
        for l in range(n_layers):
            for e in range(n_experts):
                for part in PARTS:
                    x = np.asarray(get_tensor(l, e, part))
                    sb, pb = quantize(x, group)
                    f.write(sb)
                    f.write(pb)
                    index[f"{l}.{e}.{part}"] = {
                        "offset": offset, "numel": int(x.size),
                        "scales_bytes": len(sb), "packed_bytes": len(pb),
                        "shape": list(x.shape),
                    }
                    offset += len(sb) + len(pb)
                    written += 1
                    if progress_every and written % progress_every == 0:
                        print(f"  q4 store: {written} tensors, {offset / 1e9:.2f} GB", flush=True)
    if group != GROUP:
        index["__group__"] = group
    idx_path.write_text(json.dumps(index))
    return bin_path


def convert_experts_q4(model_dir: str | Path, out_dir: str | Path,
                       n_layers: int, n_experts: int, naming: str = "qwen",
                       group: int = GROUP, progress_every: int = 512) -> Path:
    """Convert a safetensors checkpoint's experts to the Q4 store.

    Same contract as the reference converter (q4_store.py:125-166): it
    returns early when both output files exist, reads every expert tensor by
    its checkpoint name and writes the store.  Tensors are read with the
    ``safetensors`` numpy loader; bf16 tensors are widened to float32 first.
    """
    out_dir = Path(out_dir)
    bin_path, idx_path = out_dir / BIN_NAME, out_dir / INDEX_NAME
    if bin_path.exists() and idx_path.exists():
        return bin_path
    lookup = _safetensors_lookup(Path(model_dir))

    def get(l: int, e: int, part: str) -> np.ndarray:
        return lookup(expert_tensor_name(l, e, part, naming))

    return write_store(out_dir, n_layers, n_experts, get, group, progress_every)


def _safetensors_lookup(model_dir: Path) -> Callable[[str], np.ndarray]:
    """name -> float32 array over every ``*.safetensors`` file of a model."""
    from safetensors import safe_open

    files = sorted(model_dir.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files in {model_dir}")
    where: dict[str, Path] = {}
    for fp in files:
        with safe_open(str(fp), framework="pt") as f:
            for k in f.keys():
                where[k] = fp

    def get(name: str) -> np.ndarray:
        if name not in where:
            raise KeyError(name)
        with safe_open(str(where[name]), framework="pt") as f:
            return f.get_tensor(name).float().numpy()

    return get


def iter_records(bin_path: str | Path, index: Q4Index) -> Iterator[tuple[str, np.ndarray, np.ndarray]]:
    """Yield ``(key, scales u16, packed u8)`` for every record of a store."""
    mm = np.memmap(bin_path, dtype=np.uint8, mode="r")
    for key, r in index.records.items():
        o, sb, pb = r["offset"], r["scales_bytes"], r["packed_bytes"]
        yield key, np.asarray(mm[o:o + sb]).view(np.uint16), np.asarray(mm[o + sb:o + sb + pb])


def records_in(blob: np.ndarray, index: Q4Index, keys: Iterable[str]):
    """Views of ``(scales u16, packed u8)`` for the given keys of an in-memory blob."""
    out = []
    for key in keys:
        r = index.records[key]
        o, sb, pb = r["offset"], r["scales_bytes"], r["packed_bytes"]
        out.append((blob[o:o + sb].view(np.uint16), blob[o + sb:o + sb + pb]))
    return out
