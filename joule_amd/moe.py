"""HBM-resident Q4 expert store and the MoE decode block on the GPU.

Host-side mirror of the reference's MoE call surface:

* ``HbmExpertStore`` holds ``experts_q4.bin`` in device memory byte for byte
  (the reference memory-maps it and builds pointer tables,
  src/jouleai/native/decoder3.py:329-367).  ``ensure(l, e)`` returns the
  same ``((scales, packed, numel) x 3)`` records as the raw
  ``Q4ExpertPool.gather`` (src/jouleai/storage/q4_store.py:194-210), as
  device views.
* ``HbmExpertStore.layer_ffn_batch(l, x)`` is the reference's
  ``layer_ffn_batch(cfg, W, l, x, B, out)``
  (src/jouleai/native/decode_kernel.c:1387-1508) for one layer.

PyTorch provides device memory and streams; the arithmetic is in
libjoule_amd.so.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .q4_store import BIN_NAME, INDEX_NAME, PARTS, Q4Index, record_sizes


@dataclass(frozen=True)
class MoEShape:
    """MoE block shape: hidden d, intermediate m, experts E, top-k, renorm."""

    d: int
    m: int
    E: int
    topk: int
    renorm: bool
    name: str = ""

    def kernel_cfg(self, n_layers: int) -> _lib.KernelCfg:
        c = _lib.KernelCfg()
        c.L, c.d, c.E, c.topk = n_layers, self.d, self.E, self.topk
        c.intermediate = self.m
        c.norm_topk_prob = int(self.renorm)
        return c


# Shapes of the reference's two MoE families (arch/registry.py:56-94 fills
# the same fields from config.json).
OLMOE = MoEShape(d=2048, m=1024, E=64, topk=8, renorm=False, name="olmoe-1b-7b")
QWEN3 = MoEShape(d=2048, m=768, E=128, topk=8, renorm=True, name="qwen3-30b-a3b")


def check_tensor(t, name: str, shape: tuple, dtype, device) -> None:
    """Raise ValueError unless t is a contiguous tensor of exactly this shape
    and dtype on `device` (the kernels take raw pointers and sizes, so a
    wrong shape would make them read or write past the tensor)."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype or t.device != torch.device(device) or not t.is_contiguous() or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be a contiguous {dtype} tensor {list(shape)} on {device} "
                         f"(got {t.dtype} {list(t.shape)} on {t.device}"
                         f"{'' if t.is_contiguous() else ', not contiguous'})")


def offsets_for_layout(shape: MoEShape, n_layers: int, group: int) -> tuple[np.ndarray, int]:
    """(offset table [3, L*E, 2], total bytes) of a store written in the
    reference order (layer, expert, part) with records [scales][packed]."""
    sizes = [record_sizes(shape.m, shape.d, group), record_sizes(shape.m, shape.d, group),
             record_sizes(shape.d, shape.m, group)]
    per_expert = sum(a + b for a, b in sizes)
    LE = n_layers * shape.E
    tab = np.zeros((3, LE, 2), np.uint64)
    base = np.arange(LE, dtype=np.uint64) * np.uint64(per_expert)
    off = 0
    for p, (sb, pb) in enumerate(sizes):
        tab[p, :, 0] = base + np.uint64(off)
        tab[p, :, 1] = base + np.uint64(off + sb)
        off += sb + pb
    return tab, per_expert * LE


class HbmExpertStore:
    """The Q4 expert store resident in HBM, plus its router table.

    ``blob`` is a uint8 CUDA tensor holding the store file's bytes,
    ``offsets`` the [3, L*E, 2] uint64 table of (scales offset, packed
    offset) per (part, l*E+e).  The tensor stays referenced by this object.
    """

    def __init__(self, shape: MoEShape, n_layers: int, blob: torch.Tensor, offsets: np.ndarray,
                 group: int = 64):
        if blob.dtype != torch.uint8 or not blob.is_cuda or not blob.is_contiguous():
            raise ValueError("blob must be a contiguous uint8 CUDA tensor")
        self.shape, self.n_layers, self.group = shape, n_layers, group
        self.blob = blob
        self.offsets = np.ascontiguousarray(offsets, dtype=np.uint64).reshape(3, n_layers * shape.E, 2)
        self._cfg = shape.kernel_cfg(n_layers)
        handle = ctypes.c_void_p()
        _lib.check(_lib.lib().jm_store_create(ctypes.byref(self._cfg), group, _lib.ptr(blob),
                                              blob.numel(), _lib.ptr(self.offsets),
                                              ctypes.byref(handle)), "jm_store_create")
        self._h = handle
        self.router: torch.Tensor | None = None

    # ------------------------------------------------------------ loading

    @classmethod
    def from_dir(cls, store_dir: str | Path, shape: MoEShape, n_layers: int | None = None,
                 device: str | torch.device = "cuda", chunk_bytes: int = 1 << 28) -> "HbmExpertStore":
        """Upload ``experts_q4.bin`` (read in chunks) and index it."""
        store_dir = Path(store_dir)
        index = Q4Index.load(store_dir / INDEX_NAME)
        L, E, _ = index.dims()
        if E != shape.E:
            raise ValueError(f"store has {E} experts, shape says {shape.E}")
        n_layers = L if n_layers is None else n_layers
        offsets = index.offset_table(n_layers, E)
        path = store_dir / BIN_NAME
        nbytes = path.stat().st_size
        blob = torch.empty(nbytes, dtype=torch.uint8, device=device)
        with open(path, "rb") as f:
            pos = 0
            while pos < nbytes:
                buf = f.read(min(chunk_bytes, nbytes - pos))
                blob[pos:pos + len(buf)].copy_(torch.frombuffer(bytearray(buf), dtype=torch.uint8))
                pos += len(buf)
        return cls(shape, n_layers, blob, offsets, index.group)

    def set_router(self, gate_w: torch.Tensor) -> None:
        """Router table [L, E, d] (float32, or bfloat16 as in the reference)."""
        s = self.shape
        if tuple(gate_w.shape) != (self.n_layers, s.E, s.d):
            raise ValueError(f"router must be [{self.n_layers}, {s.E}, {s.d}]")
        if not gate_w.is_cuda or not gate_w.is_contiguous():
            raise ValueError("router must be a contiguous CUDA tensor")
        if gate_w.dtype == torch.float32:
            dt = _lib.JM_DTYPE_F32
        elif gate_w.dtype == torch.bfloat16:
            dt = _lib.JM_DTYPE_BF16
        else:
            raise ValueError("router dtype must be float32 or bfloat16")
        _lib.check(_lib.lib().jm_store_set_router(self._h, _lib.ptr(gate_w), dt), "jm_store_set_router")
        self.router = gate_w

    def router_bytes_per_weight(self) -> int:
        """Bytes per router weight the store's copy holds (2 for bf16-exact tables)."""
        dt = ctypes.c_int()
        _lib.check(_lib.lib().jm_store_router_dtype(self._h, ctypes.byref(dt)), "jm_store_router_dtype")
        return 2 if dt.value == _lib.JM_DTYPE_BF16 else 4

    def set_dense_min(self, min_tokens: int) -> None:
        """Segment size from which an expert takes the MFMA branch (batches
        with more than 256 slots); 0 restores the default."""
        _lib.check(_lib.lib().jm_store_set_dense_min(self._h, int(min_tokens)), "jm_store_set_dense_min")

    def set_act_digits(self, ndig: int) -> None:
        """Base-16 digit planes per activation value on the GEMV kernels: 4
        (the default; 0 restores it, about 15 bits per Q4 group) or 5 (about
        19 bits, more dot products per weight row).  Routing does not depend
        on it; the MFMA branch's int8 digit pairs are not affected."""
        _lib.check(_lib.lib().jm_store_set_act_digits(self._h, int(ndig)), "jm_store_set_act_digits")

    @property
    def act_digits(self) -> int:
        return int(_lib.lib().jm_store_act_digits(self._h))

    def dense_tiles(self, stream=None) -> int:
        """32-token tiles the MFMA branch computed in the last call."""
        t = torch.zeros(1, dtype=torch.int32, device=self.blob.device)
        _lib.check(_lib.lib().jm_store_copy_workspace(self._h, _lib.WS_N_DENSE_TILES, _lib.ptr(t), 4,
                                                      _lib.stream_handle(stream)), "jm_store_copy_workspace")
        return int(t.item())

    def reserve(self, max_B: int) -> None:
        _lib.check(_lib.lib().jm_store_reserve(self._h, int(max_B)), "jm_store_reserve")

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.lib().jm_store_destroy(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover - best effort at interpreter exit
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------- store surface

    def expert_size_bytes(self, l: int, e: int) -> int:
        s = self.shape
        return sum(sum(record_sizes(r, c, self.group)) for r, c in ((s.m, s.d), (s.m, s.d), (s.d, s.m)))

    def ensure(self, l: int, e: int):
        """((scales int16 view, packed uint8 view, numel) for gate, up, down)
        as device views, like the raw Q4ExpertPool.gather (q4_store.py:194-210)."""
        s = self.shape
        key = l * s.E + e
        outs = []
        for p, (rows, cols) in enumerate(((s.m, s.d), (s.m, s.d), (s.d, s.m))):
            sb, pb = record_sizes(rows, cols, self.group)
            so, po = (int(v) for v in self.offsets[p, key])
            outs.append((self.blob[so:so + sb].view(torch.int16), self.blob[po:po + pb], rows * cols))
        return tuple(outs)

    # --------------------------------------------------------- the block

    def layer_ffn_batch(self, l: int, x: torch.Tensor, out: torch.Tensor | None = None,
                        topk_idx: torch.Tensor | None = None, topk_w: torch.Tensor | None = None,
                        stream=None) -> torch.Tensor:
        """out[B, d] = MoE block of layer l on x[B, d] (float32, CUDA)."""
        if self.router is None:
            raise RuntimeError("router weights not set (set_router)")
        B = x.shape[0] if isinstance(x, torch.Tensor) and x.dim() == 2 else -1
        self._stage_in(x, "x", (B, self.shape.d), torch.float32)
        if out is None:
            out = torch.empty_like(x)
        else:
            self._stage_in(out, "out", (B, self.shape.d), torch.float32)
        if topk_idx is not None:
            self._stage_in(topk_idx, "topk_idx", (B, self.shape.topk), torch.int32)
        if topk_w is not None:
            self._stage_in(topk_w, "topk_w", (B, self.shape.topk), torch.float32)
        _lib.check(_lib.lib().jm_layer_ffn_batch(self._h, int(l), _lib.ptr(x), B, _lib.ptr(out),
                                                 _lib.ptr(topk_idx), _lib.ptr(topk_w),
                                                 _lib.stream_handle(stream)), "jm_layer_ffn_batch")
        return out

    # ------------------------------------------------ the block's stages

    def _stage_in(self, t: torch.Tensor, name: str, shape: tuple, dtype) -> None:
        check_tensor(t, name, shape, dtype, self.blob.device)

    def expert_gateup(self, l: int, x: torch.Tensor, top: torch.Tensor, stream=None) -> torch.Tensor:
        """act[B * topk, m]: SwiGLU of each slot's expert's gate and up rows
        against its token (ffn_expert_worker's first half,
        decode_kernel.c:1365-1375); slot = b * topk + i of top[B, topk]."""
        s = self.shape
        B = x.shape[0] if x.dim() == 2 else -1
        self._stage_in(x, "x", (B, s.d), torch.float32)
        self._stage_in(top, "top", (B, s.topk), torch.int32)
        act = torch.empty((B * s.topk, s.m), dtype=torch.float32, device=x.device)
        _lib.check(_lib.lib().jm_expert_gateup(self._h, int(l), _lib.ptr(x), _lib.ptr(top), B, _lib.ptr(act),
                                               _lib.stream_handle(stream)), "jm_expert_gateup")
        return act

    def expert_down(self, l: int, act: torch.Tensor, top: torch.Tensor, tw: torch.Tensor,
                    stream=None) -> torch.Tensor:
        """y[B * topk, d] = tw[slot] * (down rows of the slot's expert . act[slot])
        (ffn_expert_worker's second half, decode_kernel.c:1376-1383)."""
        s = self.shape
        B = top.shape[0] if top.dim() == 2 else -1
        self._stage_in(act, "act", (B * s.topk, s.m), torch.float32)
        self._stage_in(top, "top", (B, s.topk), torch.int32)
        self._stage_in(tw, "tw", (B, s.topk), torch.float32)
        y = torch.empty((B * s.topk, s.d), dtype=torch.float32, device=act.device)
        _lib.check(_lib.lib().jm_expert_down(self._h, int(l), _lib.ptr(act), _lib.ptr(top), _lib.ptr(tw), B,
                                             _lib.ptr(y), _lib.stream_handle(stream)), "jm_expert_down")
        return y

    def combine(self, y: torch.Tensor, top: torch.Tensor, stream=None) -> torch.Tensor:
        """out[B, d] = each token's y rows summed in the reference's union
        order (decode_kernel.c:1502-1507)."""
        s = self.shape
        B = top.shape[0] if top.dim() == 2 else -1
        self._stage_in(y, "y", (B * s.topk, s.d), torch.float32)
        self._stage_in(top, "top", (B, s.topk), torch.int32)
        out = torch.empty((B, s.d), dtype=torch.float32, device=y.device)
        _lib.check(_lib.lib().jm_combine(self._h, _lib.ptr(y), _lib.ptr(top), B, _lib.ptr(out),
                                         _lib.stream_handle(stream)), "jm_combine")
        return out

    def profile(self, enable: bool = True) -> None:
        """Record HIP events around each kernel of later calls."""
        _lib.check(_lib.lib().jm_store_profile(self._h, int(bool(enable))), "jm_store_profile")

    def stage_ms(self) -> dict:
        """Milliseconds per stage of the last call (waits for it)."""
        ms = (ctypes.c_float * len(_lib.STAGES))()
        _lib.check(_lib.lib().jm_store_stage_ms(self._h, ms, len(_lib.STAGES)), "jm_store_stage_ms")
        return dict(zip(_lib.STAGES, [float(v) for v in ms]))

    def read_workspace(self, B: int, stream=None) -> dict:
        """Host copies of the last call's dispatch and per-slot intermediates."""
        s = self.shape
        nslot = B * s.topk
        dev = self.blob.device

        def grab(field, shape, dtype):
            t = torch.empty(shape, dtype=dtype, device=dev)
            _lib.check(_lib.lib().jm_store_copy_workspace(self._h, field, _lib.ptr(t),
                                                          t.numel() * t.element_size(),
                                                          _lib.stream_handle(stream)),
                       "jm_store_copy_workspace")
            return t

        res = {
            "logits": grab(_lib.WS_LOGITS, (B, s.E), torch.float32),
            "seg_off": grab(_lib.WS_SEG_OFF, (s.E + 1,), torch.int32),
            "seg_slot": grab(_lib.WS_SEG_SLOT, (nslot,), torch.int32),
            "active": grab(_lib.WS_ACTIVE, (s.E,), torch.int32),
            "n_active": grab(_lib.WS_N_ACTIVE, (1,), torch.int32),
            "first_slot": grab(_lib.WS_FIRST_SLOT, (s.E,), torch.int32),
            "act": grab(_lib.WS_ACT, (nslot, s.m), torch.float32),
            "y": grab(_lib.WS_Y, (nslot, s.d), torch.float32),
        }
        torch.cuda.synchronize(dev)
        res = {k: v.cpu() for k, v in res.items()}
        res["active"] = res["active"][: int(res["n_active"][0])]
        return res


def algorithmic_bytes(shape: MoEShape, group: int, B: int, n_active: int, router_bytes: int = 4) -> int:
    """Bytes one block call must move: the routed experts' Q4 records, the
    router table and x in / out (top-k outputs are negligible)."""
    s = shape
    eb = sum(sum(record_sizes(r, c, group)) for r, c in ((s.m, s.d), (s.m, s.d), (s.d, s.m)))
    return n_active * eb + s.E * s.d * router_bytes + 2 * B * s.d * 4


PART_NAMES = PARTS
