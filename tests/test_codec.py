"""Q4 format and scalar conversions: exhaustive and known-answer tests.

Pins (reference src/jouleai/storage/q4_store.py:40-67 and
src/jouleai/native/decode_kernel.c:47-85):
* fp16 -> fp32 over all 65,536 codes against numpy's IEEE conversion;
* bf16 -> fp32 over all 65,536 codes (a 16-bit shift);
* quantiser known answers derived by hand: half-to-even ties, nibble order,
  zero and tiny groups, tail padding, record layout;
* dequantisation exact in float32 (checked in float64).
"""

import json

import numpy as np
import pytest

from joule_amd import q4_store as Q


def test_fp16_exhaustive(oracle_lib):
    codes = np.arange(65536, dtype=np.uint32)
    got = oracle_lib.fp16_to_f32_array(codes.astype(np.uint16))
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    is_nan = np.isnan(ref)
    assert np.array_equal(got[~is_nan].view(np.uint32), ref[~is_nan].view(np.uint32))
    # NaN codes keep their payload unchanged (no quieting): sign | 0x7F800000 | man << 13
    h = codes[is_nan]
    expect = ((h & 0x8000) << 16) | 0x7F800000 | ((h & 0x3FF) << 13)
    assert np.array_equal(got[is_nan].view(np.uint32), expect.astype(np.uint32))


def test_bf16_exhaustive(oracle_lib):
    codes = np.arange(65536, dtype=np.uint32)
    got = oracle_lib.bf16_to_f32_array(codes.astype(np.uint16))
    assert np.array_equal(got.view(np.uint32), (codes << 16).astype(np.uint32))


def _group(values, group=64, fill=0.0):
    g = np.full(group, fill, np.float32)
    g[:len(values)] = values
    return g


def test_quantize_known_answer_unit_scale():
    # absmax 7 -> scale fp16(1.0) = 0x3C00, q = round-half-even(v)
    v = _group([0.5, 1.5, 2.5, -0.5, -2.5, 7.0, -7.0, 3.49, -3.51, 0.0])
    sb, pb = Q.quantize(v, 64)
    sc = np.frombuffer(sb, np.uint16)
    pk = np.frombuffer(pb, np.uint8)
    assert sc.tolist() == [0x3C00]
    # q: 0, 2, 2, 0, -2, 7, -7, 3, -4, 0 then zeros -> nibbles q+8
    nib = [8, 10, 10, 8, 6, 15, 1, 11, 4, 8] + [8] * 54
    expect = [nib[2 * j] | (nib[2 * j + 1] << 4) for j in range(32)]
    assert pk.tolist() == expect
    assert pk[:5].tolist() == [0xA8, 0x8A, 0xF6, 0xB1, 0x84]


def test_quantize_zero_and_tiny_groups():
    # all-zero group: scale underflows to fp16 0, 0/0 -> NaN -> int8 0 -> nibble 8
    sb, pb = Q.quantize(np.zeros(64, np.float32), 64)
    assert np.frombuffer(sb, np.uint16).tolist() == [0]
    assert set(np.frombuffer(pb, np.uint8).tolist()) == {0x88}
    # tiny values: scale 0, +x/0 = +inf -> 7 (nibble 15), -x/0 -> -8 (nibble 0)
    v = _group([1e-10, -1e-10], 64)
    sb, pb = Q.quantize(v, 64)
    assert np.frombuffer(sb, np.uint16).tolist() == [0]
    assert np.frombuffer(pb, np.uint8)[0] == (15 | (0 << 4))
    assert np.frombuffer(pb, np.uint8)[1] == 0x88


def test_quantize_scale_rounding_and_group32():
    # absmax 1.0 -> scale fp16(1/7) = 0x3092 (0.142822265625)
    v = _group([1.0, -1.0, 0.5], 32)
    sb, pb = Q.quantize(v, 32)
    assert np.frombuffer(sb, np.uint16).tolist() == [0x3092]
    s = np.float32(np.float16(0.142822265625))
    # 1/s = 7.0017..., 0.5/s = 3.5008... -> 7, -7, 4 -> nibbles 15, 1, 12
    assert float(s) == 0.142822265625
    pk = np.frombuffer(pb, np.uint8)
    assert pk[0] == (15 | (1 << 4)) and pk[1] == (12 | (8 << 4))
    assert len(pk) == 16


def test_quantize_tail_padding():
    # 70 values, group 64: two scales, 64 packed bytes; the 58 padding
    # nibbles are stored as 0 (the padding is dropped after the clip)
    v = np.linspace(-1, 1, 70).astype(np.float32)
    sb, pb = Q.quantize(v, 64)
    assert len(sb) == 4 and len(pb) == 64
    pk = np.frombuffer(pb, np.uint8)
    assert pk[35:].tolist() == [0] * 29
    assert pk[32:35].tolist() != [0, 0, 0]
    w = Q.dequantize(sb, pb, 70, 64)
    assert w.shape == (70,)


def test_dequantize_exact():
    rng = np.random.default_rng(5)
    for group in (32, 64):
        w = rng.normal(0, 0.02, (96, 128)).astype(np.float32)
        sb, pb = Q.quantize(w, group)
        got = Q.dequantize(sb, pb, w.size, group)
        raw = np.frombuffer(pb, np.uint8)
        q = np.empty(raw.size * 2, np.int64)
        q[0::2] = (raw & 15).astype(np.int64) - 8
        q[1::2] = (raw >> 4).astype(np.int64) - 8
        s = np.frombuffer(sb, np.float16).astype(np.float64)
        exact = (q.reshape(-1, group) * s[:, None]).ravel()          # float64, exact
        assert np.array_equal(got.astype(np.float64), exact)
        # reconstruction error within half a quantisation step per element
        step = np.repeat(s, group)
        assert np.all(np.abs(got - w.ravel()) <= step * 0.5 + 1e-12)


def test_oracle_dequant_matches_codec(oracle_lib):
    rng = np.random.default_rng(6)
    w = rng.normal(0, 0.02, (64, 256)).astype(np.float32)
    for group in (32, 64):
        sb, pb = Q.quantize(w, group)
        sc = np.frombuffer(sb, np.uint16).copy()
        pk = np.frombuffer(pb, np.uint8).copy()
        a = oracle_lib.q4_dequant(pk, sc, w.size, group)
        b = Q.dequantize(sb, pb, w.size, group)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_store_record_layout(tmp_path):
    rng = np.random.default_rng(7)
    mats = {(l, e, p): rng.normal(0, 0.02, (8, 64) if p != "down" else (64, 8)).astype(np.float32)
            for l in range(2) for e in range(3) for p in Q.PARTS}
    Q.write_store(tmp_path, 2, 3, lambda l, e, p: mats[(l, e, p)], group=32)
    idx = json.loads((tmp_path / Q.INDEX_NAME).read_text())
    assert idx.pop("__group__") == 32
    blob = np.fromfile(tmp_path / Q.BIN_NAME, np.uint8)
    off = 0
    for l in range(2):
        for e in range(3):
            for p in Q.PARTS:
                r = idx[f"{l}.{e}.{p}"]
                assert r["offset"] == off
                sb, pb = Q.quantize(mats[(l, e, p)], 32)
                assert r["scales_bytes"] == len(sb) and r["packed_bytes"] == len(pb)
                assert r["numel"] == 512 and r["shape"] == list(mats[(l, e, p)].shape)
                assert blob[off:off + len(sb)].tobytes() == sb
                assert blob[off + len(sb):off + len(sb) + len(pb)].tobytes() == pb
                off += len(sb) + len(pb)
    assert off == blob.size
    index = Q.Q4Index.load(tmp_path / Q.INDEX_NAME)
    assert index.group == 32 and index.dims()[:2] == (2, 3)


def test_expert_bytes_formula():
    # 3 * rows * cols * (1/2 + 2/G) bytes per expert
    assert Q.expert_bytes(2048, 768, 64) == 2_506_752
    assert Q.expert_bytes(2048, 768, 32) == 2_654_208
    assert Q.expert_bytes(2048, 1024, 64) == 3_342_336
    assert Q.expert_bytes(2048, 1024, 32) == 3_538_944


@pytest.mark.parametrize("naming", ["qwen", "block_sparse_moe"])
def test_convert_from_safetensors(tmp_path, naming):
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file

    rng = np.random.default_rng(8)
    tensors = {}
    for l in range(2):
        for e in range(2):
            for p, shp in (("gate", (16, 64)), ("up", (16, 64)), ("down", (64, 16))):
                a = rng.normal(0, 0.02, shp).astype(np.float32)
                tensors[Q.expert_tensor_name(l, e, p, naming)] = torch.from_numpy(a).to(torch.bfloat16)
    model = tmp_path / "model"
    model.mkdir()
    save_file(tensors, str(model / "model.safetensors"))
    out = tmp_path / "store"
    path = Q.convert_experts_q4(model, out, 2, 2, naming=naming)
    idx = Q.Q4Index.load(out / Q.INDEX_NAME)
    blob = np.fromfile(path, np.uint8)
    for (l, e, p) in [(1, 1, "down"), (0, 1, "gate")]:
        r = idx.rec(l, e, p)
        src = tensors[Q.expert_tensor_name(l, e, p, naming)].float().numpy()
        sb, pb = Q.quantize(src, 64)
        o = r["offset"]
        assert blob[o:o + len(sb)].tobytes() == sb
        assert blob[o + len(sb):o + len(sb) + len(pb)].tobytes() == pb
    # idempotent: a second call returns early without rewriting
    mtime = path.stat().st_mtime_ns
    Q.convert_experts_q4(model, out, 2, 2, naming=naming)
    assert path.stat().st_mtime_ns == mtime
