"""GGUF files assembled byte for byte from the layout reader.rs:66-125 reads (not from this
repository's writer), read back by skyla_hip.gguf: header and version, every metadata value
type (reader.rs:41-61), tensor infos in an order different from their data, the data start
padded to general.alignment (32 when absent), absolute offsets, the block-geometry byte
counts of lib.rs:12-53, and a 3-dim expert tensor handed to the engine's tensor map."""
import struct

import numpy as np
import pytest

from skyla_hip import engine as E
from skyla_hip import gguf as G


def _s(text: str) -> bytes:
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, ty: int, payload: bytes) -> bytes:
    return _s(key) + struct.pack("<I", ty) + payload


def _file(version: int, kvs: list, infos: list, data: bytes, align: int) -> bytes:
    head = b"GGUF" + struct.pack("<IQQ", version, len(infos), len(kvs)) + b"".join(kvs)
    for name, dims, ty, rel in infos:
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, rel)
    pad = -len(head) % align
    return head + b"\0" * pad + data, len(head) + pad


def _fixture(version: int, align: int | None):
    rng = np.random.default_rng(version * 100 + (align or 0))
    q4 = rng.integers(0, 256, size=3 * 4 * 144, dtype=np.uint8).tobytes()       # [256, 4, 3] Q4_K experts
    q6 = rng.integers(0, 256, size=2 * 210, dtype=np.uint8).tobytes()           # [256, 2] Q6_K
    q8 = rng.integers(0, 256, size=5 * 34, dtype=np.uint8).tobytes()            # [32, 5] Q8_0
    norm = rng.standard_normal(7).astype("<f4").tobytes()                      # [7] F32
    # data in the order norm, q8, q6, q4 with gaps; infos listed q4, norm, q6, q8
    rel = {"norm": 0, "q8": 64, "q6": 64 + 192, "q4": 64 + 192 + 448}
    blob = bytearray(rel["q4"] + len(q4) + 16)
    for k, b in (("norm", norm), ("q8", q8), ("q6", q6), ("q4", q4)):
        blob[rel[k]: rel[k] + len(b)] = b
    kvs = [
        _kv("general.architecture", 8, _s("qwen3moe")),
        _kv("t.u8", 0, struct.pack("<B", 200)), _kv("t.i8", 1, struct.pack("<b", -7)),
        _kv("t.u16", 2, struct.pack("<H", 65000)), _kv("t.i16", 3, struct.pack("<h", -300)),
        _kv("t.u32", 4, struct.pack("<I", 4000000000)), _kv("t.i32", 5, struct.pack("<i", -5)),
        _kv("t.f32", 6, struct.pack("<f", 1.5)), _kv("t.bool", 7, struct.pack("<B", 1)),
        _kv("t.arr", 9, struct.pack("<IQ", 8, 2) + _s("a") + _s("bc")),
        _kv("t.u64", 10, struct.pack("<Q", 2**40 + 3)), _kv("t.i64", 11, struct.pack("<q", -2**40)),
        _kv("t.f64", 12, struct.pack("<d", 0.1)),
    ]
    if align is not None:
        kvs.append(_kv("general.alignment", 4, struct.pack("<I", align)))
    infos = [("blk.0.ffn_gate_exps.weight", (256, 4, 3), 12, rel["q4"]), ("output_norm.weight", (7,), 0, rel["norm"]),
             ("output.weight", (256, 2), 14, rel["q6"]), ("token_embd.weight", (32, 5), 8, rel["q8"])]
    raw, start = _file(version, kvs, infos, bytes(blob), align or 32)
    return raw, start, rel, {"q4": q4, "q6": q6, "q8": q8, "norm": norm}


@pytest.mark.parametrize("version,align", [(3, None), (3, 64), (2, 128)])
def test_reads_hand_assembled_file(tmp_path, version, align):
    raw, start, rel, parts = _fixture(version, align)
    path = tmp_path / "f.gguf"
    path.write_bytes(raw)
    g = G.Gguf(str(path))
    assert g.version == version
    assert start % (align or 32) == 0
    m = g.metadata
    assert (m["t.u8"], m["t.i8"], m["t.u16"], m["t.i16"]) == (200, -7, 65000, -300)
    assert (m["t.u32"], m["t.i32"], m["t.u64"], m["t.i64"]) == (4000000000, -5, 2**40 + 3, -2**40)
    assert m["t.f32"] == 1.5 and m["t.f64"] == 0.1 and m["t.bool"] is True and m["t.arr"] == ["a", "bc"]
    assert m["general.architecture"] == "qwen3moe"
    for name, key, dims, dt, n_bytes in [("blk.0.ffn_gate_exps.weight", "q4", (256, 4, 3), 12, 3 * 4 * 144),
                                         ("output_norm.weight", "norm", (7,), 0, 28),
                                         ("output.weight", "q6", (256, 2), 14, 420),
                                         ("token_embd.weight", "q8", (32, 5), 8, 170)]:
        t = g.tensor(name)
        assert (t.dims, t.dtype, t.n_bytes, t.offset) == (dims, dt, n_bytes, start + rel[key])
        assert g.data(name).tobytes() == parts[key]
    tm = G.tensors_from_gguf(g)
    dt, n_in, n_out, data, n_exp = tm["blk.0.ffn_gate_exps.weight"]
    assert (dt, n_in, n_out, n_exp) == (E.DType.Q4K, 256, 4, 3) and data.tobytes() == parts["q4"]
    assert np.array_equal(tm["output_norm.weight"], np.frombuffer(parts["norm"], "<f4"))
    p = E.Planner(1 << 30)   # the expert tensor lays out as 3 x 4 rows of one super-block each
    q = p.matrix(dt, n_in, n_out * n_exp, np.asarray(data))
    assert q.n_out == 12


def test_rejects_version_and_truncation(tmp_path):
    raw, _, _, _ = _fixture(3, None)
    bad = tmp_path / "v1.gguf"
    bad.write_bytes(raw[:4] + struct.pack("<I", 1) + raw[8:])
    with pytest.raises(ValueError, match="version"):
        G.Gguf(str(bad))
    short = tmp_path / "short.gguf"
    short.write_bytes(raw[:-20])            # the last tensor (q4) now runs past the end
    with pytest.raises(ValueError, match="past end"):
        G.Gguf(str(short))
