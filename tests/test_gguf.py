"""The GGUF reader (skyla-gguf reader.rs:66-125), its writer for synthetic models, and the
loader into the engine's tensor map and Config (skyla-ref/src/lib.rs:77-121)."""
import struct

import numpy as np
import pytest

from skyla_hip import engine as E
from skyla_hip import gguf as G
from skyla_hip import synth


def test_model_round_trip(tmp_path):
    c = synth.qwen3_config("tiny")
    t = synth.qwen3("test-gguf", c, "q4_k_m", "random")
    path = str(tmp_path / "tiny.gguf")
    G.write_model(path, "qwen3", c, t)
    g = G.Gguf(path)
    assert g.version == 3 and g.meta("general.architecture") == "qwen3"
    c2 = G.config_from_gguf(g)
    for f in ("n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_vocab", "n_layer", "n_expert"):
        assert getattr(c2, f) == getattr(c, f), f
    assert np.float32(c2.eps) == np.float32(c.eps) and np.float32(c2.rope_theta) == np.float32(c.rope_theta)
    t2 = G.tensors_from_gguf(g)
    assert set(t2) == set(t)
    for name, v in t.items():
        if isinstance(v, tuple):
            assert t2[name][:3] == v[:3], name
            assert np.array_equal(np.asarray(t2[name][3]), v[3]), name
        else:
            assert np.array_equal(t2[name], v), name
    # every tensor's data starts on the alignment
    assert all(ti.offset % 32 == 0 for ti in g.tensors.values())
    # Q6_K head: dims (n_embd, n_vocab), 210-byte blocks
    ti = g.tensor("output.weight")
    assert ti.dims == (c.n_embd, c.n_vocab) and ti.dtype == E.DType.Q6K
    assert ti.n_bytes == c.n_vocab * E.row_bytes(E.DType.Q6K, c.n_embd)


def test_metadata_value_types(tmp_path):
    """reader.rs:41-61: every value type, arrays of arrays, signed widening."""
    meta = {"a.u8": (G.U8, 250), "a.i8": (G.I8, -5), "a.u16": (G.U16, 65535), "a.i16": (G.I16, -300),
            "a.u32": (G.U32, 4_000_000_000), "a.i32": (G.I32, -7), "a.f32": (G.F32, 0.1),
            "a.bool": (G.BOOL, True), "a.str": (G.STR, "héllo"), "a.u64": (G.U64, 2**40),
            "a.i64": (G.I64, -2**40), "a.f64": (G.F64, 0.1),
            "a.arr": (G.ARRAY, (G.ARRAY, [(G.I32, [1, -2]), (G.I32, [])]))}
    path = str(tmp_path / "m.gguf")
    G.write(path, meta, [])
    g = G.Gguf(path)
    m = g.metadata
    assert m["a.u8"] == 250 and m["a.i8"] == -5 and m["a.u16"] == 65535 and m["a.i16"] == -300
    assert m["a.u32"] == 4_000_000_000 and m["a.i32"] == -7 and m["a.u64"] == 2**40 and m["a.i64"] == -2**40
    assert m["a.f32"] == float(np.float32(0.1)) and m["a.f64"] == 0.1
    assert m["a.bool"] is True and m["a.str"] == "héllo"
    assert m["a.arr"] == [[1, -2], []]
    assert m["general.alignment"] == 32 and g.tensors == {}


def _header(version=3, n_tensors=0, n_kv=0):
    return b"GGUF" + struct.pack("<IQQ", version, n_tensors, n_kv)


def test_rejects_malformed_files(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGUX" + b"\0" * 20)
    with pytest.raises(ValueError, match="not a GGUF"):
        G.Gguf(str(p))
    p.write_bytes(_header(version=1))
    with pytest.raises(ValueError, match="unsupported GGUF version 1"):
        G.Gguf(str(p))
    # a metadata value of unknown type 13
    key = b"k"
    p.write_bytes(_header(n_kv=1) + struct.pack("<Q", 1) + key + struct.pack("<I", 13) + b"\0" * 8)
    with pytest.raises(ValueError, match="unknown metadata value type 13"):
        G.Gguf(str(p))
    # truncated inside the metadata
    p.write_bytes(_header(n_kv=1) + struct.pack("<Q", 50) + b"abc")
    with pytest.raises(ValueError, match="unexpected end of file"):
        G.Gguf(str(p))
    # a tensor that runs past the end of the file
    path = str(tmp_path / "t.gguf")
    G.write(path, {}, [("w", (256, 4), int(E.DType.Q4K), np.zeros(4 * 144, np.uint8))])
    data = open(path, "rb").read()
    p.write_bytes(data[:-10])
    with pytest.raises(ValueError, match="runs past end of file"):
        G.Gguf(str(p))


def test_unsupported_tensor_type_has_no_bytes(tmp_path):
    """lib.rs: a type without a block size (here ggml type 2, Q4_0) reads as 0 bytes and fails
    only when its data is asked for."""
    path = str(tmp_path / "u.gguf")
    G.write(path, {}, [("q40", (32, 2), 2, np.zeros(0, np.uint8)), ("f", (4,), 0, np.ones(4, np.float32))])
    g = G.Gguf(path)
    assert g.tensor("q40").n_bytes == 0
    with pytest.raises(ValueError, match="unsupported ggml type 2"):
        g.data("q40")
    assert np.array_equal(g.data("f").view("<f4"), np.ones(4, np.float32))


def test_config_rejects_other_layouts(tmp_path):
    c = synth.qwen3_config("tiny")
    t = synth.qwen3("test-gguf2", c, "q8_0", "ones")
    path = str(tmp_path / "a.gguf")
    G.write_model(path, "llama", c, t)
    with pytest.raises(ValueError, match="unsupported architecture llama"):
        G.config_from_gguf(G.Gguf(path))


def _with_meta(tmp_path, name, arch, c, t, extra):
    """A model file whose metadata adds `extra` (key -> (type, value)) to write_model's."""
    base = str(tmp_path / ("base-" + name))
    G.write_model(base, arch, c, t)
    g = G.Gguf(base)
    meta = {k: (G.STR if isinstance(v, str) else G.F32 if isinstance(v, float) else G.U32, v)
            for k, v in g.metadata.items() if k != "general.alignment"}
    meta.update(extra)
    ts = [(n, tuple(ti.dims), int(ti.dtype), np.array(g.data(n))) for n, ti in g.tensors.items()]
    path = str(tmp_path / name)  # a new file: the first stays mapped by its reader
    G.write(path, meta, ts)
    return G.Gguf(path)


def test_config_reads_yarn_scaling(tmp_path):
    """RopeScaling::from_gguf (rope.rs:14-30): type yarn with factor, original context and
    attn_factor (default 1.0), the frequencies and magnitude of rope.rs:36-58; "none" and an
    absent type give no scaling; any other type is an error."""
    from oracle import skyla_oracle as so
    c = synth.qwen3_config("tiny")
    t = synth.qwen3("test-gguf-yarn", c, "q8_0", "ones")
    key = "qwen3.rope.scaling."
    g = _with_meta(tmp_path, "y.gguf", "qwen3", c, t, {key + "type": (G.STR, "yarn"), key + "factor": (G.F32, 4.0),
                                                        key + "original_context_length": (G.U32, 32768)})
    c2 = G.config_from_gguf(g)
    assert c2.rope_scaling == (4.0, 32768.0, 1.0)
    f, m = E.rope_table(c2)
    of, om = so.rope_freqs_yarn(c2.head_dim, c2.rope_theta, 4.0, 32768.0, 1.0)
    assert np.array_equal(f, of) and np.float32(m) == np.float32(om) and abs(m - (1 + 0.1 * np.log(4.0))) < 1e-6
    g = _with_meta(tmp_path, "n.gguf", "qwen3", c, t, {key + "type": (G.STR, "none")})
    assert G.config_from_gguf(g).rope_scaling is None and G.config_from_gguf(g).rope_mscale == 1.0
    g = _with_meta(tmp_path, "l.gguf", "qwen3", c, t, {key + "type": (G.STR, "linear"), key + "factor": (G.F32, 2.0)})
    with pytest.raises(ValueError, match="unsupported rope scaling linear"):
        G.config_from_gguf(g)


def test_config_round_trips_yarn(tmp_path):
    """write_model stores a Config's YaRN scaling under the keys config_from_gguf reads."""
    import dataclasses
    c = dataclasses.replace(synth.qwen3_config("tiny"), rope_scaling=(8.0, 4096.0, 0.75))
    t = synth.qwen3("test-gguf-yarn2", c, "q8_0", "ones")
    path = str(tmp_path / "r.gguf")
    G.write_model(path, "qwen3", c, t)
    assert G.config_from_gguf(G.Gguf(path)).rope_scaling == (8.0, 4096.0, 0.75)


def test_config_qwen3vl_text_and_nextn(tmp_path):
    """Config::from_gguf (lib.rs:78-101) accepts the qwen3vl text model with the qwen3
    layout, and drops the nextn_predict_layers multi-token-prediction blocks from n_layer;
    recurrent (ssm) layouts are refused."""
    c = synth.qwen3_config("tiny")
    t = synth.qwen3("test-gguf-vl", c, "q4_k_m", "ones")
    g = _with_meta(tmp_path, "vl.gguf", "qwen3vl", c, t, {"qwen3vl.nextn_predict_layers": (G.U32, 1)})
    c2 = G.config_from_gguf(g)
    assert (c2.n_layer, c2.n_embd, c2.n_head, c2.head_dim) == (c.n_layer - 1, c.n_embd, c.n_head, c.head_dim)
    g = _with_meta(tmp_path, "ssm.gguf", "qwen3", c, t, {"qwen3.ssm.state_size": (G.U32, 128)})
    with pytest.raises(ValueError, match="recurrent"):
        G.config_from_gguf(g)
