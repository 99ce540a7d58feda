"""GGUF files: the reader of skyla-gguf (reader.rs:66-125, lib.rs:12-157), a writer for
synthetic models, and the loader that turns a file into the engine's tensor map and Config
(skyla-ref/src/lib.rs:77-121 for the plain attention layouts).

The file is memory-mapped read-only; tensor data are views into the map (no copy until the
planner splits the blocks into regions).  Version 2 and 3 files, little-endian.
"""
from __future__ import annotations

import dataclasses
import struct
from typing import Any

import numpy as np

from .engine import BLOCK, Config, DType

# metadata value types (reader.rs:41-61)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<u1", I8: "<i1", U16: "<u2", I16: "<i2", U32: "<u4", I32: "<i4", F32: "<f4",
           BOOL: "<u1", U64: "<u8", I64: "<i8", F64: "<f8"}


@dataclasses.dataclass
class TensorInfo:
    """lib.rs:96-110: dims in GGUF order (dims[0] is the row length), absolute offset."""
    name: str
    dims: tuple
    dtype: int
    offset: int
    n_bytes: int

    def n_elements(self) -> int:
        return int(np.prod(self.dims, dtype=np.uint64)) if self.dims else 1


class _Reader:
    def __init__(self, buf: np.ndarray):
        self.buf, self.pos = buf, 0

    def bytes(self, n: int) -> np.ndarray:
        end = self.pos + n
        if n < 0 or end > self.buf.size:
            raise ValueError(f"unexpected end of file at {self.pos}")
        s = self.buf[self.pos:end]
        self.pos = end
        return s

    def scalar(self, ty: int):
        dt = np.dtype(_SCALAR[ty])
        return self.bytes(dt.itemsize).view(dt)[0]

    def u32(self) -> int:
        return int(self.scalar(U32))

    def u64(self) -> int:
        return int(self.scalar(U64))

    def string(self) -> str:
        return self.bytes(self.u64()).tobytes().decode("utf-8", errors="replace")

    def value(self, ty: int) -> Any:
        """reader.rs:41-61: integers widen to int, f32 to float, arrays recurse."""
        if ty in (U8, U16, U32, U64, I8, I16, I32, I64):
            return int(self.scalar(ty))
        if ty in (F32, F64):
            return float(self.scalar(ty))
        if ty == BOOL:
            return bool(self.scalar(ty))
        if ty == STR:
            return self.string()
        if ty == ARRAY:
            inner, n = self.u32(), self.u64()
            return [self.value(inner) for _ in range(n)]
        raise ValueError(f"unknown metadata value type {ty}")


def _block(dtype: int):
    try:
        return BLOCK[DType(dtype)]
    except ValueError:
        return None


class Gguf:
    """Gguf::open (reader.rs:66-125): header, metadata, tensor infos, data start aligned to
    general.alignment (32 by default); each tensor must end inside the file."""

    def __init__(self, path: str):
        self.path = path
        self.map = np.memmap(path, dtype=np.uint8, mode="r")
        r = _Reader(self.map)
        if r.bytes(4).tobytes() != b"GGUF":
            raise ValueError(f"{path} is not a GGUF file")
        self.version = r.u32()
        if self.version not in (2, 3):
            raise ValueError(f"unsupported GGUF version {self.version}")
        n_tensors, n_kv = r.u64(), r.u64()
        self.metadata: dict[str, Any] = {}
        for _ in range(n_kv):
            key = r.string()
            self.metadata[key] = r.value(r.u32())
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            n_dims = r.u32()
            dims = tuple(r.u64() for _ in range(n_dims))
            infos.append((name, dims, r.u32(), r.u64()))
        align = int(self.metadata.get("general.alignment", 32))
        data_start = -(-r.pos // align) * align
        self.tensors: dict[str, TensorInfo] = {}
        for name, dims, dtype, rel in infos:
            n = int(np.prod(dims, dtype=np.uint64)) if dims else 1
            blk = _block(dtype)
            n_bytes = -(-n // blk[0]) * blk[1] if blk else 0  # unsupported types: 0 bytes (lib.rs)
            offset = data_start + rel
            if offset + n_bytes > self.map.size:
                raise ValueError(f"tensor {name} runs past end of file")
            self.tensors[name] = TensorInfo(name, dims, dtype, offset, n_bytes)

    def meta(self, key: str):
        if key not in self.metadata:
            raise KeyError(f"missing metadata key {key}")
        return self.metadata[key]

    def tensor(self, name: str) -> TensorInfo:
        if name not in self.tensors:
            raise KeyError(f"missing tensor {name}")
        return self.tensors[name]

    def data(self, name: str) -> np.ndarray:
        """The tensor's raw bytes, a view into the map."""
        t = self.tensor(name)
        if _block(t.dtype) is None:
            raise ValueError(f"unsupported ggml type {t.dtype} ({name})")
        return self.map[t.offset: t.offset + t.n_bytes]


def _value_bytes(ty: int, v) -> bytes:
    if ty == STR:
        b = str(v).encode()
        return struct.pack("<Q", len(b)) + b
    if ty == ARRAY:
        inner, items = v
        return struct.pack("<IQ", inner, len(items)) + b"".join(_value_bytes(inner, x) for x in items)
    return np.array([v], dtype=_SCALAR[ty]).tobytes()


def write(path: str, metadata: dict, tensors: list, alignment: int = 32) -> None:
    """A version-3 GGUF file.  metadata: key -> (type, value) (ARRAY: (inner type, list));
    tensors: (name, dims, dtype, raw bytes) in file order, each aligned to `alignment`."""
    meta = dict(metadata)
    meta.setdefault("general.alignment", (U32, alignment))
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for key, (ty, v) in meta.items():
        kb = key.encode()
        out += struct.pack("<Q", len(kb)) + kb + struct.pack("<I", ty) + _value_bytes(ty, v)
    rel, placed = 0, []
    for name, dims, dtype, raw in tensors:
        raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
        nb = name.encode()
        out += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", int(d)) for d in dims)
        out += struct.pack("<IQ", int(dtype), rel)
        placed.append((rel, raw))
        rel = -(-(rel + raw.size) // alignment) * alignment
    start = -(-len(out) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(bytes(out) + b"\0" * (start - len(out)))
        pos = 0
        for off, raw in placed:
            f.write(b"\0" * (off - pos))
            f.write(raw.tobytes())
            pos = off + raw.size


# ---- skyla-ref Config::from_gguf and the tensor map ------------------------------------
# Config::from_gguf also accepts qwen35 (skyla-ref/src/lib.rs:80-83), whose recurrent
# layers and gated attention output are not on this path.
ARCHS = ("qwen3", "qwen3moe", "qwen3vl")


def rope_scaling_from_gguf(g: Gguf, arch: str):
    """RopeScaling::from_gguf (skyla-ref/src/rope.rs:14-30): (factor, original context
    length, attn_factor) for "yarn", None when the type is absent or "none"."""
    k = lambda s: f"{arch}.rope.scaling.{s}"  # noqa: E731
    kind = g.metadata.get(k("type"))
    if kind is None or kind == "none":
        return None
    if kind != "yarn":
        raise ValueError(f"unsupported rope scaling {kind}")
    f32 = lambda v: float(np.float32(v))  # noqa: E731  (meta_f64 as f32)
    return (f32(g.meta(k("factor"))), f32(g.meta(k("original_context_length"))),
            f32(g.metadata.get(k("attn_factor"), 1.0)))


def config_from_gguf(g: Gguf) -> Config:
    """skyla-ref/src/lib.rs:77-121 for the attention layouts of qwen3, qwen3moe and the
    qwen3vl text model (n_rot = head_dim, no recurrent layers); layers past block_count -
    nextn_predict_layers (the multi-token prediction heads) are not part of the model."""
    arch = g.meta("general.architecture")
    if arch not in ARCHS:
        raise ValueError(f"unsupported architecture {arch} (the GPU path serves {', '.join(ARCHS)})")
    k = lambda s: f"{arch}.{s}"  # noqa: E731
    opt = lambda s: int(g.metadata.get(k(s), 0))  # noqa: E731
    if g.metadata.get(k("ssm.state_size")) is not None:
        raise ValueError("recurrent (ssm) layers are outside the GPU path")
    n_embd, n_head = int(g.meta(k("embedding_length"))), int(g.meta(k("attention.head_count")))
    head_dim = int(g.metadata.get(k("attention.key_length"), n_embd // n_head))
    n_rot = opt("rope.dimension_count") or head_dim
    if n_rot != head_dim:
        raise ValueError(f"partial RoPE ({n_rot} of {head_dim}) is outside the GPU path")
    return Config(
        n_embd=n_embd, n_ff=opt("feed_forward_length"), n_head=n_head,
        n_head_kv=int(g.meta(k("attention.head_count_kv"))), head_dim=head_dim,
        n_vocab=int(g.tensor("token_embd.weight").dims[1]), n_expert=opt("expert_count"),
        n_expert_used=opt("expert_used_count"), n_ff_expert=opt("expert_feed_forward_length"),
        eps=float(np.float32(g.meta(k("attention.layer_norm_rms_epsilon")))),
        n_layer=int(g.meta(k("block_count"))) - opt("nextn_predict_layers"),
        rope_theta=float(np.float32(g.meta(k("rope.freq_base")))),
        rope_scaling=rope_scaling_from_gguf(g, arch))


def tensors_from_gguf(g: Gguf) -> dict:
    """The engine's tensor map: F32 tensors (norms, routers) as float32 arrays, quantized ones
    as (dtype, n_in, n_out, raw blocks[, n_expert]) with dims (n_in, n_out[, n_expert])."""
    out = {}
    for name, t in g.tensors.items():
        raw = g.data(name)
        if t.dtype == DType.F32:
            out[name] = raw.view("<f4").reshape(tuple(reversed(t.dims)) if len(t.dims) > 1 else -1)
        elif t.dtype in (DType.Q8_0, DType.Q4K, DType.Q6K):
            n_in, n_out = int(t.dims[0]), int(t.dims[1]) if len(t.dims) > 1 else 1
            entry = (DType(t.dtype), n_in, n_out, raw)
            out[name] = entry + (int(t.dims[2]),) if len(t.dims) > 2 else entry
    return out


def write_model(path: str, arch: str, c: Config, tensors: dict) -> None:
    """A GGUF file of a tensor map (as synth.qwen3 makes) with the metadata config_from_gguf
    reads."""
    meta = {"general.architecture": (STR, arch),
            f"{arch}.block_count": (U32, c.n_layer),
            f"{arch}.embedding_length": (U32, c.n_embd),
            f"{arch}.attention.head_count": (U32, c.n_head),
            f"{arch}.attention.head_count_kv": (U32, c.n_head_kv),
            f"{arch}.attention.key_length": (U32, c.head_dim),
            f"{arch}.feed_forward_length": (U32, c.n_ff),
            f"{arch}.rope.freq_base": (F32, c.rope_theta),
            f"{arch}.attention.layer_norm_rms_epsilon": (F32, c.eps)}
    if c.rope_scaling is not None:
        factor, original_ctx, attn_factor = c.rope_scaling
        meta.update({f"{arch}.rope.scaling.type": (STR, "yarn"), f"{arch}.rope.scaling.factor": (F32, factor),
                     f"{arch}.rope.scaling.original_context_length": (U32, int(original_ctx)),
                     f"{arch}.rope.scaling.attn_factor": (F32, attn_factor)})
    if c.n_expert:
        meta.update({f"{arch}.expert_count": (U32, c.n_expert), f"{arch}.expert_used_count": (U32, c.n_expert_used),
                     f"{arch}.expert_feed_forward_length": (U32, c.n_ff_expert)})
    ts = []
    for name, v in tensors.items():
        if isinstance(v, tuple):
            dims = (v[1], v[2]) + ((v[4],) if len(v) > 4 else ())
            ts.append((name, dims, int(v[0]), np.asarray(v[3])))
        else:
            a = np.ascontiguousarray(v, np.float32)
            ts.append((name, tuple(reversed(a.shape)), int(DType.F32), a))
    write(path, meta, ts)
