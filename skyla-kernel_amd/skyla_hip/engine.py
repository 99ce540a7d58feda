"""The skyla-engine side of the quantized weight path, restated over the HIP backend.

skyla-engine is the caller of the backend: it lays weights out (planner.rs), creates the
pipelines with their tactics (kernels.rs), computes every dispatch's push words and grid
(graph.rs:23-46, graph/moe.rs:8-80) and owns the activation arena (arena.rs).  This module
restates those pieces so the GPU path is driven exactly the way the engine drives it; the
constants of the HIP arm of backend.rs are at the top.
"""
from __future__ import annotations

import dataclasses
from enum import IntEnum
from typing import Sequence


import numpy as np

from .abi import Buffer, Context, Pipeline, Recorder
from .abi import tactic as switch

# ---- backend.rs: the skyla-hip arm of `mod selected` ----------------------------------
MATMUL_TILE_COLS = 128   # tokens per matmul workgroup (matmul.hip TN, dense)
MOE_TILE_COLS = 32      # tokens per grouped-expert workgroup (matmul.hip TN, MOE)
HALF_INPUTS = False     # GEMM inputs stay f32: the matmul stages them to f16 itself, with a
                        # range guard (activations such as silu(g)*u can exceed f16's 65504)
HYBRID = False
# per-backend matvec tactics (waves per workgroup, rows per wave); kernels.rs:10-14
Q8_0_TACTIC = (4, 2)
KQUANT_TACTIC = (4, 2)
MATMUL_TILE_ROWS = 128
EXPERT_LPR = (64, 32, 16)

# arena.rs:6-7
ATTENTION_CHUNK = 64
FUSE_LEVELS = ("none", "qkv", "ffn", "all", "auto")  # the decode graph's fusion levels (Engine fuse)
MAX_SPLITS = 4096       # splits the attention merge weighs in LDS (kernels/attention.hip)
# Split counts the engine records its decode and prefill graphs for: a replay uses the
# smallest that covers the positions in play (each recording's attention grid and merge
# then span only those splits; the arena's own count is the last bucket).
SPLIT_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128, 256)
BATCH = 128
# What the MoE kernels hold (moe.hip): moe_route ranks at most 256 logits, one per thread of
# its workgroup, and picks at most 16; moe_sort ranks at most 1024 slots (moe_sort.comp:15).
MOE_MAX_EXPERTS, MOE_MAX_USED, MOE_MAX_SLOTS = 256, 16, 1024
# moe_sort's tile map of the grouped matmuls, directly before its table: a count and up to
# 280 two-word (expert, 32-slot tile) entries (moe.hip, matmul.hip)
MOE_TILE_MAP = 640


class DType(IntEnum):
    """ggml type ids (skyla-gguf/src/lib.rs:23-31)."""
    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q4K = 12
    Q6K = 14


BLOCK = {DType.F32: (1, 4), DType.F16: (1, 2), DType.Q8_0: (32, 34), DType.Q4K: (256, 144),
         DType.Q6K: (256, 210)}


def row_bytes(dtype: DType, n: int) -> int:
    """DType::row_bytes (skyla-gguf/src/lib.rs:45-53)."""
    per, nbytes = BLOCK[DType(dtype)]
    if n % per:
        raise ValueError(f"row of {n} elements is not a multiple of {per}")
    return n // per * nbytes


# ---- planner.rs ------------------------------------------------------------------------
# (block bytes, [(byte range, unit)]) per format (planner.rs:8-15)
LAYOUT = {
    DType.Q8_0: (34, [((2, 34), 16), ((0, 2), 2)]),
    DType.Q4K: (144, [((16, 144), 16), ((0, 16), 16)]),
    DType.Q6K: (210, [((0, 128), 16), ((128, 192), 16), ((192, 208), 16), ((208, 210), 2)]),
}


@dataclasses.dataclass(frozen=True)
class QMatrix:
    """weights.rs:7-14: region offsets are in units of each region's binding."""
    dtype: DType
    buf: int
    off: tuple
    n_in: int
    n_out: int


class Planner:
    """planner.rs:24-117: splits each block into 16-byte-aligned regions (a byte
    permutation) and packs matrices into buffers of at most `cap` bytes."""

    def __init__(self, cap: int):
        self.cap = cap
        self.sizes = [0]
        self.tables: list[tuple[int, np.ndarray]] = []
        self.splits: list[tuple[int, np.ndarray, int, list]] = []

    def _alloc(self, buf: int, nbytes: int) -> int:
        off = -(-self.sizes[buf] // 16) * 16
        self.sizes[buf] = off + nbytes
        return off

    def table(self, data: np.ndarray) -> int:
        """An f32 table (norm weights, RoPE frequencies, a [n_expert][n_embd] router) in
        buffer 0, row-major."""
        data = np.ascontiguousarray(data, dtype="<f4").reshape(-1)
        off = self._alloc(0, data.size * 4)
        self.tables.append((off, data))
        return off // 4

    def matrix(self, dtype: DType, n_in: int, n_out: int, data: np.ndarray) -> QMatrix:
        """`data` holds the tensor's raw GGUF blocks ([n_expert][n_out] rows of n_in)."""
        dtype = DType(dtype)
        if not (n_in % 256 == 0 or dtype == DType.Q8_0):
            raise ValueError(f"unsupported input size {n_in}")
        if dtype not in LAYOUT:
            raise ValueError(f"no GPU kernel for {dtype.name} weights")
        block, parts = LAYOUT[dtype]
        data = np.frombuffer(np.ascontiguousarray(data).tobytes(), dtype=np.uint8)
        n_blocks = data.size // block
        total = n_blocks * block + len(parts) * 16
        last = len(self.sizes) - 1
        if self.sizes[last] + total <= self.cap:
            buf = last
        else:
            self.sizes.append(0)
            buf = last + 1
        off, dst = [0, 0, 0, 0], []
        for i, ((lo, hi), unit) in enumerate(parts):
            start = self._alloc(buf, n_blocks * (hi - lo))
            off[i] = start // unit
            dst.append(((lo, hi), start))
        self.splits.append((buf, data[: n_blocks * block], block, dst))
        return QMatrix(dtype, buf, tuple(off), n_in, n_out)

    def buffer_size(self, buf: int) -> int:
        return -(-self.sizes[buf] // 16) * 16

    def fill(self, buf: int, out: np.ndarray) -> None:
        if buf == 0:
            for off, data in self.tables:
                out[off: off + data.size * 4] = data.view(np.uint8)
        for b, data, block, dst in self.splits:
            if b != buf:
                continue
            blocks = data.reshape(-1, block)
            for (lo, hi), start in dst:
                n = blocks.shape[0] * (hi - lo)
                out[start: start + n] = blocks[:, lo:hi].reshape(-1)


def upload_weights(ctx: Context, planner: Planner) -> list[Buffer]:
    """The buffer fill of Weights::load (weights.rs:127-136) plus the explicit upload a
    discrete GPU needs."""
    bufs = []
    for i in range(len(planner.sizes)):
        b = ctx.alloc_host(max(16, planner.buffer_size(i)))
        planner.fill(i, b.host())
        b.upload()
        bufs.append(b)
    return bufs


# ---- kernels.rs ------------------------------------------------------------------------
class Matvec:
    """kernels.rs:51-90 (the pipelines of one format) and 196-213 (pipeline, grouped,
    experts)."""

    def __init__(self, pipelines, experts, lanes, rows_per_group):
        self.pipelines, self.experts_, self.lanes, self.rows_per_group = pipelines, experts, lanes, rows_per_group

    def pipeline(self, accum: bool) -> Pipeline:
        return self.pipelines[int(accum)]

    def grouped(self) -> Pipeline:
        return self.experts_[0][1]

    def experts(self, units_per_row: int) -> tuple[Pipeline, int]:
        wanted = min(max(1 << max(0, (units_per_row - 1).bit_length()), 16), self.lanes)
        lpr, p = next(((l, q) for l, q in self.experts_ if l == wanted), self.experts_[0])
        return p, self.rows_per_group * self.lanes // lpr


def _matvec(ctx: Context, shader: str, dual_view: bool, push: int, matmul_type, tactic, lanes,
            weights: Sequence[Buffer], a: Buffer) -> Matvec:
    """kernels.rs:90-129."""
    waves, rows = tactic

    def build(accum: int, moe: int, lpr: int) -> Pipeline:
        if matmul_type is not None:
            spec = [matmul_type, accum, moe, 1] if HALF_INPUTS else [matmul_type, accum, moe]
        else:
            spec = [waves, accum, rows, moe, lpr]
        n_buffers = 4 + int(dual_view)
        p = ctx.create_pipeline_sets(shader, n_buffers, push, spec, len(weights))
        for i, w in enumerate(weights):
            bufs = [w] + ([w] if dual_view else []) + [a, a, a]
            p.bind_set_buffers(i, bufs)
        return p

    pipelines = [build(0, 0, lanes), build(1, 0, lanes)]
    if matmul_type is not None:
        experts = [(0, build(0, 1, 0))]
    else:
        experts = [(l, build(0, 1, l)) for l in EXPERT_LPR if l <= lanes]
    rpg = MATMUL_TILE_ROWS if matmul_type is not None else waves * rows
    return Matvec(pipelines, experts, lanes, rpg)


def _fused(ctx: Context, shader: str, dual_view: bool, push: int, tactic, accum: int,
           weights: Sequence[Buffer], a: Buffer) -> Matvec:
    """A fused decode matvec (matvec_*_norm / matvec_*_silu): the plain kernel's spec and
    bindings, two push words more (the second vector's offset, eps); one accum form."""
    waves, rows = tactic
    p = ctx.create_pipeline_sets(shader, 4 + int(dual_view), push, [waves, accum, rows, 0, 64], len(weights))
    for i, w in enumerate(weights):
        p.bind_set_buffers(i, [w] + ([w] if dual_view else []) + [a, a, a])
    return Matvec([p, p], [], 64, waves * rows)


class Kernels:
    """Kernels::new (kernels.rs:101-184), restricted to the pipelines of the quantized
    weight path."""

    def __init__(self, ctx: Context, weights: Sequence[Buffer], a: Buffer,
                 kquant_tactic=None, q8_0_tactic=None, kv: Buffer | None = None, c: Config | None = None,
                 precision: KvPrecision | None = None, embd_dtype: DType | None = None, fuse: str = "none"):
        if ctx.subgroup_size != 64:
            raise ValueError(f"no kernels for subgroup size {ctx.subgroup_size} (need 64)")
        lanes = 64
        kq = kquant_tactic or KQUANT_TACTIC
        q8 = q8_0_tactic or Q8_0_TACTIC
        w0 = weights[0]
        self.decode = [
            _matvec(ctx, "matvec_q8_0", True, 36, None, q8, lanes, weights, a),
            _matvec(ctx, "matvec_q4k", False, 36, None, kq, lanes, weights, a),
            _matvec(ctx, "matvec_q6k", True, 44, None, kq, lanes, weights, a),
        ]
        self.batch = [_matvec(ctx, "matmul", True, 52, t, (0, 0), lanes, weights, a) for t in (0, 1, 2)]
        # decode matvecs with the RMSNorm before them / the SiLU gate folded in (compiled for the
        # default tactics only)
        self.norm = self.silu_mv = self.glu = self.glu_norm = None
        if fuse not in FUSE_LEVELS:
            raise ValueError(f"fuse {fuse!r}: one of {', '.join(FUSE_LEVELS)}")
        self.fuse = fuse
        if fuse != "none":
            if kq != KQUANT_TACTIC or q8 != Q8_0_TACTIC:
                raise ValueError("the fused decode matvecs exist for the default tactics only")
            self.norm = [_fused(ctx, "matvec_q8_0_norm", True, 44, q8, 0, weights, a),
                         _fused(ctx, "matvec_q4k_norm", False, 44, kq, 0, weights, a),
                         _fused(ctx, "matvec_q6k_norm", True, 52, kq, 0, weights, a)]
            self.silu_mv = [_fused(ctx, "matvec_q8_0_silu", True, 44, q8, 1, weights, a),
                            _fused(ctx, "matvec_q4k_silu", False, 44, kq, 1, weights, a),
                            _fused(ctx, "matvec_q6k_silu", True, 52, kq, 1, weights, a)]
            # Q4_K gate and up in one launch writing silu(gate) * up: eight waves, half on
            # each matrix, 16 lanes per row, 16 outputs per workgroup
            self.glu = ctx.create_pipeline_sets("matvec_q4k_glu", 4, 44, [8, 0, 1, 0, 16], len(weights))
            # ... and the same launch with the FFN RMSNorm folded in (fuse "ffn")
            self.glu_norm = ctx.create_pipeline_sets("matvec_q4k_glun", 4, 52, [8, 0, 1, 0, 16], len(weights))
            for i, wb in enumerate(weights):
                self.glu.bind_set_buffers(i, [wb, a, a, a])
                self.glu_norm.bind_set_buffers(i, [wb, a, a, a])

        def build(name, bufs, push):
            p = ctx.create_pipeline(name, len(bufs), push, [])
            p.bind_buffers(bufs)
            return p

        self.silu = build("silu_mul", [a, a], 16)
        self.logits = build("moe_logits", [w0, a, a], 20)
        self.route = build("moe_route", [a, a], 20)
        self.combine = build("moe_combine", [a], 24)
        self.sort = build("moe_sort", [a], 20)
        self.to_half = build("to_half", [a, a, a], 24) if HALF_INPUTS else None
        if kv is None:
            return
        # the rest of the decode step (kernels.rs:186-193); heads are 128 wide, no gate
        if c.head_dim != 128 or c.n_head % c.n_head_kv or c.n_head // c.n_head_kv not in (1, 2, 4, 8):
            raise ValueError(f"no attention kernels for head_dim {c.head_dim}, "
                             f"{c.n_head}/{c.n_head_kv} heads")
        pr = KvPrecision(precision)
        k8, v8 = int(pr.keys_q8), int(pr.values_q8)

        def build_spec(name, bufs, push, spec):
            p = ctx.create_pipeline(name, len(bufs), push, spec)
            p.bind_buffers(bufs)
            return p

        self.rmsnorm = build("rmsnorm", [w0, a, a], 24)
        self.qkv = build_spec("qkv_prep", [w0, a, a, kv, kv], 64, [k8, v8, c.head_dim, c.head_dim, 0])
        self.attention = build_spec("attention", [a, a, kv, kv, kv], 44,
                                    [c.n_head // c.n_head_kv, ATTENTION_CHUNK, k8, v8, c.head_dim, c.head_dim])
        self.merge = build_spec("attention_merge", [a, a], 24, [c.head_dim, 0])
        # single-token steps: qkv_prep folded into the attention (kernels/attention.hip)
        self.attn_prep = self.attn_prep1 = self.rope_table = None
        if self.fuse != "none":
            spec = [c.n_head // c.n_head_kv, ATTENTION_CHUNK, k8, v8, c.head_dim, c.head_dim]
            self.attn_prep = build_spec("attention_prep", [w0, a, a, kv, kv], 72, spec)
            # a decode step's rope pairs, once for every layer's attention_prep
            # (tactic rope_table=0: each workgroup computes them)
            if switch("rope_table", "1") != "0":
                self.rope_table = build("rope_table", [w0, a, a], 12)
            # recordings of one split: the attention writes the merged rows itself
            # (tactic prep1=0 keeps attention_prep and the merge there)
            if switch("prep1", "1") != "0":
                self.attn_prep1 = build_spec("attention_prep1", [w0, a, a, kv, kv], 80, spec)
        self.take_last = build("take_last", [a, a], 16)
        # token rows gathered from the HBM token_embd, one binding set per weight buffer
        ty = {DType.Q8_0: 0, DType.Q4K: 1, DType.Q6K: 2}[DType(embd_dtype)]
        self.embed = ctx.create_pipeline_sets("embed", 4, 32, [ty], len(weights))
        for i, wb in enumerate(weights):
            self.embed.bind_set_buffers(i, [wb, wb, a, a])

    def matvec(self, dtype: DType, batched: bool, form: str | None = None) -> Matvec:
        if batched:
            s = self.batch
        else:
            s = self.decode if form is None else {"norm": self.norm, "silu": self.silu_mv}[form]
        return {DType.Q4K: s[1], DType.Q6K: s[2]}.get(DType(dtype), s[0])


# ---- arena.rs ----------------------------------------------------------------------------
@dataclasses.dataclass
class Config:
    """The fields of skyla_ref::Config (skyla-ref/src/lib.rs:17-37) the path reads (the
    attention layouts of qwen3, qwen3moe and qwen3vl text: n_rot = head_dim, no output gate,
    no recurrent layers; RoPE with or without YaRN scaling)."""
    n_embd: int
    n_ff: int = 0
    n_head: int = 1
    n_head_kv: int = 1
    head_dim: int = 128
    n_vocab: int = 64
    n_expert: int = 0
    n_expert_used: int = 0
    n_ff_expert: int = 0
    eps: float = 1e-6
    n_layer: int = 0
    rope_theta: float = 1e6
    # YaRN (rope.rs:7-31): (factor, original context length, attn_factor), or None
    rope_scaling: tuple | None = None

    @property
    def rope_mscale(self) -> float:
        """rope.rs:56: the magnitude YaRN puts on every rotated pair (1 without scaling)."""
        return rope_table(self)[1]


_libm = None


def _libm_f32(name: str):
    """The C library's f32 function `name` (powf, logf): the ones Rust's f32::powf and
    f32::ln call on this platform."""
    global _libm
    if _libm is None:
        import ctypes
        import ctypes.util
        _libm = ctypes.CDLL(ctypes.util.find_library("m"))
        for fn, n_args in (("powf", 2), ("logf", 1)):
            f = getattr(_libm, fn)
            f.restype = ctypes.c_float
            f.argtypes = [ctypes.c_float] * n_args
    return getattr(_libm, name)


def _corr_dim(n_dims: np.float32, original_ctx: np.float32, n_rot: float, base: np.float32) -> np.float32:
    """rope.rs:32-34, in f32."""
    f32, logf = np.float32, _libm_f32("logf")
    turns = f32(f32(f32(n_rot) * f32(2.0)) * f32(np.pi))  # n_rot * 2 * pi, left to right
    return f32(n_dims * f32(logf(f32(original_ctx / turns)))) / f32(f32(2.0) * f32(logf(base)))


def rope_table(c: Config) -> tuple[np.ndarray, float]:
    """rope.rs:36-58: the RoPE frequency of every pair, theta^(-2i / head_dim) with the f32
    exponent and the C library's powf, and under YaRN scaling each times
    freq_scale (1 - mix) + mix, mix ramping from 1 below the dimension of 32 turns over the
    original context to 0 above that of 1 turn; and the magnitude scale
    attn_factor (1 + 0.1 ln(1 / freq_scale)) (1 without scaling).  f32 arithmetic throughout,
    one rounding per operation as in Rust."""
    f32 = np.float32
    powf = _libm_f32("powf")
    d = f32(c.head_dim)
    base = [f32(powf(f32(c.rope_theta), f32(-2.0) * f32(i) / d)) for i in range(c.head_dim // 2)]
    if c.rope_scaling is None:
        return np.asarray(base, np.float32), 1.0
    factor, original_ctx, attn_factor = (f32(v) for v in c.rope_scaling)
    theta = f32(c.rope_theta)
    freq_scale = f32(1.0) / factor
    low = max(f32(np.floor(_corr_dim(d, original_ctx, 32.0, theta))), f32(0.0))
    high = min(f32(np.ceil(_corr_dim(d, original_ctx, 1.0, theta))), f32(d - f32(1.0)))
    out = []
    for i, f in enumerate(base):
        y = f32(f32(i) - low) / max(f32(high - low), f32(0.001))
        mix = f32(1.0) - min(max(y, f32(0.0)), f32(1.0))
        out.append(f32(f * f32(f32(freq_scale * f32(f32(1.0) - mix)) + mix)))
    mscale = f32(attn_factor * f32(f32(1.0) + f32(f32(0.1) * f32(_libm_f32("logf")(f32(f32(1.0) / freq_scale))))))
    return np.asarray(out, np.float32), float(mscale)


def rope_frequencies(c: Config) -> np.ndarray:
    """The frequency table the attention kernels read (rope_table's first half)."""
    return rope_table(c)[0]


# ---- kv.rs -------------------------------------------------------------------------------
class KvPrecision(IntEnum):
    """kv.rs:1-16."""
    F16 = 0
    Q8 = 1
    F16_KEYS_Q8_VALUES = 2

    @property
    def keys_q8(self) -> bool:
        return self == KvPrecision.Q8

    @property
    def values_q8(self) -> bool:
        return self != KvPrecision.F16


class KvLayout:
    """kv.rs:18-88: keys of every cached layer, then values, then the f16 scales of the
    8-bit halves; offsets in units of the view that reads them (f16 or i8 entries, f16
    scales)."""

    def __init__(self, precision: KvPrecision, layers: Sequence[bool], max_ctx: int, kv_dim: int):
        self.precision = KvPrecision(precision)
        n, self.slots = 0, []
        for cached in layers:
            n += int(cached)
            self.slots.append(max(n - 1, 0))
        self.n_layer = n
        self.per_layer = max_ctx * kv_dim

    @staticmethod
    def _width(q8: bool) -> int:
        return 1 if q8 else 2

    def keys_bytes(self) -> int:
        return self.n_layer * self.per_layer * self._width(self.precision.keys_q8)

    def values_bytes(self) -> int:
        return self.n_layer * self.per_layer * self._width(self.precision.values_q8)

    def scales_per_layer(self) -> int:
        return self.per_layer // 32

    def bytes(self) -> int:
        scaled = int(self.precision.keys_q8) + int(self.precision.values_q8)
        return self.keys_bytes() + self.values_bytes() + scaled * self.n_layer * self.scales_per_layer() * 2

    def keys(self, layer: int) -> int:
        return self.slots[layer] * self.per_layer

    def values(self, layer: int) -> int:
        return self.keys_bytes() // self._width(self.precision.values_q8) + self.slots[layer] * self.per_layer

    def _scales_base(self) -> int:
        return (self.keys_bytes() + self.values_bytes()) // 2

    def key_scales(self, layer: int) -> int:
        return self._scales_base() + self.slots[layer] * self.scales_per_layer()

    def value_scales(self, layer: int) -> int:
        skip = int(self.precision.keys_q8) * self.n_layer * self.scales_per_layer()
        return self._scales_base() + skip + self.slots[layer] * self.scales_per_layer()


def _next64(n: int) -> int:
    return -(-n // 64) * 64


@dataclasses.dataclass
class MoeRegions:
    logits: int
    ids: int
    weights: int
    gate: int
    up: int
    down: int
    table: int
    list: int
    stride: int
    tiles: int = 0  # the tile map, MOE_TILE_MAP words ending where the table starts


class Arena:
    """arena.rs:82-181 without the recurrent-state regions: fixed f32 offsets after 64
    control words, BATCH rows per batched region, and (with a precision) the KV cache
    buffer of kv.rs.  Two regions more than the reference: `tokens`, the u32 ids of the
    chunk, which the embed kernel gathers rows for (the reference dequantises them on the
    host into x, engine.rs:100-117), and the MoE tile map moe_sort writes before its table."""

    def __init__(self, ctx: Context, c: Config, max_ctx: int = 64, precision: KvPrecision | None = None):
        self.size = 64
        n_split = -(-max_ctx // ATTENTION_CHUNK)
        if n_split > MAX_SPLITS:
            raise ValueError(f"max_ctx {max_ctx} above {MAX_SPLITS * ATTENTION_CHUNK} positions (the merge's split table)")

        def batched(width):
            stride = _next64(width)
            off = self.size
            self.size += stride * BATCH
            return off, stride

        def single(width):
            off = self.size
            self.size += _next64(width)
            return off

        self.x, self.s_embd = batched(c.n_embd)
        self.n, _ = batched(c.n_embd)
        self.q, self.s_q = batched(c.n_head * c.head_dim)
        self.k, self.s_kv = batched(c.n_head_kv * c.head_dim)
        self.v, _ = batched(c.n_head_kv * c.head_dim)
        self.attn, self.s_attn = batched(c.n_head * c.head_dim)
        self.gate, self.s_ff = batched(c.n_ff)
        self.up, _ = batched(c.n_ff)
        self.part, self.s_part = batched(c.n_head * n_split * (c.head_dim + 2))
        self.last = single(c.n_embd)
        self.logits = single(c.n_vocab)
        self.rope_cs = single(c.head_dim)  # a decode step's (cos, sin) pairs (rope_table)
        stride = _next64(c.n_ff_expert)
        slots = c.n_expert_used * BATCH
        if c.n_expert:  # the limits of the MoE kernels (moe.hip), checked before any launch
            if c.n_expert > MOE_MAX_EXPERTS:
                raise ValueError(f"{c.n_expert} experts: moe_route and moe_sort take at most {MOE_MAX_EXPERTS}")
            if not 1 <= c.n_expert_used <= min(MOE_MAX_USED, c.n_expert):
                raise ValueError(f"{c.n_expert_used} experts per token: moe_route picks 1 to "
                                 f"{min(MOE_MAX_USED, c.n_expert)}")
            if slots > MOE_MAX_SLOTS:
                raise ValueError(f"{c.n_expert_used} experts x {BATCH} tokens = {slots} slots: moe_sort sorts at "
                                 f"most {MOE_MAX_SLOTS} (moe_sort.comp:15)")
        logits, ids, weights = single(c.n_expert * BATCH), single(slots), single(slots)
        gate, up, down = single(stride * slots), single(stride * slots), single(self.s_embd * slots)
        tiles = single(MOE_TILE_MAP)
        self.moe = MoeRegions(logits=logits, ids=ids, weights=weights, gate=gate, up=up, down=down,
                              table=single(2 * c.n_expert), list=single(slots), stride=stride, tiles=tiles)
        assert self.moe.table == tiles + MOE_TILE_MAP
        widest = max([_next64(w) * BATCH for w in (c.n_embd, c.n_head * c.head_dim, c.n_ff)]
                     + [stride * slots])
        self.half = single(widest // 2 + 64)
        self.tokens = single(BATCH)
        # the RMSNorm weights the fused decode matvecs read beside x: per layer the attention
        # and FFN norms, then the output norm (filled by Engine from the weight tables)
        self.s_norm, self.n_layer = _next64(c.n_embd), c.n_layer
        self.norms = single(self.s_norm * (2 * c.n_layer + 1)) if c.n_layer else None
        self.buffer = ctx.alloc_host(self.size * 4)
        self.n_split = n_split
        self.max_ctx = max_ctx
        self.kv_layout, self.kv = None, None
        if precision is not None:
            self.kv_layout = KvLayout(precision, [True] * c.n_layer, max_ctx, c.n_head_kv * c.head_dim)
            if self.kv_layout.bytes() > ctx.max_buffer():
                raise ValueError(f"KV cache for {max_ctx} tokens needs {self.kv_layout.bytes() >> 20} MiB, "
                                 "above the allocation cap")
            self.kv = ctx.alloc_host(max(16, self.kv_layout.bytes()))

    def f32(self):
        return self.buffer.as_f32()

    def u32(self):
        return self.buffer.as_u32()

    def norm(self, layer: int, ffn: bool = False) -> int:
        """Offset of a layer's attention (ffn False) or FFN norm weights in the norms region;
        layer -1 is the output norm."""
        slot = 2 * self.n_layer if layer < 0 else 2 * layer + int(ffn)
        return self.norms + self.s_norm * slot

    def set_ctl(self, first_token: int, pos: int, n_tokens: int) -> None:
        """Engine::load's control words (engine.rs:119-123)."""
        u = self.u32()
        u[0], u[1], u[2] = first_token, pos, n_tokens


# ---- graph.rs / graph/moe.rs -------------------------------------------------------------
class Graph:
    """The dispatches of graph.rs and graph/moe.rs that belong to the weight path."""

    def __init__(self, r: Recorder, k: Kernels, a: Arena, c: Config, batched: bool, n_split: int | None = None):
        self.r, self.k, self.a, self.c, self.batched = r, k, a, c, batched
        # attention splits of this recording (the grids of attention / attention_prep and the
        # merge's span): the arena's, or fewer for a recording that serves early positions
        self.n_split = n_split if n_split is not None else getattr(a, "n_split", 0)
        self.b = BATCH if batched else 1
        self.rope_done = False  # rope_table has written the step's pairs (decode_rope)
        # decode with the fused matvecs (Kernels.fuse): "qkv" folds the attention norm into
        # q/k/v; "ffn" also the FFN norm into the Q4_K gate/up pair; "all" the FFN norm into
        # gate/up, the SiLU into down and the output norm into the head; "auto" per layer:
        # "ffn" where gate and up run as the Q4_K pair, the FFN forms of "all" elsewhere
        fuse = getattr(k, "fuse", "none")
        on = not batched and fuse != "none" and a is not None and a.norms is not None
        self.fused = on
        self.fused_ffn = on and fuse in ("ffn", "auto")
        self.fused_all = on and fuse == "all"
        self.fused_auto = on and fuse == "auto"

    def stage(self, label: str) -> None:
        self.r.barrier()
        self.r.mark(label)

    def matvec(self, m: QMatrix, x, y, accum: bool, batched: bool, groups_z: int | None = None,
               form: str | None = None, aux: int = 0) -> None:
        """graph.rs:23-34.  `form` "norm" / "silu" (decode only) dispatches the fused kernel:
        x is the raw residual (norm, `aux` = the norm weights) or the gate rows (silu, `aux` =
        the up rows)."""
        mv = self.k.matvec(m.dtype, batched, form)
        groups = -(-m.n_out // mv.rows_per_group)
        o = m.off
        if batched:
            push = [o[0], o[1], o[2], o[3], x[0], y[0], m.n_in, m.n_out, x[1], y[1], 0, 0, 1]
        elif m.dtype == DType.Q6K:
            push = [o[0], o[1], o[2], o[3], x[0], y[0], m.n_in, m.n_out, 0, 0, 0]
        else:
            push = [o[0], o[1], x[0], y[0], m.n_in, m.n_out, 0, 0, 0]
        if form is not None:
            push += [aux, f32_bits(self.c.eps if form == "norm" else 0.0)]
        cols = (groups_z if groups_z is not None else BATCH // MATMUL_TILE_COLS) if batched else 1
        self.r.dispatch_set(mv.pipeline(accum), m.buf, [groups, 1, cols], push)

    def input(self, x, width: int, per_token: int, rows: int | None = None):
        """graph.rs:36-46: f32 -> f16 staging of a GEMM input (HALF_INPUTS)."""
        p = self.k.to_half
        if p is None or not self.batched:
            return x
        dst, stride = 2 * self.a.half, _next64(width)
        push = [x[0], dst, width, x[1], stride, per_token]
        n_rows = (rows if rows is not None else BATCH) * per_token
        self.r.dispatch(p, [-(-(width // 4) // 256), n_rows, 1], push)
        self.r.barrier()
        return dst, stride

    def experts(self, m: QMatrix, x, y) -> None:
        """graph/moe.rs:8-24."""
        units = {DType.Q4K: m.n_in // 32, DType.Q6K: m.n_in // 64}.get(m.dtype, 64)
        pipeline, rpg = self.k.matvec(m.dtype, False).experts(units)
        groups = -(-m.n_out // rpg)
        o = m.off
        push = [o[0], o[1], o[2], o[3]] if m.dtype == DType.Q6K else [o[0], o[1]]
        push += [x[0], y[0], m.n_in, m.n_out, self.a.moe.ids, x[1], y[1]]
        self.r.dispatch_set(pipeline, m.buf, [groups, self.c.n_expert_used, 1], push)

    def grouped(self, m: QMatrix, x, x_div: int, y) -> None:
        """graph/moe.rs:26-40."""
        mv = self.k.matvec(m.dtype, True)
        groups = -(-m.n_out // mv.rows_per_group)
        o, moe = m.off, self.a.moe
        push = [o[0], o[1], o[2], o[3], x[0], y[0], m.n_in, m.n_out, x[1], y[1], moe.table, moe.list, x_div]
        self.r.dispatch_set(mv.grouped(), m.buf, [groups, self.c.n_expert, BATCH // MOE_TILE_COLS], push)

    def moe(self, gate: QMatrix, up: QMatrix, down: QMatrix, router: int) -> None:
        """graph/moe.rs:42-80: logits -> route -> [sort] -> gate/up -> silu -> down -> combine."""
        a, c, m, b = self.a, self.c, self.a.moe, self.b
        used, n_embd, n_expert = c.n_expert_used, c.n_embd, c.n_expert
        self.r.dispatch(self.k.logits, [n_expert, b, 1], [a.n, router, m.logits, n_embd, a.s_embd])
        self.stage("moe logits")
        self.r.dispatch(self.k.route, [1, b, 1], [m.logits, m.ids, m.weights, n_expert, used])
        self.stage("moe route")
        if self.batched:
            self.r.dispatch(self.k.sort, [1, 1, 1], [m.ids, m.table, m.list, n_expert, used])
            self.stage("moe sort")
            xn = self.input((a.n, a.s_embd), n_embd, 1)
            self.grouped(gate, xn, used, (m.gate, m.stride))
            self.grouped(up, xn, used, (m.up, m.stride))
        else:
            self.experts(gate, (a.n, 0), (m.gate, m.stride))
            self.experts(up, (a.n, 0), (m.up, m.stride))
        self.stage("experts gate+up")
        n = b * used * m.stride
        self.r.dispatch(self.k.silu, [-(-n // 256), 1, 1], [m.gate, m.up, n, 0])
        self.stage("silu")
        if self.batched:
            xg = self.input((m.gate, m.stride), c.n_ff_expert, used)
            self.grouped(down, xg, 1, (m.down, a.s_embd))
        else:
            self.experts(down, (m.gate, m.stride), (m.down, a.s_embd))
        self.stage("experts down")
        self.r.dispatch(self.k.combine, [-(-n_embd // 256), b, 1],
                        [a.x, m.down, m.weights, n_embd, a.s_embd, used])
        self.stage("moe combine")

    def glu_pair(self, gate: QMatrix, up: QMatrix) -> bool:
        """A decode step's Q4_K gate and up of one shape and buffer run as one launch."""
        return (self.fused and not self.fused_all and self.k.glu is not None and gate.dtype == up.dtype == DType.Q4K
                and gate.buf == up.buf and (gate.n_in, gate.n_out) == (up.n_in, up.n_out))

    def ffn_all_forms(self, gate: QMatrix, up: QMatrix) -> bool:
        """The FFN norm folded into gate and up, the SiLU into down (fuse "all"; "auto" where
        gate and up are no Q4_K pair)."""
        return self.fused_all or (self.fused_auto and not self.glu_pair(gate, up))

    def dense_ffn(self, gate: QMatrix, up: QMatrix, down: QMatrix, l: int = 0) -> None:
        """graph.rs:174-184 (after the ffn rmsnorm): gate, up -> silu -> down (+= x)."""
        a, c, b, bt = self.a, self.c, self.b, self.batched
        if self.glu_pair(gate, up):
            # gate and up in one launch that writes silu(gate) * up: no silu_mul launch
            # ("ffn": from the raw residual, with the FFN norm folded in: no rmsnorm launch)
            g, u = gate.off, up.off
            push = [g[0], g[1], a.n, a.gate, gate.n_in, gate.n_out, 0, 0, 0, u[0], u[1]]
            kern = self.k.glu
            if self.fused_ffn:
                push[2] = a.x
                push += [a.norm(l, True), f32_bits(c.eps)]
                kern = self.k.glu_norm
            self.r.dispatch_set(kern, gate.buf, [-(-gate.n_out // 16), 1, 1], push)
            self.stage("matvec gate+up (silu)")
            self.matvec(down, (a.gate, a.s_ff), (a.x, a.s_embd), True, False)
            self.stage("matvec down")
            return
        if self.ffn_all_forms(gate, up):  # the FFN norm folded into gate and up, the SiLU into down
            f = dict(form="norm", aux=a.norm(l, True))
            self.matvec(gate, (a.x, a.s_embd), (a.gate, a.s_ff), False, False, **f)
            self.matvec(up, (a.x, a.s_embd), (a.up, a.s_ff), False, False, **f)
            self.stage("matvec gate+up")
            self.matvec(down, (a.gate, a.s_ff), (a.x, a.s_embd), True, False, form="silu", aux=a.up)
            self.stage("matvec down")
            return
        xn = self.input((a.n, a.s_embd), c.n_embd, 1)
        self.matvec(gate, xn, (a.gate, a.s_ff), False, bt)
        self.matvec(up, xn, (a.up, a.s_ff), False, bt)
        self.stage("matvec gate+up")
        self.r.dispatch(self.k.silu, [-(-c.n_ff // 256), b, 1], [a.gate, a.up, c.n_ff, a.s_ff])
        self.stage("silu")
        xg = self.input((a.gate, a.s_ff), c.n_ff, 1)
        self.matvec(down, xg, (a.x, a.s_embd), True, bt)
        self.stage("matvec down")

    # ---- the rest of graph.rs: norms, attention, a layer ----------------------------
    def rmsnorm(self, x: int, w: int, y: int, tokens: int) -> None:
        """graph.rs:48-52."""
        c = self.c
        push = [x, w, y, c.n_embd, f32_bits(c.eps), self.a.s_embd]
        self.r.dispatch(self.k.rmsnorm, [1, tokens, 1], push)

    def decode_rope(self, rope: int) -> None:
        """A single-token step's rope pairs for its position, once for every layer's
        attention_prep (rope_table; the values norm_rope would compute in each of its
        workgroups)."""
        if not (self.fused and self.k.attn_prep is not None and getattr(self.k, "rope_table", None) is not None):
            return
        a, c = self.a, self.c
        self.r.dispatch(self.k.rope_table, [1, 1, 1], [rope, a.rope_cs, f32_bits(c.rope_mscale)])
        self.stage("rope table")
        self.rope_done = True

    def embed(self, m: QMatrix) -> None:
        """The chunk's token rows into x (the reference's host-side Engine::load,
        engine.rs:100-117, as a gather from the HBM token_embd)."""
        a, c = self.a, self.c
        o = m.off
        # a single-token step reads its id from ctl[0] (the first token, engine.rs:119-123),
        # so Engine.step uploads the control words only
        ids = a.tokens if self.batched else 0
        push = [o[0], o[1], o[2], o[3], c.n_embd, ids, a.x, a.s_embd]
        self.r.dispatch_set(self.k.embed, m.buf, [-(-(c.n_embd // 32) // 256), self.b, 1], push)
        self.stage("embed")

    def attention(self, l: int, at: "AttnWeights", rope: int) -> None:
        """graph.rs:59-113: q/k/v matvecs, QK-norm + RoPE + KV write, split-K attention,
        merge, o (+= x)."""
        a, c, bt = self.a, self.c, self.batched
        if self.fused:  # the attention norm folded into q, k, v (x is the raw residual)
            f = dict(form="norm", aux=a.norm(l))
            for wm, out in ((at.wq, (a.q, a.s_q)), (at.wk, (a.k, a.s_kv)), (at.wv, (a.v, a.s_kv))):
                self.matvec(wm, (a.x, a.s_embd), out, False, False, **f)
        else:
            xn = self.input((a.n, a.s_embd), c.n_embd, 1)
            self.matvec(at.wq, xn, (a.q, a.s_q), False, bt)
            self.matvec(at.wk, xn, (a.k, a.s_kv), False, bt)
            self.matvec(at.wv, xn, (a.v, a.s_kv), False, bt)
        self.stage("matvec qkv")
        if self.fused and self.k.attn_prep is not None:
            self.attend_prep(l, at.q_norm, at.k_norm, rope)
        else:
            self.qk_rope(l, at.q_norm, at.k_norm, rope)
            self.attend(l)
        xa = self.input((a.attn, a.s_attn), c.n_head * c.head_dim, 1)
        self.matvec(at.wo, xa, (a.x, a.s_embd), True, bt)
        self.stage("matvec o")

    def qk_rope(self, l: int, q_norm: int, k_norm: int, rope: int) -> None:
        """graph.rs:67-88: QK-norm + RoPE of q (in place) and k, and k, v into layer l's cache."""
        a, c, kv = self.a, self.c, self.a.kv_layout
        push = [a.q, a.k, a.v, q_norm, k_norm, kv.keys(l), kv.values(l), c.n_head, c.n_head_kv,
                f32_bits(c.eps), rope, f32_bits(c.rope_mscale), a.s_q, a.s_kv, kv.key_scales(l),
                kv.value_scales(l)]
        self.r.dispatch(self.k.qkv, [c.n_head + 2 * c.n_head_kv, self.b, 1], push)
        self.stage("qk norm + rope")

    def attend_prep(self, l: int, q_norm: int, k_norm: int, rope: int) -> None:
        """qk_rope and attend of a single-token step as one launch (attention_prep), then the
        merge.  The step's q, k, v rows are raw: each workgroup norms and rotates its query
        heads, the one holding the new position writes its key and value."""
        a, c, kv = self.a, self.c, self.a.kv_layout
        scale = np.float32(1.0) / np.sqrt(np.float32(c.head_dim))
        push = [a.q, a.k, a.v, q_norm, k_norm, kv.keys(l), kv.values(l), c.n_head_kv, f32_bits(c.eps), rope,
                f32_bits(c.rope_mscale), kv.key_scales(l), kv.value_scales(l), a.part, self.n_split, f32_bits(scale),
                a.s_part, a.rope_cs if self.rope_done else 0xFFFFFFFF]
        if self.n_split == 1 and self.k.attn_prep1 is not None:
            # one split (every position in the first 64): the merged rows straight from the
            # attention (attention_prep1: the merge over one split is acc / l, same bits)
            self.r.dispatch(self.k.attn_prep1, [c.n_head_kv, 1, 1], push + [a.attn, a.s_attn])
            self.stage("attention (+ qk norm, rope, kv write, merge of one split)")
            return
        self.r.dispatch(self.k.attn_prep, [c.n_head_kv, self.n_split, 1], push)
        self.stage("attention (+ qk norm, rope, kv write)")
        push = [a.part, a.attn, self.n_split, ATTENTION_CHUNK, a.s_part, a.s_attn]
        self.r.dispatch(self.k.merge, [c.n_head, 1, 1], push)
        self.stage("attention merge")

    def attend(self, l: int) -> None:
        """graph.rs:89-109: split-K attention over layer l's cache, then the merge into attn."""
        a, c, kv = self.a, self.c, self.a.kv_layout
        scale = np.float32(1.0) / np.sqrt(np.float32(c.head_dim))
        push = [a.q, a.part, kv.keys(l), kv.values(l), c.n_head_kv, self.n_split, f32_bits(scale), a.s_q,
                a.s_part, kv.key_scales(l), kv.value_scales(l)]
        self.r.dispatch(self.k.attention, [c.n_head_kv, self.n_split, self.b], push)
        self.stage("attention")
        push = [a.part, a.attn, self.n_split, ATTENTION_CHUNK, a.s_part, a.s_attn]
        self.r.dispatch(self.k.merge, [c.n_head, self.b, 1], push)
        self.stage("attention merge")

    def layer(self, l: int, lw: "LayerWeights", rope: int) -> None:
        """graph.rs:150-185."""
        a, b = self.a, self.b
        if not self.fused:
            self.rmsnorm(a.x, lw.attn_norm, a.n, b)
            self.stage("rmsnorm")
        self.attention(l, lw.attn, rope)
        moe = lw.router is not None
        norm_folded = self.ffn_all_forms(lw.gate, lw.up) or (self.fused_ffn and self.glu_pair(lw.gate, lw.up))
        if not norm_folded or moe:
            self.rmsnorm(a.x, lw.ffn_norm, a.n, b)
            self.stage("rmsnorm")
        if moe:
            self.moe(lw.gate, lw.up, lw.down, lw.router)
        else:
            self.dense_ffn(lw.gate, lw.up, lw.down, l)


def f32_bits(v: float) -> int:
    """f32::to_bits of a push word."""
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0])


# ---- weights.rs --------------------------------------------------------------------------
@dataclasses.dataclass
class AttnWeights:
    q_norm: int
    k_norm: int
    wq: QMatrix
    wk: QMatrix
    wv: QMatrix
    wo: QMatrix


@dataclasses.dataclass
class LayerWeights:
    attn_norm: int
    ffn_norm: int
    attn: AttnWeights
    gate: QMatrix
    up: QMatrix
    down: QMatrix
    router: int | None = None


@dataclasses.dataclass
class Weights:
    buffers: list
    output: QMatrix
    embd: QMatrix
    out_norm: int
    rope: int
    layers: list


def load_weights(ctx: Context, model: dict, c: Config) -> Weights:
    """weights.rs:58-144 for the dense attention layout (and MoE FFNs), from a tensor map:
    name -> f32 array (norms, router) or (dtype, n_in, n_out, raw GGUF blocks[, n_expert]).
    Tables (RoPE frequencies, norms, routers) go first in buffer 0, as the planner puts them.
    token_embd is also laid out for the GPU embedding gather; a tied model (no
    output.weight) uses that one copy as its output head, as weights.rs:133-136 does."""
    p = Planner(ctx.max_buffer())
    rope = p.table(rope_frequencies(c))
    out_norm = p.table(model["output_norm.weight"])
    moe = c.n_expert > 0
    norms = []
    for i in range(c.n_layer):
        n = lambda s: f"blk.{i}.{s}.weight"  # noqa: E731
        norms.append((p.table(model[n("attn_norm")]), p.table(model[n("ffn_norm")]),
                      p.table(model[n("attn_q_norm")]), p.table(model[n("attn_k_norm")]),
                      p.table(model[n("ffn_gate_inp")]) if moe else None))

    def mat(name):  # expert tensors hold n_expert matrices of n_out rows (QMatrix.n_out per expert)
        t = model[name]
        return p.matrix(t[0], t[1], t[2], t[3])

    embd = mat("token_embd.weight")
    output = mat("output.weight") if "output.weight" in model else embd
    layers = []
    ffn = (lambda s: f"{s}_exps") if moe else (lambda s: s)
    for i, (attn_norm, ffn_norm, q_norm, k_norm, router) in enumerate(norms):
        n = lambda s: f"blk.{i}.{s}.weight"  # noqa: E731
        at = AttnWeights(q_norm, k_norm, mat(n("attn_q")), mat(n("attn_k")), mat(n("attn_v")), mat(n("attn_output")))
        gate, up, down = (mat(n(ffn(s))) for s in ("ffn_gate", "ffn_up", "ffn_down"))
        layers.append(LayerWeights(attn_norm, ffn_norm, at, gate, up, down, router))
    return Weights(upload_weights(ctx, p), output, embd, out_norm, rope, layers)


# ---- graph.rs::record, engine.rs ---------------------------------------------------------
def record(ctx: Context, k: Kernels, w: Weights, a: Arena, c: Config, batched: bool, profile: bool = False,
           n_split: int | None = None):
    """graph.rs:199-233: the decode step (one token) or a prefill chunk (BATCH rows, ctl[2]
    of them live), ending in the output head over the last row; `n_split` attention splits
    (default: the arena's), enough for positions below n_split * ATTENTION_CHUNK."""
    def body(r: Recorder) -> None:
        g = Graph(r, k, a, c, batched, n_split)
        g.embed(w.embd)
        g.decode_rope(w.rope)
        for l, lw in enumerate(w.layers):
            g.layer(l, lw, w.rope)
        src = a.x
        if batched:
            n = c.n_embd
            r.dispatch(k.take_last, [-(-n // 256), 1, 1], [a.x, a.last, n, a.s_embd])
            g.stage("take last")
            src = a.last
        if g.fused_all:
            g.matvec(w.output, (src, 0), (a.logits, 0), False, False, form="norm", aux=a.norm(-1))
        else:
            g.rmsnorm(src, w.out_norm, a.last, 1)
            g.stage("rmsnorm")
            g.matvec(w.output, (a.last, 0), (a.logits, 0), False, False)
        r.host_barrier()
        r.mark("matvec output")
    return ctx.record(profile, body)


class Engine:
    """engine.rs:12-152 over the HIP backend: weights, arena (with the KV cache), kernels,
    and the decode and prefill recordings; step() and prefill() return the logits of the
    last token."""

    def __init__(self, ctx: Context, model: dict, c: Config, max_ctx: int,
                 precision: KvPrecision = KvPrecision.F16_KEYS_Q8_VALUES, profile: bool = False,
                 fuse: str = "auto"):
        """fuse (decode step only; prefill keeps the separate launches): "qkv" folds the
        attention RMSNorm into the q/k/v matvecs; "ffn" also the FFN norm into the Q4_K
        gate/up pair; "all" folds the FFN norm into gate/up, the SiLU gate into the down
        projection and the output norm into the head; "auto" (the default) is "ffn" for
        layers whose gate and up run as the Q4_K pair and the FFN forms of "all" for the
        others, the head unfused; "none" keeps graph.rs's launches.  Measured on MI355X
        (tok/s, qkv / ffn / all): config 5 (Qwen3-8B Q4_K_M) at 1k context 495 / 513 / 474,
        at 16k 382 / 394 / 371; config 1 (Qwen3-0.6B Q8_0, no pair form) 890 / 886 / 970."""
        self.ctx, self.c = ctx, c
        self.weights = load_weights(ctx, model, c)
        self.arena = Arena(ctx, c, max_ctx, precision)
        a = self.arena
        if fuse != "none":
            f = a.f32()
            for l in range(c.n_layer):
                for ffn, name in ((False, "attn_norm"), (True, "ffn_norm")):
                    o = a.norm(l, ffn)
                    f[o: o + c.n_embd] = model[f"blk.{l}.{name}.weight"]
            f[a.norm(-1): a.norm(-1) + c.n_embd] = model["output_norm.weight"]
            a.buffer.upload(a.norms * 4, a.s_norm * (2 * c.n_layer + 1) * 4)
        self.kernels = Kernels(ctx, self.weights.buffers, self.arena.buffer, kv=self.arena.kv, c=c,
                               precision=precision, embd_dtype=self.weights.embd.dtype, fuse=fuse)
        self.profile = profile
        self.recordings = {}  # (batched, attention splits) -> recording, made on first use
        self.pos = 0
        self.recording(False, 1)
        self.recording(True, BATCH)

    def recording(self, batched: bool, n_pos: int):
        """The decode (batched False) or prefill recording for a replay whose positions stay
        below n_pos: the smallest split bucket that covers them.  graph.rs records one graph
        over the arena's splits; the splits past a token's position do no work there, but
        their workgroups still launch (an arena sized for 16k positions launches 2056 decode
        attention workgroups per layer, 136 of them with work at 1k), so the engine keeps a
        recording per bucket.  The merge adds the same splits in the same order either way,
        so the logits are the same bits."""
        need = -(-n_pos // ATTENTION_CHUNK)
        n_split = next((b for b in SPLIT_BUCKETS if need <= b < self.arena.n_split), self.arena.n_split)
        key = (batched, n_split)
        if key not in self.recordings:
            self.recordings[key] = record(self.ctx, self.kernels, self.weights, self.arena, self.c, batched,
                                          self.profile, n_split)
        return self.recordings[key]

    @property
    def decode(self):
        """The decode step's recording for the current position."""
        return self.recording(False, self.pos + 1)

    @property
    def prefill_rec(self):
        """The prefill chunk's recording for the current position."""
        return self.recording(True, self.pos + BATCH)

    def reset(self) -> None:
        self.pos = 0

    def load(self, tokens, batched: bool = True) -> None:
        """engine.rs:98-124: the chunk's token ids and the control words (a single-token
        step's id travels in ctl[0] only)."""
        a = self.arena
        if self.pos + len(tokens) > a.max_ctx:
            raise ValueError(f"context full ({a.max_ctx} tokens)")
        if len(tokens) > BATCH or any(int(t) >= self.c.n_vocab for t in tokens):
            raise ValueError("token outside the vocabulary or chunk longer than BATCH")
        u = a.u32()
        u[a.tokens: a.tokens + len(tokens)] = np.asarray(tokens, np.uint32)
        u[0], u[1], u[2] = int(tokens[0]), self.pos, len(tokens)
        a.buffer.upload(0, 64 * 4)
        if batched:
            a.buffer.upload(a.tokens * 4, len(tokens) * 4)

    def logits(self) -> np.ndarray:
        a = self.arena
        a.buffer.download(a.logits * 4, self.c.n_vocab * 4)
        return a.f32()[a.logits: a.logits + self.c.n_vocab].copy()

    def step(self, token: int) -> np.ndarray:
        """engine.rs:137-142."""
        self.load([token], batched=False)
        self.ctx.replay(self.decode)
        self.pos += 1
        return self.logits()

    def prefill(self, tokens) -> np.ndarray:
        """engine.rs:144-152: BATCH-token chunks."""
        if len(tokens) == 0:
            raise ValueError("prefill needs at least one token")
        for i in range(0, len(tokens), BATCH):
            chunk = tokens[i: i + BATCH]
            self.load(chunk)
            self.ctx.replay(self.prefill_rec)
            self.pos += len(chunk)
        return self.logits()

    def free(self) -> None:
        for rec in self.recordings.values():
            rec.free()
        self.recordings = {}
        for b in self.weights.buffers:
            b.free()
        if self.arena.kv is not None:
            self.arena.kv.free()
        self.arena.buffer.free()
