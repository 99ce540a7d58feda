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
BATCH = 128


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
        data = np.ascontiguousarray(data, dtype="<f4")
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
    """Weights::load (weights.rs:245-254) plus the explicit upload a discrete GPU needs."""
    bufs = []
    for i in range(len(planner.sizes)):
        b = ctx.alloc_host(max(16, planner.buffer_size(i)))
        planner.fill(i, b.host())
        b.upload()
        bufs.append(b)
    return bufs


# ---- kernels.rs ------------------------------------------------------------------------
class Matvec:
    """kernels.rs:55-60, 235-252."""

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


class Kernels:
    """kernels.rs:139-233, restricted to the pipelines of the quantized weight path."""

    def __init__(self, ctx: Context, weights: Sequence[Buffer], a: Buffer,
                 kquant_tactic=None, q8_0_tactic=None):
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

    def matvec(self, dtype: DType, batched: bool) -> Matvec:
        s = self.batch if batched else self.decode
        return {DType.Q4K: s[1], DType.Q6K: s[2]}.get(DType(dtype), s[0])


# ---- arena.rs ----------------------------------------------------------------------------
@dataclasses.dataclass
class Config:
    """The fields of skyla_ref::Config (skyla-ref/src/lib.rs:17-37) the path reads."""
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


class Arena:
    """arena.rs:82-113 without the KV cache and recurrent-state regions: fixed f32
    offsets after 64 control words, BATCH rows per batched region."""

    def __init__(self, ctx: Context, c: Config, max_ctx: int = 64):
        self.size = 64
        n_split = -(-max_ctx // ATTENTION_CHUNK)

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
        stride = _next64(c.n_ff_expert)
        slots = c.n_expert_used * BATCH
        self.moe = MoeRegions(
            logits=single(c.n_expert * BATCH), ids=single(slots), weights=single(slots),
            gate=single(stride * slots), up=single(stride * slots), down=single(self.s_embd * slots),
            table=single(2 * c.n_expert), list=single(slots), stride=stride)
        widest = max([_next64(w) * BATCH for w in (c.n_embd, c.n_head * c.head_dim, c.n_ff)]
                     + [stride * slots])
        self.half = single(widest // 2 + 64)
        self.buffer = ctx.alloc_host(self.size * 4)
        self.n_split = n_split

    def f32(self):
        return self.buffer.as_f32()

    def u32(self):
        return self.buffer.as_u32()

    def set_ctl(self, first_token: int, pos: int, n_tokens: int) -> None:
        """Engine::load's control words (engine.rs:119-123)."""
        u = self.u32()
        u[0], u[1], u[2] = first_token, pos, n_tokens


# ---- graph.rs / graph/moe.rs -------------------------------------------------------------
class Graph:
    """The dispatches of graph.rs and graph/moe.rs that belong to the weight path."""

    def __init__(self, r: Recorder, k: Kernels, a: Arena, c: Config, batched: bool):
        self.r, self.k, self.a, self.c, self.batched = r, k, a, c, batched
        self.b = BATCH if batched else 1

    def stage(self, label: str) -> None:
        self.r.barrier()
        self.r.mark(label)

    def matvec(self, m: QMatrix, x, y, accum: bool, batched: bool, groups_z: int | None = None) -> None:
        """graph.rs:23-34."""
        mv = self.k.matvec(m.dtype, batched)
        groups = -(-m.n_out // mv.rows_per_group)
        o = m.off
        if batched:
            push = [o[0], o[1], o[2], o[3], x[0], y[0], m.n_in, m.n_out, x[1], y[1], 0, 0, 1]
        elif m.dtype == DType.Q6K:
            push = [o[0], o[1], o[2], o[3], x[0], y[0], m.n_in, m.n_out, 0, 0, 0]
        else:
            push = [o[0], o[1], x[0], y[0], m.n_in, m.n_out, 0, 0, 0]
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

    def dense_ffn(self, gate: QMatrix, up: QMatrix, down: QMatrix) -> None:
        """graph.rs:174-184 (after the ffn rmsnorm): gate, up -> silu -> down (+= x)."""
        a, c, b, bt = self.a, self.c, self.b, self.batched
        xn = self.input((a.n, a.s_embd), c.n_embd, 1)
        self.matvec(gate, xn, (a.gate, a.s_ff), False, bt)
        self.matvec(up, xn, (a.up, a.s_ff), False, bt)
        self.stage("matvec gate+up")
        self.r.dispatch(self.k.silu, [-(-c.n_ff // 256), b, 1], [a.gate, a.up, c.n_ff, a.s_ff])
        self.stage("silu")
        xg = self.input((a.gate, a.s_ff), c.n_ff, 1)
        self.matvec(down, xg, (a.x, a.s_embd), True, bt)
        self.stage("matvec down")
