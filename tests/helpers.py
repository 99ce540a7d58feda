"""Shared test plumbing: drives the C-ABI the way skyla-engine does (engine.py) on small
self-contained arenas."""
from __future__ import annotations

import contextlib
import os

import numpy as np

from skyla_hip import engine as E
from skyla_hip.abi import Context


def rel_l2(got: np.ndarray, want: np.ndarray) -> float:
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


# Floor of the f32 bar: a plain f32 reordering of a short dot product can land much closer
# to the oracle than one of 4096 terms by chance.
F32_FLOOR = 2e-6


def f32_reorder_bar(dtype, data, n_in: int, n_out: int, x, want) -> float:
    """Twice the relative L2 distance between a plain f32 reordering of the same product
    (numpy's float32 W @ x over the oracle's dequantised rows: blocked BLAS sums) and the
    oracle's sequential f32 dot (matrix.rs:50-53), floored at F32_FLOOR.  A kernel that
    multiplies f32 activations by the exact quants in f32 lands inside it."""
    from oracle import skyla_oracle as so

    w = so.dequantize(int(dtype), data, n_in * n_out).reshape(n_out, n_in)
    return max(2.0 * rel_l2(w @ np.asarray(x, np.float32), want), F32_FLOOR)


def pad64(n: int) -> int:
    return -(-n // 64) * 64


@contextlib.contextmanager
def tactics(**kw):
    """Tactic overrides (SKYLA_HIP_TACTIC's key=value entries, added after any already set),
    read when a pipeline is created or a recording ends.  A value of None adds nothing."""
    old = os.environ.get("SKYLA_HIP_TACTIC")
    items = [f"{k}={v}" for k, v in kw.items() if v is not None]
    os.environ["SKYLA_HIP_TACTIC"] = ",".join(([old] if old else []) + items)
    try:
        yield
    finally:
        if old is None:
            del os.environ["SKYLA_HIP_TACTIC"]
        else:
            os.environ["SKYLA_HIP_TACTIC"] = old


class Setup:
    """Weights (one planner) + a flat f32 arena: [64 ctl words][x rows][y rows][half]."""

    def __init__(self, ctx: Context, mats, n_in_max: int, n_out_max: int, rows: int = 1,
                 kquant_tactic=None, q8_0_tactic=None, extra_f32: int = 0):
        self.ctx = ctx
        self.planner = E.Planner(ctx.max_buffer())
        self.q = [self.planner.matrix(*m) for m in mats]  # (dtype, n_in, n_out, data)
        self.weights = E.upload_weights(ctx, self.planner)
        self.s_in, self.s_out = pad64(n_in_max), pad64(n_out_max)
        self.rows = rows
        self.x_off = 64
        self.y_off = self.x_off + self.s_in * rows
        self.half_off = self.y_off + self.s_out * rows          # f32 units
        self.extra_off = self.half_off + (self.s_in * rows) // 2 + 64
        size = (self.extra_off + extra_f32 + 64) * 4
        self.arena = ctx.alloc_host(size)
        self.k = E.Kernels(ctx, self.weights, self.arena, kquant_tactic, q8_0_tactic)

    def set_x(self, x: np.ndarray, n_tok: int | None = None) -> None:
        x = np.atleast_2d(np.asarray(x, np.float32))
        f = self.arena.as_f32()
        for t in range(x.shape[0]):
            f[self.x_off + t * self.s_in: self.x_off + t * self.s_in + x.shape[1]] = x[t]
        self.arena.as_u32()[2] = x.shape[0] if n_tok is None else n_tok
        self.arena.upload()

    def set_x_half(self, x: np.ndarray) -> None:
        """f16 activations in the half region (X_HALF inputs), stride s_in f16."""
        x = np.atleast_2d(np.asarray(x, np.float16))
        h = self.arena.host().view("<f2")
        base = 2 * self.half_off
        for t in range(x.shape[0]):
            h[base + t * self.s_in: base + t * self.s_in + x.shape[1]] = x[t]
        self.arena.as_u32()[2] = x.shape[0]
        self.arena.upload()

    def set_y(self, y: np.ndarray) -> None:
        y = np.atleast_2d(np.asarray(y, np.float32))
        f = self.arena.as_f32()
        for t in range(y.shape[0]):
            f[self.y_off + t * self.s_out: self.y_off + t * self.s_out + y.shape[1]] = y[t]
        self.arena.upload()

    def y(self, n_tok: int, n_out: int) -> np.ndarray:
        self.arena.download()
        f = self.arena.as_f32()
        return np.stack([f[self.y_off + t * self.s_out: self.y_off + t * self.s_out + n_out] for t in range(n_tok)])

    def run(self, fn, profile: bool = False):
        rec = self.ctx.record(profile, fn)
        try:
            self.ctx.replay(rec)
            return self.ctx.marks(rec) if profile else None
        finally:
            rec.free()

    def matvec(self, i: int, accum: bool = False):
        m = self.q[i]

        def body(r):
            g = E.Graph(r, self.k, None, None, False)
            g.matvec(m, (self.x_off, 0), (self.y_off, 0), accum, False)
        self.run(body)

    def matmul(self, i: int, n_tok: int, accum: bool = False):
        """The engine's batched Graph::matvec (f32 or f16 inputs per HALF_INPUTS)."""
        m = self.q[i]
        z = -(-n_tok // E.MATMUL_TILE_COLS)

        def body(r):
            g = E.Graph(r, self.k, None, None, True)
            x = (2 * self.half_off, self.s_in) if E.HALF_INPUTS else (self.x_off, self.s_in)
            g.matvec(m, x, (self.y_off, self.s_out), accum, True, groups_z=z)
        self.run(body)

    def matmul_variant(self, i: int, n_tok: int, accum: bool, x_half: bool):
        """A matmul pipeline built directly, with f16 (x_half) or f32 inputs."""
        m = self.q[i]
        ty = {E.DType.Q8_0: 0, E.DType.Q4K: 1, E.DType.Q6K: 2}[m.dtype]
        spec = [ty, int(accum), 0] + ([1] if x_half else [])
        p = self.ctx.create_pipeline("matmul", 5, 52, spec)
        w = self.weights[m.buf]
        p.bind_buffers([w, w, self.arena, self.arena, self.arena])
        x_off = 2 * self.half_off if x_half else self.x_off
        push = [m.off[0], m.off[1], m.off[2], m.off[3], x_off, self.y_off, m.n_in, m.n_out, self.s_in,
                self.s_out, 0, 0, 1]
        z = -(-n_tok // E.MATMUL_TILE_COLS)
        try:
            self.run(lambda r: r.dispatch(p, [-(-m.n_out // 128), 1, z], push))
        finally:
            p.free()

    def free(self):
        for b in self.weights:
            b.free()
        self.arena.free()
