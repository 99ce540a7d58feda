"""skyla_hip_dispatch_noalloc, the entry point that allocates nothing, against the existing
one-dispatch entry point (skyla_hip_time_dispatch with one repetition) through the C-ABI.

A dense Q4_K matmul at M = 512 (128 tiles: the K split, S = 2) and then at M = 128 (32
tiles, S = 4) takes its partial tiles and counters from the context's static scratch array;
both calls must give the same bits as the existing entry point (same kernels, same split,
a workspace of its own) and stay within the GEMM bar of the oracle.  A matvec pipeline
(no workspace) goes through the same entry point too.
"""
import numpy as np
import pytest

from helpers import Setup, rel_l2
from oracle import skyla_oracle as so
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu


def _matmul_pipeline(ctx, s, m):
    p = ctx.create_pipeline("matmul", 5, 52, [1, 0, 0])
    w = s.weights[m.buf]
    p.bind_buffers([w, w, s.arena, s.arena, s.arena])
    push = [m.off[0], m.off[1], m.off[2], m.off[3], s.x_off, s.y_off, m.n_in, m.n_out, s.s_in, s.s_out, 0, 0, 1]
    return p, push


def test_dispatch_noalloc_matches_time_dispatch(ctx):
    n_in, n_out = 4096, 4096
    data = synth.matrix("test-noalloc", "q4k", E.DType.Q4K, n_in, n_out)
    s = Setup(ctx, [(E.DType.Q4K, n_in, n_out, data)], n_in, n_out, rows=512)
    p, push = _matmul_pipeline(ctx, s, s.q[0])
    try:
        for n_tok in (512, 128):   # the second call smaller: fewer tiles, another split
            x = synth.activations("test-noalloc", f"x-{n_tok}", (n_tok, n_in))
            x = x.astype(np.float16).astype(np.float32)   # config 3: f16-valued activations
            groups = [-(-n_out // 128), 1, -(-n_tok // E.MATMUL_TILE_COLS)]
            s.set_x(x)
            s.set_y(np.full((n_tok, n_out), np.nan, np.float32))
            ctx.time_dispatch(p, groups, push, 1)
            want = s.y(n_tok, n_out)
            s.set_y(np.full((n_tok, n_out), np.nan, np.float32))
            ctx.dispatch_noalloc(p, groups, push)
            got = s.y(n_tok, n_out)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n_tok
            ref = so.matmul(int(E.DType.Q4K), data, n_in, n_out, x)
            assert rel_l2(got, ref) <= 3e-3, (n_tok, rel_l2(got, ref))
    finally:
        p.free()
        s.free()


def test_dispatch_noalloc_without_workspace(ctx):
    """A matvec (its kernels use no workspace) through the allocation-free entry point."""
    n_in, n_out = 4096, 1000
    data = synth.matrix("test-noalloc", "mv", E.DType.Q4K, n_in, n_out)
    x = synth.activations("test-noalloc", "x-mv", n_in)
    s = Setup(ctx, [(E.DType.Q4K, n_in, n_out, data)], n_in, n_out)
    m = s.q[0]
    try:
        s.set_x(x)
        s.matvec(0)
        want = s.y(1, n_out)[0]
        assert m.buf == 0                 # set 0 of the pipeline binds this weight buffer
        p = s.k.matvec(m.dtype, False).pipeline(False)
        s.set_y(np.zeros(n_out, np.float32))
        push = [m.off[0], m.off[1], s.x_off, s.y_off, n_in, n_out, 0, 0, 0]
        ctx.dispatch_noalloc(p, [-(-n_out // 8), 1, 1], push)
        got = s.y(1, n_out)[0]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        s.free()
