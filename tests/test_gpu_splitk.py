"""GPU check of the K split the runtime applies to dense K-quant matmul launches with few
tiles: the launch runs the split kernel (partials in a recording-owned workspace, summed in
split order by the last workgroup of each tile), and must agree with the single-pass kernel
up to f32 summation order and with the oracle to the matmul bar.  Replaying the recording
again must give the same bits (the per-tile counters are left at zero by every launch)."""

import numpy as np
import pytest

from helpers import Setup, rel_l2, tactics
from oracle import skyla_oracle as so
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu

GUARD = 3e-3


def _run(ctx, dtype, n_in, n_out, n_tok, accum, x_half, split, replays):
    data = synth.matrix("mm-split", f"{dtype.name}-{n_in}-{n_out}", dtype, n_in, n_out)
    x = synth.activations("mm-split", f"x-{n_tok}-{n_in}", (n_tok, n_in))
    if x_half:
        x = x.astype(np.float16).astype(np.float32)
    y0 = synth.activations("mm-split", f"y0-{n_tok}-{n_out}", (n_tok, n_out))
    s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out, rows=n_tok)
    with tactics(splitk=split):
        m = s.q[0]
        ty = {E.DType.Q4K: 1, E.DType.Q6K: 2}[dtype]
        p = ctx.create_pipeline("matmul", 5, 52, [ty, int(accum), 0] + ([1] if x_half else []))
    outs = []
    try:
        w = s.weights[m.buf]
        p.bind_buffers([w, w, s.arena, s.arena, s.arena])
        x_off = 2 * s.half_off if x_half else s.x_off
        push = [m.off[0], m.off[1], m.off[2], m.off[3], x_off, s.y_off, m.n_in, m.n_out, s.s_in, s.s_out, 0, 0, 1]
        grid = [-(-m.n_out // 128), 1, -(-n_tok // E.MATMUL_TILE_COLS)]
        rec = ctx.record(False, lambda r: r.dispatch(p, grid, push))
        try:
            for _ in range(replays):
                s.set_x(x)
                s.set_x_half(x)
                s.set_y(y0)
                ctx.replay(rec)
                outs.append(s.y(n_tok, n_out))
        finally:
            rec.free()
    finally:
        p.free()
        s.free()
    want = so.matmul(int(dtype), data, n_in, n_out, x)
    return [o.astype(np.float64) - (y0 if accum else 0.0) for o in outs], want


@pytest.mark.parametrize("dtype,n_in", [(E.DType.Q4K, 4096), (E.DType.Q6K, 3072)])
@pytest.mark.parametrize("accum", [False, True])
@pytest.mark.parametrize("x_half", [False, True])
def test_k_split_matches_single_pass(ctx, dtype, n_in, accum, x_half):
    # 3 row tiles x 2 token tiles (the second partial): few tiles, so the launch splits K
    n_out, n_tok = 384, 200
    single, want = _run(ctx, dtype, n_in, n_out, n_tok, accum, x_half, "0", 1)
    split, _ = _run(ctx, dtype, n_in, n_out, n_tok, accum, x_half, "1", 3)
    assert all(np.array_equal(o, split[0]) for o in split[1:])   # replays agree bit for bit
    assert not np.array_equal(split[0], single[0])                 # a different summation ran
    assert rel_l2(split[0], single[0]) < 1e-5
    assert rel_l2(split[0], want) <= GUARD
