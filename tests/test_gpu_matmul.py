"""GPU parity of the prefill matmul (MFMA) against the oracle's f32 GEMM (M x matvec).

Bar: 1e-2 relative L2 (north star).  Inputs are f16 activations as in config 3, so the
oracle is fed the same f16-rounded values widened to f32; the remaining difference is the
kernel's f16 weight rounding and accumulation order.
"""
import numpy as np
import pytest

from helpers import Setup, rel_l2
from oracle import skyla_oracle as so
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu

TOL = 1e-2
GUARD = 3e-3


def _run(ctx, dtype, n_in, n_out, n_tok, accum=False, half=True, tag="mm"):
    data = synth.matrix(tag, f"{dtype.name}-{n_in}-{n_out}", dtype, n_in, n_out)
    x = synth.activations(tag, f"x-{n_tok}-{n_in}", (n_tok, n_in)).astype(np.float16).astype(np.float32)
    y0 = synth.activations(tag, f"y0-{n_tok}-{n_out}", (n_tok, n_out)) if accum else None
    s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out, rows=max(n_tok, 1))
    try:
        if half:
            s.set_x_half(x)
        else:
            s.set_x(x)
        if accum:
            s.set_y(y0)
        if half:
            s.matmul(0, n_tok, accum)
        else:
            ty = {E.DType.Q8_0: 0, E.DType.Q4K: 1, E.DType.Q6K: 2}[dtype]
            p = ctx.create_pipeline("matmul", 5, 52, [ty, int(accum), 0])
            w = s.weights[0]
            p.bind_buffers([w, w, s.arena, s.arena, s.arena])
            m = s.q[0]
            push = [m.off[0], m.off[1], m.off[2], m.off[3], s.x_off, s.y_off, n_in, n_out, s.s_in, s.s_out, 0, 0, 1]
            z = -(-n_tok // E.MATMUL_TILE_COLS)
            rec = ctx.record(False, lambda r: r.dispatch(p, [-(-n_out // 128), 1, z], push))
            ctx.replay(rec)
            rec.free()
            p.free()
        got = s.y(n_tok, n_out)
    finally:
        s.free()
    want = so.matmul(int(dtype), data, n_in, n_out, x)
    if accum:  # the GPU added y0; judge the product part
        got = got - y0
    return got, want


@pytest.mark.parametrize("dtype,n_in,n_out,n_tok", [
    (E.DType.Q4K, 256, 128, 64), (E.DType.Q4K, 512, 200, 37), (E.DType.Q4K, 1024, 256, 128),
    (E.DType.Q6K, 256, 128, 64), (E.DType.Q6K, 768, 130, 100),
    (E.DType.Q8_0, 256, 128, 64), (E.DType.Q8_0, 96, 64, 5), (E.DType.Q8_0, 1056, 140, 70),
])
def test_matmul_small(ctx, dtype, n_in, n_out, n_tok):
    got, want = _run(ctx, dtype, n_in, n_out, n_tok)
    assert rel_l2(got, want) <= GUARD


@pytest.mark.parametrize("dtype", [E.DType.Q4K, E.DType.Q6K, E.DType.Q8_0])
def test_matmul_f32_input_and_accum(ctx, dtype):
    got, want = _run(ctx, dtype, 512, 192, 70, accum=True, half=False, tag="mm-f32")
    assert rel_l2(got, want) <= GUARD
    got, want = _run(ctx, dtype, 512, 192, 70, accum=True, half=True, tag="mm-acc")
    assert rel_l2(got, want) <= GUARD


@pytest.mark.parametrize("name,dtype,n_in,n_out", [
    ("q", E.DType.Q4K, 4096, 4096), ("down", E.DType.Q6K, 12288, 4096),
])
def test_matmul_config3(ctx, name, dtype, n_in, n_out):
    """Config 3: M = 512 tokens at the Qwen3-8B shapes."""
    got, want = _run(ctx, dtype, n_in, n_out, 512, tag="qwen3-8b-prefill")
    err = rel_l2(got, want)
    assert err <= TOL and err <= GUARD, err
