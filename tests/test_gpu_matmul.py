"""GPU parity of the prefill matmul (MFMA) against the oracle's f32 GEMM (M x matvec).

Bar: 1e-2 relative L2 (north star); 3e-3 asserted as a regression guard.  The engine path
feeds f32 activations (HALF_INPUTS = false for this backend) which the kernel stages as
f16; the f16-input variant (spec X_HALF = 1) is checked with f16-rounded inputs given to
the oracle as well.
"""
import numpy as np
import pytest

from helpers import Setup, rel_l2, tactics
from oracle import skyla_oracle as so
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu

TOL = 1e-2
GUARD = 3e-3


def _run(ctx, dtype, n_in, n_out, n_tok, accum=False, x_half=None, tag="mm", x=None):
    data = synth.matrix(tag, f"{dtype.name}-{n_in}-{n_out}", dtype, n_in, n_out)
    if x is None:
        x = synth.activations(tag, f"x-{n_tok}-{n_in}", (n_tok, n_in))
    if x_half:
        x = x.astype(np.float16).astype(np.float32)
    y0 = synth.activations(tag, f"y0-{n_tok}-{n_out}", (n_tok, n_out)) if accum else None
    s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out, rows=max(n_tok, 1))
    try:
        s.set_x(x)
        s.set_x_half(x)
        if accum:
            s.set_y(y0)
        if x_half is None:
            s.matmul(0, n_tok, accum)
        else:
            s.matmul_variant(0, n_tok, accum, x_half)
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
@pytest.mark.parametrize("x_half", [False, True])
def test_matmul_variants_and_accum(ctx, dtype, x_half):
    got, want = _run(ctx, dtype, 512, 192, 70, accum=True, x_half=x_half, tag="mm-var")
    assert rel_l2(got, want) <= GUARD


def test_matmul_range_guard_large_activations(ctx):
    """Tokens whose activations exceed f16's range (up to 1e6) in some 256-k stages."""
    n_in, n_out, n_tok = 1024, 256, 70
    x = synth.activations("mm-range", "x", (n_tok, n_in))
    x[3, 300:340] *= 1e6           # stage 1 of token 3
    x[10, :] *= 3e4                # every stage of token 10, some values just above 2^15
    x[64, 1000] = -2.5e5           # token in the second tile, last stage
    got, want = _run(ctx, E.DType.Q4K, n_in, n_out, n_tok, tag="mm-range", x=x)
    assert np.all(np.isfinite(got))
    for t in range(n_tok):
        assert rel_l2(got[t], want[t]) <= GUARD, t


@pytest.mark.parametrize("name,dtype,n_in,n_out", [
    ("q", E.DType.Q4K, 4096, 4096), ("gate", E.DType.Q4K, 4096, 12288), ("down", E.DType.Q6K, 12288, 4096),
])
def test_matmul_config3(ctx, name, dtype, n_in, n_out):
    """Config 3: M = 512 tokens at the Qwen3-8B shapes (f16 activations N(0,1))."""
    got, want = _run(ctx, dtype, n_in, n_out, 512, tag="qwen3-8b-prefill", x_half=True)
    err = rel_l2(got, want)
    assert err <= TOL and err <= GUARD, err
    got, want = _run(ctx, dtype, n_in, n_out, 512, tag="qwen3-8b-prefill")
    err = rel_l2(got, want)
    assert err <= TOL and err <= GUARD, err


@pytest.mark.parametrize("x4d", ["1", "0"])
@pytest.mark.parametrize("name,dtype,n_in,n_out,n_tok,accum", [
    ("q", E.DType.Q4K, 4096, 4096, 512, False), ("gate", E.DType.Q4K, 4096, 12288, 512, False),
    ("down", E.DType.Q6K, 12288, 4096, 512, True), ("ragged", E.DType.Q4K, 1024, 200, 37, True),
    ("ragged6", E.DType.Q6K, 768, 130, 100, False), ("ragged4", E.DType.Q4K, 1024, 20000, 37, True),
])
def test_matmul_f16_prepass_same_bits(ctx, name, dtype, n_in, n_out, n_tok, accum, x4d):
    """The runtime's f16 row prepass (x_half_rows, then the tile on f16 rows: four waves
    unless the launch is K-split; tactic xhalf=4 keeps the four-wave tile's plain grid)
    against the eight-wave tile's own f32 staging (xhalf=0): the same bits while no
    activation reaches 2^15, K split or not, ACCUM or not, ragged rows and token counts.
    Q4_K launches of more than 128 tiles (gate, ragged4) run the four-wave tile with its
    operands loaded straight into LDS, or with tactic dl=0 the register-staged one; the
    K-split launches (q, down) run the 128 x 128 direct-to-LDS tile (dl=1) or the
    register-staged one (dl=0)."""
    with tactics(xhalf=4, dl=x4d):
        got1, want = _run(ctx, dtype, n_in, n_out, n_tok, accum=accum, tag="mm-xh")
    with tactics(xhalf=0):
        got0, _ = _run(ctx, dtype, n_in, n_out, n_tok, accum=accum, tag="mm-xh")
    assert np.array_equal(got1.view(np.uint32), got0.view(np.uint32))
    assert rel_l2(got1, want) <= GUARD


def test_matmul_f16_prepass_shared(ctx):
    """Two matmuls on the same rows with no barrier between them share one prepass and run as
    one launch of two segments (two launches in all, three without the f16 rows), and each
    gives the bits of its own f32-staged launch."""
    n_in, n_tok = 1024, 70
    mats = [(E.DType.Q4K, n_in, n, synth.matrix("mm-xh", f"shared-{n}", E.DType.Q4K, n_in, n)) for n in (256, 384)]
    x = synth.activations("mm-xh", "shared-x", (n_tok, n_in))
    got = {}
    for xh in ("1", "0"):
        with tactics(xhalf=xh):
            s = Setup(ctx, mats, n_in, 384, rows=2 * n_tok)
            try:
                s.set_x(x)
                z = -(-n_tok // E.MATMUL_TILE_COLS)

                def body(r):
                    g = E.Graph(r, s.k, None, None, True)
                    for i, m in enumerate(s.q):
                        g.matvec(m, (s.x_off, s.s_in), (s.y_off + i * n_tok * s.s_out, s.s_out), False, True,
                                 groups_z=z)
                rec = ctx.record(False, body)
                try:
                    launches = rec.launches()
                    ctx.replay(rec)
                finally:
                    rec.free()
                got[xh] = (launches, s.y(2 * n_tok, s.s_out))
            finally:
                s.free()
    assert got["1"][0] == 2 and got["0"][0] == 2
    assert np.array_equal(got["1"][1].view(np.uint32), got["0"][1].view(np.uint32))
    for i, (dt, _, n, d) in enumerate(mats):
        want = so.matmul(int(dt), d, n_in, n, x)
        assert rel_l2(got["1"][1][i * n_tok:(i + 1) * n_tok, :n], want) <= GUARD


CUS = 256  # MI355X: two four-wave workgroups per CU, 512 slots


@pytest.mark.parametrize("name,dtype,n_in,n_out,n_tok,accum,x4d", [
    ("gate", E.DType.Q4K, 4096, 12288, 512, False, "1"), ("gate", E.DType.Q4K, 4096, 12288, 512, False, "0"),
    ("ragged4", E.DType.Q4K, 768, 20000, 200, True, "1"), ("ragged6", E.DType.Q6K, 768, 9000, 500, True, "1"),
])
def test_matmul_balanced_grid(ctx, name, dtype, n_in, n_out, n_tok, accum, x4d):
    """A launch of more tiles than CUs and fewer than the two-per-CU slots runs the four-wave
    tile over a balanced grid: hf = 2 tiles - 512 tiles whole (the same bits as the plain
    grid, tactic xhalf=4) and the rest in two K halves added in order (within f32
    reordering of the plain grid), against the oracle at the bar; ACCUM, ragged rows and
    tokens."""
    with tactics(dl=x4d):
        got, want = _run(ctx, dtype, n_in, n_out, n_tok, accum=accum, tag="mm-bal")
    with tactics(xhalf=4, dl=x4d):
        plain, _ = _run(ctx, dtype, n_in, n_out, n_tok, accum=accum, tag="mm-bal")
    hz = -(-n_tok // E.MATMUL_TILE_COLS)
    tiles = -(-n_out // 128) * hz
    assert CUS < tiles < 2 * CUS
    hf = 2 * tiles - 2 * CUS
    whole_rows = (hf // hz) * 128      # row tiles whose every token tile ran whole
    assert 0 < whole_rows < n_out
    assert np.array_equal(got[:, :whole_rows].view(np.uint32), plain[:, :whole_rows].view(np.uint32))
    assert rel_l2(got[:, whole_rows:], plain[:, whole_rows:]) <= 1e-6
    assert rel_l2(got, want) <= GUARD


@pytest.mark.parametrize("dl", ["1", "0"])
@pytest.mark.parametrize("n_tok", [128, 100])
def test_matmul_segments_qkv(ctx, n_tok, dl):
    """q, k and v of a prefill chunk (Q4_K 4096 -> 4096, 1024, 1024 in one buffer, no barrier
    between them) run as one launch of three segments after the shared f16 row prepass: the
    bits of the three separate launches (tactic fuse=0; the same K split here: at least four
    super-blocks a split, so four ways for all of them), and each within the bar of the
    oracle; on the direct-to-LDS 128 x 128 tile (dl=1) and the register-staged one (dl=0)."""
    n_in = 4096
    outs = [4096, 1024, 1024]
    mats = [(E.DType.Q4K, n_in, n, synth.matrix("mm-seg", f"qkv-{i}-{n}", E.DType.Q4K, n_in, n))
            for i, n in enumerate(outs)]
    x = synth.activations("mm-seg", f"x-{n_tok}", (n_tok, n_in))
    got = {}
    for fuse in ("1", "0"):
        with tactics(fuse=fuse, dl=dl, split_stages=4):
            s = Setup(ctx, mats, n_in, max(outs), rows=len(outs) * n_tok)
            try:
                s.set_x(x)
                z = -(-n_tok // E.MATMUL_TILE_COLS)

                def body(r):
                    g = E.Graph(r, s.k, None, None, True)
                    for i, m in enumerate(s.q):
                        g.matvec(m, (s.x_off, s.s_in), (s.y_off + i * n_tok * s.s_out, s.s_out), False, True,
                                 groups_z=z)
                rec = ctx.record(False, body)
                try:
                    launches = rec.launches()
                    ctx.replay(rec)
                finally:
                    rec.free()
                got[fuse] = (launches, s.y(len(outs) * n_tok, s.s_out))
            finally:
                s.free()
    assert got["1"][0] == 2 and got["0"][0] == 4   # prepass + one fused launch / + three launches
    assert np.array_equal(got["1"][1].view(np.uint32), got["0"][1].view(np.uint32))
    for i, (dt, _, n, d) in enumerate(mats):
        want = so.matmul(int(dt), d, n_in, n, x)
        assert rel_l2(got["1"][1][i * n_tok:(i + 1) * n_tok, :n], want) <= GUARD


def test_matmul_gate_up_one_launch(ctx):
    """Gate and up of a prefill chunk at M = 128 (Q4_K 4096 -> 12288 each on the same f16 rows,
    no barrier between them: 2 x 96 row tiles) run as one launch of two segments split two
    ways (tactic seg_big): the bits of the two separate launches (each also split two ways),
    and within the bar of the oracle over the first 256 rows of each."""
    n_in, n_out, n_tok = 4096, 12288, 128
    mats = [(E.DType.Q4K, n_in, n_out, synth.matrix("mm-gu", f"gu-{i}", E.DType.Q4K, n_in, n_out)) for i in range(2)]
    x = synth.activations("mm-gu", f"x-{n_tok}", (n_tok, n_in))
    got = {}
    for big in ("512", "0"):
        with tactics(seg_big=big):
            s = Setup(ctx, mats, n_in, n_out, rows=2 * n_tok)
            try:
                s.set_x(x)

                def body(r):
                    g = E.Graph(r, s.k, None, None, True)
                    for i, m in enumerate(s.q):
                        g.matvec(m, (s.x_off, s.s_in), (s.y_off + i * n_tok * s.s_out, s.s_out), False, True,
                                 groups_z=1)
                rec = ctx.record(False, body)
                try:
                    launches = rec.launches()
                    ctx.replay(rec)
                finally:
                    rec.free()
                got[big] = (launches, s.y(2 * n_tok, s.s_out))
            finally:
                s.free()
    assert got["512"][0] == 2 and got["0"][0] == 3   # prepass + one launch / + two
    assert np.array_equal(got["512"][1].view(np.uint32), got["0"][1].view(np.uint32))
    rows = 256
    for i, (dt, _, n, d) in enumerate(mats):
        want = so.matmul(int(dt), d[: rows * (n_in // 256) * 144], n_in, rows, x)
        assert rel_l2(got["512"][1][i * n_tok:(i + 1) * n_tok, :rows], want) <= GUARD
