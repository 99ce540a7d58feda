"""GPU parity of the decode matvec and the bit-exact dequantisation (through the C-ABI).

Bar: dequantised weights bit-exact against the oracle (quant.rs restated); matvec within
1e-2 relative L2 of the oracle's f32 Matrix::matvec and, since
the kernels multiply f32 activations by the exact quants in f32 as the reference does,
within twice what a plain f32 reordering of the same product gives (f32_reorder_bar,
about 1.5e-6 to 2.5e-6 at the Qwen3-8B shapes).
"""
import numpy as np
import pytest

from helpers import F32_FLOOR, Setup, f32_reorder_bar, pad64, rel_l2, tactics
from oracle import skyla_oracle as so
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu

TOL = 1e-2
F32 = 1e-5     # f32 arithmetic, where the product is composed with other f32 work (norm, SiLU)


def _dequant_gpu(ctx, dtype, n_in, n_out, data):
    s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out, extra_f32=n_in * n_out)
    try:
        m = s.q[0]
        ty = {E.DType.Q8_0: 0, E.DType.Q4K: 1, E.DType.Q6K: 2}[dtype]
        p = ctx.create_pipeline("dequant", 3, 28, [ty])
        p.bind_buffers([s.weights[0], s.weights[0], s.arena])
        groups = n_out * n_in // 32
        push = [m.off[0], m.off[1], m.off[2], m.off[3], n_in, n_out, s.extra_off]
        rec = ctx.record(False, lambda r: r.dispatch(p, [-(-groups // 256), 1, 1], push))
        ctx.replay(rec)
        rec.free()
        p.free()
        s.arena.download()
        return s.arena.as_f32()[s.extra_off: s.extra_off + n_in * n_out].copy()
    finally:
        s.free()


@pytest.mark.parametrize("dtype,n_in,n_out", [
    (E.DType.Q4K, 512, 48), (E.DType.Q6K, 512, 48), (E.DType.Q8_0, 96, 40), (E.DType.Q4K, 4096, 8),
])
def test_dequant_bit_exact(ctx, dtype, n_in, n_out):
    data = synth.matrix("test-dequant", f"{dtype.name}", dtype, n_in, n_out)
    got = _dequant_gpu(ctx, dtype, n_in, n_out, data)
    want = so.dequantize(int(dtype), data, n_in * n_out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


SMALL = [
    (E.DType.Q4K, 256, 1), (E.DType.Q4K, 512, 37), (E.DType.Q4K, 2304, 64), (E.DType.Q4K, 768, 9),
    (E.DType.Q6K, 256, 1), (E.DType.Q6K, 512, 37), (E.DType.Q6K, 2304, 64), (E.DType.Q6K, 512, 256),
    (E.DType.Q6K, 512, 1024), (E.DType.Q6K, 1024, 256),
    (E.DType.Q8_0, 32, 1), (E.DType.Q8_0, 96, 13), (E.DType.Q8_0, 1024, 70),
]


@pytest.mark.parametrize("dtype,n_in,n_out", SMALL)
@pytest.mark.parametrize("accum", [False, True])
def test_matvec_small(ctx, dtype, n_in, n_out, accum):
    data = synth.matrix("test-matvec", f"{dtype.name}-{n_in}-{n_out}", dtype, n_in, n_out)
    x = synth.activations("test-matvec", f"x-{n_in}", n_in)
    y0 = synth.activations("test-matvec", f"y0-{n_out}", n_out) if accum else np.zeros(n_out, np.float32)
    s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out)
    try:
        s.set_x(x)
        s.set_y(y0)
        s.matvec(0, accum)
        got = s.y(1, n_out)[0]
    finally:
        s.free()
    want = so.matvec(int(dtype), data, n_in, n_out, x)
    # ACCUM adds y0 on the GPU; judge the matvec part (y0 + dot may cancel)
    err = rel_l2(got - y0, want)
    bar = f32_reorder_bar(dtype, data, n_in, n_out, x, want) + (4e-7 if accum else 0.0)
    assert err <= bar, (err, bar)


@pytest.mark.parametrize("tactic", [(1, 1), (1, 2), (2, 2), (2, 4), (4, 1), (4, 2), (4, 4), (8, 1), (8, 2)])
def test_matvec_tactics(ctx, tactic):
    """Every instantiated (waves, rows) tactic covers every row exactly once."""
    n_in, n_out = 1024, 301
    mats = [(E.DType.Q4K, n_in, n_out, synth.matrix("tac", "q4k", E.DType.Q4K, n_in, n_out)),
            (E.DType.Q6K, n_in, n_out, synth.matrix("tac", "q6k", E.DType.Q6K, n_in, n_out)),
            (E.DType.Q8_0, n_in, n_out, synth.matrix("tac", "q8", E.DType.Q8_0, n_in, n_out))]
    x = synth.activations("tac", "x", n_in)
    s = Setup(ctx, mats, n_in, n_out, kquant_tactic=tactic, q8_0_tactic=tactic)
    try:
        s.set_x(x)
        for i, (dt, _, _, data) in enumerate(mats):
            s.set_y(np.full(n_out, np.nan, np.float32))
            s.matvec(i)
            got = s.y(1, n_out)[0]
            want = so.matvec(int(dt), data, n_in, n_out, x)
            assert rel_l2(got, want) <= f32_reorder_bar(dt, data, n_in, n_out, x, want), (dt, tactic)
    finally:
        s.free()


# config 2: the Qwen3-8B decode shapes
QWEN3_8B = [
    ("q", E.DType.Q4K, 4096, 4096), ("k", E.DType.Q4K, 4096, 1024), ("o", E.DType.Q4K, 4096, 4096),
    ("gate", E.DType.Q4K, 4096, 12288), ("down", E.DType.Q6K, 12288, 4096),
    ("down_q4k", E.DType.Q4K, 12288, 4096),
]


@pytest.mark.parametrize("name,dtype,n_in,n_out", QWEN3_8B)
def test_matvec_qwen3_8b_shapes(ctx, name, dtype, n_in, n_out):
    data = synth.matrix("qwen3-8b", name, dtype, n_in, n_out)
    x = synth.activations("qwen3-8b", f"x-{n_in}", n_in)
    s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out)
    try:
        s.set_x(x)
        s.matvec(0)
        got = s.y(1, n_out)[0]
    finally:
        s.free()
    want = so.matvec(int(dtype), data, n_in, n_out, x)
    err = rel_l2(got, want)
    bar = f32_reorder_bar(dtype, data, n_in, n_out, x, want)
    print(f"{name}: rel-L2 {err:.3e}, plain f32 reordering bar {bar:.3e}")
    assert err <= TOL and err <= bar, (err, bar)


def test_matvec_linearity_full_size(ctx):
    """Size-independent property at the full gate shape: A(x1 + x2) = A x1 + A x2."""
    dtype, n_in, n_out = E.DType.Q4K, 4096, 12288
    data = synth.matrix("qwen3-8b", "gate", dtype, n_in, n_out)
    x1 = synth.activations("lin", "x1", n_in)
    x2 = synth.activations("lin", "x2", n_in)
    s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out)
    try:
        outs = []
        for x in (x1, x2, x1 + x2):
            s.set_x(x)
            s.matvec(0)
            outs.append(s.y(1, n_out)[0].astype(np.float64))
    finally:
        s.free()
    assert rel_l2(outs[2], outs[0] + outs[1]) <= 4 * F32_FLOOR


@pytest.mark.parametrize("dtype,n_in,n_out", [
    (E.DType.Q4K, 4096, 301), (E.DType.Q4K, 12288, 4096), (E.DType.Q6K, 2304, 64),
    (E.DType.Q6K, 12288, 4096), (E.DType.Q8_0, 1024, 70), (E.DType.Q8_0, 3072, 301),
])
def test_matvec_large_activations(ctx, dtype, n_in, n_out):
    """Activations past the f16 range (silu(gate) * up reaches 1e5-1e6 in real checkpoints):
    multiplied in f32, as the reference does, with the same f32 bar."""
    data = synth.matrix("test-big", f"{dtype.name}-{n_in}-{n_out}", dtype, n_in, n_out)
    x = synth.activations("test-big", f"x-{n_in}", n_in)
    x[: n_in // 3] *= np.float32(3e5)
    x[n_in // 2] = np.float32(-1.5e6)
    x[n_in - 1] = np.float32(70000.0)
    s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out)
    try:
        s.set_x(x)
        s.matvec(0)
        got = s.y(1, n_out)[0]
    finally:
        s.free()
    want = so.matvec(int(dtype), data, n_in, n_out, x)
    assert np.isfinite(got).all()
    err = rel_l2(got, want)
    assert err <= f32_reorder_bar(dtype, data, n_in, n_out, x, want), err


FUSED = [(E.DType.Q4K, 4096, 301), (E.DType.Q4K, 4096, 6144), (E.DType.Q4K, 12288, 4096),
         (E.DType.Q6K, 4096, 301), (E.DType.Q6K, 4096, 12288), (E.DType.Q6K, 12288, 4096),
         (E.DType.Q8_0, 1024, 70)]


@pytest.mark.parametrize("retile", ["1", "0"])
@pytest.mark.parametrize("form", ["norm", "silu"])
@pytest.mark.parametrize("dtype,n_in,n_out", FUSED)
def test_fused_matvec_forms(ctx, dtype, n_in, n_out, form, retile):
    """The decode matvecs with the RMSNorm before them (matvec_*_norm: y = A rmsnorm(x, w))
    and with the SiLU gate of the down projection (matvec_*_silu: y += A (silu(g) * u))
    against the oracle's rmsnorm / silu then Matrix::matvec; every size variant the runtime
    may pick (retile on) and the engine's own tactic (retile off)."""
    g = synth.rng("test-fused", f"{dtype.name}-{n_in}-{n_out}-{form}")
    data = synth.matrix("test-fused", f"{dtype.name}-{n_in}-{n_out}", dtype, n_in, n_out)
    x = (g.standard_normal(n_in) * 3).astype(np.float32)
    if form == "norm":
        aux = g.uniform(0.5, 1.5, n_in).astype(np.float32)
        y0 = np.zeros(n_out, np.float32)
    else:
        aux = g.standard_normal(n_in).astype(np.float32)
        aux[: n_in // 8] *= np.float32(2e4)   # silu(g) * u past the f16 range, as in real checkpoints
        y0 = g.standard_normal(n_out).astype(np.float32)
    c = E.Config(n_embd=n_in, eps=1e-6)
    with tactics(retile=retile):
        s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out, extra_f32=n_in)
        k = E.Kernels(ctx, s.weights, s.arena, fuse="all")
    try:
        s.arena.as_f32()[s.extra_off: s.extra_off + n_in] = aux
        s.set_x(x)
        s.set_y(y0)
        s.run(lambda r: E.Graph(r, k, None, c, False).matvec(
            s.q[0], (s.x_off, 0), (s.y_off, 0), form == "silu", False, form=form, aux=s.extra_off))
        got = s.y(1, n_out)[0]
    finally:
        s.free()
    if form == "norm":
        xin = so.rmsnorm(x, aux, c.eps)
    else:
        xin = (x / (np.float32(1) + np.exp(-x)) * aux).astype(np.float32)
    want = so.matvec(int(dtype), data, n_in, n_out, xin)
    assert np.isfinite(got).all()
    err = rel_l2(got - y0, want)
    assert err <= F32, err


@pytest.mark.parametrize("ks", ["1", "4_1", "4_3", "0"])
@pytest.mark.parametrize("big", [False, True])
@pytest.mark.parametrize("n_in,n_out", [(4096, 12288), (4096, 1000), (1024, 1536), (2048, 100)])
def test_glu_norm_pair_against_oracle(ctx, n_in, n_out, big, ks):
    """matvec_q4k_glun (the gate/up pair with the FFN RMSNorm folded in, from the raw
    residual) against the oracle's rmsnorm, the two Matrix::matvec and silu * up; `big`
    puts an eighth of the residual past the f16 range (3e4 to 1e5).  With n_in 4096 the
    runtime runs the K-split pair form (its default shape, or tactic ksglun=4_1), with
    ksglun=0 and for other widths the LDS-staged one; n_out 1000 leaves a ragged
    last workgroup."""
    g = synth.matrix("test-glu", f"gate-{n_in}-{n_out}", E.DType.Q4K, n_in, n_out)
    u = synth.matrix("test-glu", f"up-{n_in}-{n_out}", E.DType.Q4K, n_in, n_out)
    rg = synth.rng("test-glu", f"norm-{n_in}-{big}")
    x = (rg.standard_normal(n_in) * 3).astype(np.float32)
    if big:
        x[: n_in // 8] *= np.float32(3e4)
    w = rg.uniform(0.5, 1.5, n_in).astype(np.float32)
    eps = 1e-6
    s = Setup(ctx, [(E.DType.Q4K, n_in, n_out, g), (E.DType.Q4K, n_in, n_out, u)], n_in, n_out, extra_f32=n_in)
    with tactics(ksglun=ks):
        k = E.Kernels(ctx, s.weights, s.arena, fuse="ffn")
    try:
        s.arena.as_f32()[s.extra_off: s.extra_off + n_in] = w
        s.set_x(x)
        gq, uq = s.q
        push = [gq.off[0], gq.off[1], s.x_off, s.y_off, n_in, n_out, 0, 0, 0, uq.off[0], uq.off[1], s.extra_off,
                E.f32_bits(eps)]
        s.run(lambda r: r.dispatch_set(k.glu_norm, gq.buf, [-(-n_out // 16), 1, 1], push))
        got = s.y(1, n_out)[0]
    finally:
        s.free()
    n = so.rmsnorm(x, w, np.float32(eps))
    gg = so.matvec(int(E.DType.Q4K), g, n_in, n_out, n).astype(np.float64)
    uu = so.matvec(int(E.DType.Q4K), u, n_in, n_out, n).astype(np.float64)
    want = gg / (1.0 + np.exp(-gg)) * uu
    assert np.isfinite(got).all()
    assert rel_l2(got, want) <= F32, rel_l2(got, want)


@pytest.mark.parametrize("n_in,n_out", [(4096, 12288), (4096, 4096), (1024, 1536), (2048, 100)])
def test_glu_pair_equals_gate_up_then_silu(ctx, n_in, n_out):
    """matvec_q4k_glu (gate and up in one launch writing silu(gate) * up) against the two
    matvecs and silu_mul on the same device: bit for bit where both run the 16-lane rows."""
    g = synth.matrix("test-glu", f"gate-{n_in}-{n_out}", E.DType.Q4K, n_in, n_out)
    u = synth.matrix("test-glu", f"up-{n_in}-{n_out}", E.DType.Q4K, n_in, n_out)
    x = synth.activations("test-glu", f"x-{n_in}", n_in)
    s = Setup(ctx, [(E.DType.Q4K, n_in, n_out, g), (E.DType.Q4K, n_in, n_out, u)], n_in, n_out,
              extra_f32=2 * pad64(n_out))
    k = E.Kernels(ctx, s.weights, s.arena, fuse="qkv")
    try:
        s.set_x(x)
        gq, uq = s.q
        assert gq.buf == uq.buf
        go, uo = s.extra_off, s.extra_off + pad64(n_out)

        def fused(r):
            push = [gq.off[0], gq.off[1], s.x_off, s.y_off, n_in, n_out, 0, 0, 0, uq.off[0], uq.off[1]]
            r.dispatch_set(k.glu, gq.buf, [-(-n_out // 16), 1, 1], push)

        def plain(r):
            gr = E.Graph(r, k, None, E.Config(n_embd=n_in), False)
            gr.matvec(gq, (s.x_off, 0), (go, 0), False, False)
            gr.matvec(uq, (s.x_off, 0), (uo, 0), False, False)
            r.barrier()
            r.dispatch(k.silu, [-(-n_out // 256), 1, 1], [go, uo, n_out, 0])
        s.run(fused)
        s.run(plain)
        s.arena.download()
        f = s.arena.as_f32()
        got, want = f[s.y_off: s.y_off + n_out].copy(), f[go: go + n_out].copy()
    finally:
        s.free()
    assert np.isfinite(got).all()
    # plain Q4_K launches with n_in 4096 run the K-split form; the pair takes it below 8192
    # outputs (the runtime's K-split rules) and the LDS-staged pair form above
    if n_in == 4096 and n_out < 8192:  # the same K-split sums on both sides
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:                              # another lane split of the same sums
        assert rel_l2(got, want) <= 1e-5


KS_SHAPES = ["2_1", "2_2", "4_1", "4_2", "4_3", "4_6", "8_1", "8_3"]


@pytest.mark.parametrize("shape", KS_SHAPES)
@pytest.mark.parametrize("accum", [False, True])
def test_ks_shapes_against_oracle(ctx, shape, accum):
    """Every compiled shape of the K-split Q4_K form (n_in = 4096; tactic ks=R_G forces one)
    over three fused segments whose row counts are not multiples of its workgroup (q, k, v
    of 4096 + 333 + 1), ACCUM on and off, against the oracle at the f32 bar; rows past
    n_out stay untouched."""
    n_in, outs = 4096, [4096, 333, 1]
    datas = [synth.matrix("test-ks", f"{i}-{n}", E.DType.Q4K, n_in, n) for i, n in enumerate(outs)]
    x = synth.activations("test-ks", "x", n_in)
    with tactics(ks=shape):
        s = Setup(ctx, [(E.DType.Q4K, n_in, n, d) for n, d in zip(outs, datas)], n_in, max(outs), rows=len(outs))
    try:
        y0 = synth.activations("test-ks", "y0", (len(outs), s.s_out))
        s.set_x(x)
        s.set_y(y0)

        def body(r):
            g = E.Graph(r, s.k, None, None, False)
            for i, m in enumerate(s.q):
                g.matvec(m, (s.x_off, 0), (s.y_off + i * s.s_out, 0), accum, False)
        rec = ctx.record(False, body)
        try:
            assert rec.launches() == 1           # the three dispatches run as one launch
            ctx.replay(rec)
        finally:
            rec.free()
        got = s.y(len(outs), s.s_out)
    finally:
        s.free()
    for i, (n, d) in enumerate(zip(outs, datas)):
        want = so.matvec(int(E.DType.Q4K), d, n_in, n, x)
        part = got[i, :n].astype(np.float64) - (y0[i, :n] if accum else 0.0)
        bar = f32_reorder_bar(E.DType.Q4K, d, n_in, n, x, want) + (4e-7 if accum else 0.0)
        assert rel_l2(part, want) <= bar, (shape, i, rel_l2(part, want), bar)
        assert np.array_equal(got[i, n:], y0[i, n:])        # rows past n_out untouched


def test_ks_shapes_same_bits(ctx):
    """A row's K-split sum does not depend on the shape that computes it: every compiled
    (rows per slot, row-groups) shape, and the default size rule (a fused gate+up launch of
    2 x 12288 rows on its own shape), give the same bits."""
    n_in, outs = 4096, [12288, 12288]
    datas = [synth.matrix("test-ks-bits", f"{i}", E.DType.Q4K, n_in, n) for i, n in enumerate(outs)]
    x = synth.activations("test-ks-bits", "x", n_in)
    got = {}
    for shape in [None] + KS_SHAPES:
        with tactics(ks=shape):
            s = Setup(ctx, [(E.DType.Q4K, n_in, n, d) for n, d in zip(outs, datas)], n_in, max(outs), rows=2)
        try:
            s.set_x(x)

            def body(r):
                g = E.Graph(r, s.k, None, None, False)
                for i, m in enumerate(s.q):
                    g.matvec(m, (s.x_off, 0), (s.y_off + i * s.s_out, 0), False, False)
            rec = ctx.record(False, body)
            try:
                assert rec.launches() == 1
                ctx.replay(rec)
            finally:
                rec.free()
            got[shape] = s.y(2, s.s_out)[:, :12288].copy()
        finally:
            s.free()
    for shape, y in got.items():
        assert np.array_equal(y.view(np.uint32), got[None].view(np.uint32)), shape


KS6_SHAPES = ["1_8_1", "1_8_2", "1_8_7", "1_16_2", "2_4_2", "8_1_1"]


@pytest.mark.parametrize("shape", KS6_SHAPES)
@pytest.mark.parametrize("accum", [False, True])
def test_ks6_shapes_against_oracle(ctx, shape, accum):
    """Every compiled shape of the K-split Q6_K form (n_in = 12288; tactic ks6=R_G_D forces one)
    over three fused segments whose row counts are not multiples of its workgroup (4096 +
    333 + 1), ACCUM on and off, against the oracle at the f32 bar; rows past n_out stay
    untouched."""
    n_in, outs = 12288, [4096, 333, 1]
    datas = [synth.matrix("test-ks6", f"{i}-{n}", E.DType.Q6K, n_in, n) for i, n in enumerate(outs)]
    x = synth.activations("test-ks6", "x", n_in)
    with tactics(ks6=shape):
        s = Setup(ctx, [(E.DType.Q6K, n_in, n, d) for n, d in zip(outs, datas)], n_in, max(outs), rows=len(outs))
    try:
        y0 = synth.activations("test-ks6", "y0", (len(outs), s.s_out))
        s.set_x(x)
        s.set_y(y0)

        def body(r):
            g = E.Graph(r, s.k, None, None, False)
            for i, m in enumerate(s.q):
                g.matvec(m, (s.x_off, 0), (s.y_off + i * s.s_out, 0), accum, False)
        rec = ctx.record(False, body)
        try:
            assert rec.launches() == 1           # the three dispatches run as one launch
            ctx.replay(rec)
        finally:
            rec.free()
        got = s.y(len(outs), s.s_out)
    finally:
        s.free()
    for i, (n, d) in enumerate(zip(outs, datas)):
        want = so.matvec(int(E.DType.Q6K), d, n_in, n, x)
        part = got[i, :n].astype(np.float64) - (y0[i, :n] if accum else 0.0)
        bar = f32_reorder_bar(E.DType.Q6K, d, n_in, n, x, want) + (4e-7 if accum else 0.0)
        assert rel_l2(part, want) <= bar, (shape, i, rel_l2(part, want), bar)
        assert np.array_equal(got[i, n:], y0[i, n:])        # rows past n_out untouched


KS3_SHAPES = ["2_1", "2_2", "4_1"]


@pytest.mark.parametrize("shape", KS3_SHAPES)
@pytest.mark.parametrize("accum", [False, True])
def test_ks3_shapes_against_oracle(ctx, shape, accum):
    """Every compiled shape of the K-split Q4_K form for n_in = 12288 (three 4096-value parts
    per row; tactic ks3=R_G forces one) over three fused segments whose row counts are not
    multiples of its workgroup (4096 + 333 + 1), ACCUM on and off, against the oracle at the
    f32 bar; rows past n_out stay untouched."""
    n_in, outs = 12288, [4096, 333, 1]
    datas = [synth.matrix("test-ks3", f"{i}-{n}", E.DType.Q4K, n_in, n) for i, n in enumerate(outs)]
    x = synth.activations("test-ks3", "x", n_in)
    with tactics(ks3=shape):
        s = Setup(ctx, [(E.DType.Q4K, n_in, n, d) for n, d in zip(outs, datas)], n_in, max(outs), rows=len(outs))
    try:
        y0 = synth.activations("test-ks3", "y0", (len(outs), s.s_out))
        s.set_x(x)
        s.set_y(y0)

        def body(r):
            g = E.Graph(r, s.k, None, None, False)
            for i, m in enumerate(s.q):
                g.matvec(m, (s.x_off, 0), (s.y_off + i * s.s_out, 0), accum, False)
        rec = ctx.record(False, body)
        try:
            assert rec.launches() == 1           # the three dispatches run as one launch
            ctx.replay(rec)
        finally:
            rec.free()
        got = s.y(len(outs), s.s_out)
    finally:
        s.free()
    for i, (n, d) in enumerate(zip(outs, datas)):
        want = so.matvec(int(E.DType.Q4K), d, n_in, n, x)
        part = got[i, :n].astype(np.float64) - (y0[i, :n] if accum else 0.0)
        bar = f32_reorder_bar(E.DType.Q4K, d, n_in, n, x, want) + (4e-7 if accum else 0.0)
        assert rel_l2(part, want) <= bar, (shape, i, rel_l2(part, want), bar)
        assert np.array_equal(got[i, n:], y0[i, n:])        # rows past n_out untouched


@pytest.mark.parametrize("ks3", ["2_2", "0"])
def test_q4k_mixed_widths_in_one_launch(ctx, ks3):
    """A fused launch whose segments have n_in 12288 and 4096 fits neither K-split form (each
    needs every segment at its width): it runs the LDS-staged variant, within the bar; with
    the ks3 tactic off, a 12288-wide launch alone does too."""
    shapes = [(12288, 300), (4096, 77)]
    datas = [synth.matrix("test-ks3", f"mixed-{n_in}", E.DType.Q4K, n_in, n) for n_in, n in shapes]
    x = synth.activations("test-ks3", "x-mixed", 12288)
    with tactics(ks3=ks3):
        s = Setup(ctx, [(E.DType.Q4K, n_in, n, d) for (n_in, n), d in zip(shapes, datas)], 12288, 300,
                  rows=len(shapes))
    try:
        s.set_x(x)
        s.set_y(np.zeros((len(shapes), s.s_out), np.float32))

        def body(r):
            g = E.Graph(r, s.k, None, None, False)
            for i, m in enumerate(s.q):
                g.matvec(m, (s.x_off, 0), (s.y_off + i * s.s_out, 0), False, False)
        rec = ctx.record(False, body)
        try:
            assert rec.launches() == 1
            ctx.replay(rec)
        finally:
            rec.free()
        got = s.y(len(shapes), s.s_out)
    finally:
        s.free()
    for i, ((n_in, n), d) in enumerate(zip(shapes, datas)):
        xi = x[:n_in]
        want = so.matvec(int(E.DType.Q4K), d, n_in, n, xi)
        assert rel_l2(got[i, :n], want) <= f32_reorder_bar(E.DType.Q4K, d, n_in, n, xi, want), (i, ks3)


def test_ks6_other_widths_keep_their_variant(ctx):
    """The K-split Q6_K form serves n_in = 12288 only: a forced shape leaves a launch of
    another width (n_in 1024) on the LDS-staged variant, and the result stays in the bar."""
    n_in, n_out = 1024, 301
    data = synth.matrix("test-ks6", "narrow", E.DType.Q6K, n_in, n_out)
    x = synth.activations("test-ks6", "x-narrow", n_in)
    with tactics(ks6="1_8_2"):
        s = Setup(ctx, [(E.DType.Q6K, n_in, n_out, data)], n_in, n_out)
    try:
        s.set_x(x)
        s.set_y(np.full(n_out, np.nan, np.float32))
        s.matvec(0)
        got = s.y(1, n_out)[0]
    finally:
        s.free()
    want = so.matvec(int(E.DType.Q6K), data, n_in, n_out, x)
    assert rel_l2(got, want) <= f32_reorder_bar(E.DType.Q6K, data, n_in, n_out, x, want)


def test_q8_0_head_variant(ctx):
    """Config 1's tied output head (Q8_0 1024 -> 151936): dense Q8_0 launches of 65536 rows or
    more run the (4, 1, 16) variant (tactic q8_big), within the f32 reordering bar of the
    oracle, as the engine's own variant (q8_big empty) is; the two sum in different orders."""
    n_in, n_out = 1024, 151936
    data = synth.matrix("q8-head", "head", E.DType.Q8_0, n_in, n_out)
    x = synth.activations("q8-head", "x", n_in)
    got = {}
    for v in ("4_1_16", ""):
        with tactics(q8_big=v):
            s = Setup(ctx, [(E.DType.Q8_0, n_in, n_out, data)], n_in, n_out)
            try:
                s.set_x(x)
                s.matvec(0)
                got[v] = s.y(1, n_out)[0].copy()
            finally:
                s.free()
    want = so.matvec(int(E.DType.Q8_0), data, n_in, n_out, x)
    bar = f32_reorder_bar(E.DType.Q8_0, data, n_in, n_out, x, want)
    for v, g in got.items():
        assert rel_l2(g, want) <= bar, (v, rel_l2(g, want), bar)
    assert not np.array_equal(got["4_1_16"], got[""])

