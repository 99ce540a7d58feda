"""GPU check of launch fusion: consecutive dispatches of one matvec pipeline with no barrier
between them (independent by the engine's contract, graph.rs:23-34) replay as one launch
over their combined rows.  The fused replay must give the same bits as one launch per
dispatch (tactic fuse=0) and stay within the oracle bar."""
import numpy as np
import pytest

from helpers import Setup, rel_l2, tactics
from oracle import skyla_oracle as so
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu

CASES = [
    (E.DType.Q4K, 1024, [64, 37, 200, 8, 129]),
    (E.DType.Q6K, 768, [48, 1, 96, 33, 17]),
    (E.DType.Q8_0, 256, [70, 13, 256, 5, 40]),
]


def _record(s, ms, accum, fuse):
    with tactics(fuse=1 if fuse else 0):
        def body(r):
            g = E.Graph(r, s.k, None, None, False)
            for i, m in enumerate(ms):
                g.matvec(m, (s.x_off, 0), (s.y_off + i * s.s_out, 0), accum, False)
            r.barrier()
        return s.ctx.record(False, body)


@pytest.mark.parametrize("dtype,n_in,outs", CASES)
@pytest.mark.parametrize("accum", [False, True])
def test_fused_launch_matches_separate_launches(ctx, dtype, n_in, outs, accum):
    datas = [synth.matrix("test-fusion", f"{dtype.name}-{i}", dtype, n_in, n) for i, n in enumerate(outs)]
    s = Setup(ctx, [(dtype, n_in, n, d) for n, d in zip(outs, datas)], n_in, max(outs), rows=len(outs))
    try:
        x = synth.activations("test-fusion", f"x-{n_in}", n_in)
        y0 = synth.activations("test-fusion", "y0", (len(outs), s.s_out))
        results = {}
        for fuse in (False, True):
            s.set_x(x)
            s.set_y(y0)
            rec = _record(s, s.q, accum, fuse)
            try:
                assert len(rec) == len(outs)
                results[fuse] = (rec.launches(), None)
                ctx.replay(rec)
            finally:
                rec.free()
            results[fuse] = (results[fuse][0], s.y(len(outs), s.s_out))
        assert results[False][0] == len(outs)
        assert results[True][0] == -(-len(outs) // 4)       # runs of at most 4 per launch
        assert np.array_equal(results[True][1].view(np.uint32), results[False][1].view(np.uint32))
        got = results[True][1]
        for i, (n, d) in enumerate(zip(outs, datas)):
            want = so.matvec(int(dtype), d, n_in, n, x).astype(np.float64)
            part = got[i, :n].astype(np.float64) - (y0[i, :n] if accum else 0.0)
            assert rel_l2(part, want) < 1e-5, (i, n)
            assert np.array_equal(got[i, n:], y0[i, n:])        # rows past n_out untouched
    finally:
        s.free()


def test_barrier_and_other_pipelines_split_runs(ctx):
    """A barrier, or a dispatch of another pipeline, ends a fused run."""
    n_in = 512
    mats = [(E.DType.Q4K, n_in, 32, synth.matrix("test-fusion", f"split-{i}", E.DType.Q4K, n_in, 32))
            for i in range(4)]
    s = Setup(ctx, mats, n_in, 32, rows=4)
    try:
        def body(r):
            g = E.Graph(r, s.k, None, None, False)
            g.matvec(s.q[0], (s.x_off, 0), (s.y_off, 0), False, False)
            g.matvec(s.q[1], (s.x_off, 0), (s.y_off + s.s_out, 0), False, False)
            r.barrier()
            g.matvec(s.q[2], (s.x_off, 0), (s.y_off + 2 * s.s_out, 0), False, False)
            g.matvec(s.q[3], (s.x_off, 0), (s.y_off + 3 * s.s_out, 0), True, False)   # ACCUM pipeline
        rec = ctx.record(False, body)
        try:
            assert len(rec) == 4 and rec.launches() == 3
        finally:
            rec.free()
    finally:
        s.free()


@pytest.mark.parametrize("dtype,n_in,n_out", [(E.DType.Q4K, 4096, 8192), (E.DType.Q6K, 12288, 512),
                                              (E.DType.Q6K, 1024, 12288)])
@pytest.mark.parametrize("accum", [False, True])
def test_variant_choice_matches_requested_variant(ctx, dtype, n_in, n_out, accum):
    """Large dense launches run on the variant the runtime picks for their size; the result
    equals the engine-requested variant's up to f32 summation order, and the oracle."""
    data = synth.matrix("test-fusion", f"retile-{dtype.name}-{n_in}-{n_out}", dtype, n_in, n_out)
    x = synth.activations("test-fusion", f"rx-{n_in}", n_in)
    y0 = synth.activations("test-fusion", f"ry-{n_out}", n_out)
    got = {}
    for retile in ("0", "1"):
        with tactics(retile=retile):
            s = Setup(ctx, [(dtype, n_in, n_out, data)], n_in, n_out)
        try:
            s.set_x(x)
            s.set_y(y0)
            s.matvec(0, accum)
            got[retile] = s.y(1, n_out)[0].astype(np.float64)
        finally:
            s.free()
    assert rel_l2(got["1"], got["0"]) < 1e-5
    want = so.matvec(int(dtype), data, n_in, n_out, x).astype(np.float64)
    assert rel_l2(got["1"] - (y0 if accum else 0.0), want) < 1e-5
