"""GPU checks of the chained decode matvecs (chain.hip, matvec_chain; opt-in with
SKYLA_HIP_CHAIN=1): a run of dependent dense matvec launches (Q4_K n_in 4096, Q6_K n_in
12288) replays as one persistent launch with a grid barrier between stages.

  * Q4_K stages compute exactly the K-split form's arithmetic, so they must give the same
    bits as the unchained replay with every Q4_K launch on the K-split form
    (SKYLA_HIP_KS=4_1);
  * every stage stays within the f32 reorder bar of the oracle applied to the stage's own
    input as the GPU left it (Matrix::matvec, matrix.rs:50-53; accumulating stages add to the
    old values, graph.rs:23-34);
  * the chain leaves its barrier words at zero (SKYLA_HIP_CHAIN_CHECK=1 makes each replay
    check them) and replays give the same bits.
Stages have ragged segments (rows not a multiple of the chunk), up to four segments, and
fewer chunks than CUs."""
import numpy as np
import pytest

from helpers import env, f32_reorder_bar, rel_l2
from oracle import skyla_oracle as so
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu

CFG = "test-chain"
Q4, Q6, Q8 = E.DType.Q4K, E.DType.Q6K, E.DType.Q8_0

# activation regions (f32 offsets) and widths
REGIONS = [("x0", 4096), ("y1", 4096), ("y2", 4096), ("y3", 12288), ("y4", 4096), ("y5", 128), ("y6", 512)]

# stages: (dtype, n_in, [(n_out, y region, row offset in it)], x region, accum)
STAGES = [
    (Q4, 4096, [(2001, "y1", 0), (999, "y1", 2001), (96, "y1", 3000), (1000, "y1", 3096)], "x0", False),
    (Q4, 4096, [(4000, "y2", 0)], "y1", True),
    (Q4, 4096, [(6144, "y3", 0), (6144, "y3", 6144)], "y2", False),
    (Q6, 12288, [(2047, "y4", 0), (2049, "y4", 2047)], "y3", True),
    (Q4, 4096, [(77, "y5", 0)], "y4", True),
]


class Chain:
    def __init__(self, ctx, stages, extra=None):
        self.ctx = ctx
        self.stages = stages
        self.off, o = {}, 64
        for name, width in REGIONS:
            self.off[name] = o
            o += width
        self.size = o
        planner = E.Planner(ctx.max_buffer())
        self.mats = []
        for si, (dt, n_in, segs, _, _) in enumerate(stages):
            row = []
            for j, (n_out, _, _) in enumerate(segs):
                data = synth.matrix(CFG, f"s{si}-{j}-{dt.name}-{n_in}-{n_out}", dt, n_in, n_out)
                row.append((planner.matrix(dt, n_in, n_out, data), data))
            self.mats.append(row)
        self.extra = None
        if extra is not None:  # a Q8_0 matvec that no chain takes: x0 -> y6
            data = synth.matrix(CFG, "q8-extra", Q8, 4096, 512)
            self.extra = (planner.matrix(Q8, 4096, 512, data), data)
        self.weights = E.upload_weights(ctx, planner)
        self.arena = ctx.alloc_host(self.size * 4)
        self.k = E.Kernels(ctx, self.weights, self.arena)
        self.init = synth.activations(CFG, "arena", self.size)
        self.init[:64] = 0

    def body(self, r, extra_at=None):
        g = E.Graph(r, self.k, None, None, False)
        for si, (dt, n_in, segs, xr, accum) in enumerate(self.stages):
            if extra_at == si:
                m, _ = self.extra
                g.matvec(m, (self.off["x0"], 0), (self.off["y6"], 0), False, False)
                r.barrier()
            for (n_out, yr, ro), (m, _) in zip(segs, self.mats[si]):
                g.matvec(m, (self.off[xr], 0), (self.off[yr] + ro, 0), accum, False)
            r.barrier()

    def run(self, extra_at=None, replays=1, **switches):
        """Replays from the initial arena; returns (launches, arena after each replay)."""
        with env(**{"SKYLA_HIP_CHAIN": 1, "SKYLA_HIP_CHAIN_CHECK": 1, **switches}):
            rec = self.ctx.record(False, lambda r: self.body(r, extra_at))
            try:
                outs = []
                for _ in range(replays):
                    f = self.arena.as_f32()
                    f[:] = self.init
                    self.arena.as_u32()[2] = 1
                    self.arena.upload()
                    self.ctx.replay(rec)
                    self.arena.download()
                    outs.append(self.arena.as_f32().copy())
                return rec.launches(), outs
            finally:
                rec.free()

    def region(self, f, name, width=None):
        o = self.off[name]
        return f[o: o + (width if width is not None else dict(REGIONS)[name])]

    def check_oracle(self, f):
        """Each stage against the oracle on its input as the GPU left it."""
        for si, (dt, n_in, segs, xr, accum) in enumerate(self.stages):
            x = self.region(f, xr)[:n_in].copy()
            for (n_out, yr, ro), (m, data) in zip(segs, self.mats[si]):
                want = so.matvec(int(dt), data, n_in, n_out, x).astype(np.float64)
                got = self.region(f, yr)[ro: ro + n_out].astype(np.float64)
                old = self.region(self.init, yr)[ro: ro + n_out].astype(np.float64)
                part = got - old if accum else got
                bar = f32_reorder_bar(dt, data, n_in, n_out, x, want)
                assert rel_l2(part, want) <= bar + (1e-6 if accum else 0.0), (si, n_out, rel_l2(part, want), bar)

    def free(self):
        for b in self.weights:
            b.free()
        self.arena.free()


@pytest.fixture(scope="module")
def chain(ctx):
    c = Chain(ctx, STAGES, extra=True)
    yield c
    c.free()


def test_chain_matches_k_split_launches_and_oracle(chain):
    n_chain, (got,) = chain.run()
    n_plain, (ref,) = chain.run(SKYLA_HIP_CHAIN=0, SKYLA_HIP_KS="4_1")
    assert n_chain == 1, n_chain            # five stages, one launch
    assert n_plain == len(STAGES), n_plain
    # Q4_K stages before the Q6_K one: the same bits as the K-split launches
    for name in ("y1", "y2", "y3"):
        assert np.array_equal(chain.region(got, name).view(np.uint32), chain.region(ref, name).view(np.uint32)), name
    # rows no stage writes keep their values
    assert np.array_equal(chain.region(got, "y2")[4000:], chain.region(chain.init, "y2")[4000:])
    assert np.array_equal(chain.region(got, "y5")[77:], chain.region(chain.init, "y5")[77:])
    chain.check_oracle(got)
    chain.check_oracle(ref)


def test_chain_replays_are_identical(chain):
    _, outs = chain.run(replays=3)
    for f in outs[1:]:
        assert np.array_equal(f.view(np.uint32), outs[0].view(np.uint32))


def test_other_launch_splits_the_chain(chain):
    """A Q8_0 matvec between stages 2 and 3 runs as its own launch: two chains around it."""
    n, (got,) = chain.run(extra_at=2)
    assert n == 3, n
    chain.check_oracle(got)
    m, data = chain.extra
    want = so.matvec(int(Q8), data, 4096, 512, chain.region(got, "x0").copy())
    assert rel_l2(chain.region(got, "y6"), want) <= f32_reorder_bar(Q8, data, 4096, 512, chain.region(got, "x0"), want)


def test_single_stage_recording(ctx):
    """One chainable launch alone (no run to chain) replays as an ordinary launch."""
    c = Chain(ctx, STAGES[:1])
    try:
        n, (got,) = c.run()
        assert n == 1
        c.check_oracle(got)
    finally:
        c.free()
