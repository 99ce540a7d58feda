"""GPU parity of the MoE top-k dispatch (config 4) through the C-ABI.

Kernels are checked one by one against exact or brute-force references (route: ties to the
lowest index; sort: stable counting sort; combine: the oracle's summation order, bit-exact)
and then as the whole graph/moe.rs sequence against the oracle's Ffn::forward (Moe arm,
skyla-ref/src/ffn.rs:58-76), for a decode token and a 128-token prefill chunk.  Router
near-ties can legitimately flip the route between two summation orders, so the chain tests
skip a token whose 8th and 9th logits are closer than 1e-5 (none do at these seeds).
"""

import numpy as np
import pytest

from helpers import rel_l2, tactics
from oracle import skyla_oracle as so
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu
# decode: f32 matvecs composed with f32 SiLU and combine; prefill: f16-input GEMMs
F32 = 1e-5

CFG = "qwen3-30b-a3b-moe"
N_EMBD, N_FF_EXP, N_EXPERT, N_USED = 2048, 768, 128, 8


def _cfg():
    return E.Config(n_embd=N_EMBD, n_ff=64, n_expert=N_EXPERT, n_expert_used=N_USED, n_ff_expert=N_FF_EXP)


class MoeSetup:
    def __init__(self, ctx, router=None, base=None):
        """Config 4's MoE layer; `router` replaces the seeded router, `base` lends its experts."""
        self.ctx = ctx
        self.c = _cfg()
        self.router = synth.router(CFG, "router", N_EXPERT, N_EMBD) if router is None else router
        if base is None:
            self.gate = synth.matrix(CFG, "gate_exps", E.DType.Q4K, N_EMBD, N_FF_EXP, N_EXPERT)
            self.up = synth.matrix(CFG, "up_exps", E.DType.Q4K, N_EMBD, N_FF_EXP, N_EXPERT)
            self.down = synth.matrix(CFG, "down_exps", E.DType.Q4K, N_FF_EXP, N_EMBD, N_EXPERT)
        else:
            self.gate, self.up, self.down = base.gate, base.up, base.down
        p = E.Planner(ctx.max_buffer())
        self.router_off = p.table(self.router.reshape(-1))
        self.qg = p.matrix(E.DType.Q4K, N_EMBD, N_FF_EXP, self.gate)
        self.qu = p.matrix(E.DType.Q4K, N_EMBD, N_FF_EXP, self.up)
        self.qd = p.matrix(E.DType.Q4K, N_FF_EXP, N_EMBD, self.down)
        self.weights = E.upload_weights(ctx, p)
        self.a = E.Arena(ctx, self.c)
        self.k = E.Kernels(ctx, self.weights, self.a.buffer)

    def load(self, n: np.ndarray, x0: np.ndarray) -> None:
        """Writes the normed input rows (arena n) and the residual rows (arena x)."""
        a = self.a
        f = a.f32()
        for t in range(n.shape[0]):
            f[a.n + t * a.s_embd: a.n + t * a.s_embd + N_EMBD] = n[t]
            f[a.x + t * a.s_embd: a.x + t * a.s_embd + N_EMBD] = x0[t]
        a.set_ctl(0, 0, n.shape[0])
        a.buffer.upload()

    def run_moe(self, batched: bool, kernels=None):
        k = kernels or self.k

        def body(r):
            E.Graph(r, k, self.a, self.c, batched).moe(self.qg, self.qu, self.qd, self.router_off)
        rec = self.ctx.record(False, body)
        self.ctx.replay(rec)
        rec.free()
        self.a.buffer.download()

    def rows(self, off: int, stride: int, n_tok: int, width: int) -> np.ndarray:
        f = self.a.f32()
        return np.stack([f[off + t * stride: off + t * stride + width] for t in range(n_tok)])

    def free(self):
        for b in self.weights:
            b.free()
        self.a.buffer.free()


@pytest.fixture(scope="module")
def moe(ctx):
    s = MoeSetup(ctx)
    yield s
    s.free()


def _near_tie(router, n, eps=1e-5) -> bool:
    lg = np.sort(router.astype(np.float64) @ n.astype(np.float64))[::-1]
    return abs(lg[N_USED - 1] - lg[N_USED]) < eps


def _dispatch(ctx, p, groups, push):
    rec = ctx.record(False, lambda r: r.dispatch(p, groups, push))
    ctx.replay(rec)
    rec.free()


@pytest.mark.parametrize("n_embd,n_tok", [(2048, 1), (2048, 37), (2048, 128), (2560, 21)])
def test_logits_kernel_batches(ctx, n_embd, n_tok):
    """Router logits for a decode token and for ragged batches (the runtime runs batches
    16 tokens per workgroup; 2560 values take the re-read path for rows past 2048): each
    logit within f32 summation-order error of an f64 reference, and nothing written for
    tokens past the batch."""
    router = synth.router(CFG, f"router-{n_embd}", N_EXPERT, n_embd)
    x = synth.activations(CFG, f"logits-x-{n_embd}-{n_tok}", (n_tok, n_embd))
    p = E.Planner(ctx.max_buffer())
    roff = p.table(router.reshape(-1))
    weights = E.upload_weights(ctx, p)
    x_off, lg_off = 64, 64 + n_tok * n_embd
    size = (lg_off + (n_tok + 16) * N_EXPERT + 64) * 4
    arena = ctx.alloc_host(size)
    try:
        f = arena.as_f32()
        f[x_off: x_off + x.size] = x.reshape(-1)
        f[lg_off: lg_off + (n_tok + 16) * N_EXPERT] = -7.0
        arena.upload()
        k = E.Kernels(ctx, weights, arena)
        _dispatch(ctx, k.logits, [N_EXPERT, n_tok, 1], [x_off, roff, lg_off, n_embd, n_embd])
        arena.download()
        got = arena.as_f32()[lg_off: lg_off + (n_tok + 16) * N_EXPERT].reshape(n_tok + 16, N_EXPERT)
        want = x.astype(np.float64) @ router.astype(np.float64).T
        bound = 1e-5 * (np.abs(x).astype(np.float64) @ np.abs(router).astype(np.float64).T)
        assert np.all(np.abs(got[:n_tok] - want) <= bound)
        assert np.all(got[n_tok:] == -7.0)
    finally:
        arena.free()
        for b in weights:
            b.free()


def test_route_kernel_ties_and_order(ctx, moe):
    a, m = moe.a, moe.a.moe
    n_tok = 128
    g = np.random.default_rng(7)
    logits = g.standard_normal((n_tok, N_EXPERT)).astype(np.float32)
    logits[0, :] = 1.0                      # all tied: experts 0..7
    logits[1, [5, 9, 77, 3]] = 9.0          # tie at the top: 3, 5, 9, 77
    logits[2, 100] = -0.0
    logits[2, :] = np.where(np.arange(N_EXPERT) == 40, 0.0, -1.0)  # +0 beats -1s, then ties
    f = a.f32()
    f[m.logits: m.logits + logits.size] = logits.reshape(-1)
    a.set_ctl(0, 0, n_tok)
    a.buffer.upload()
    _dispatch(ctx, moe.k.route, [1, n_tok, 1], [m.logits, m.ids, m.weights, N_EXPERT, N_USED])
    a.buffer.download()
    ids = a.u32()[m.ids: m.ids + n_tok * N_USED].reshape(n_tok, N_USED)
    w = a.f32()[m.weights: m.weights + n_tok * N_USED].reshape(n_tok, N_USED)
    for t in range(n_tok):
        order = sorted(range(N_EXPERT), key=lambda e: (-float(logits[t, e]), e))[:N_USED]
        assert list(ids[t]) == order, t
        v = logits[t, order].astype(np.float64)
        want = np.exp(v - v[0]) / np.exp(v - v[0]).sum()
        assert np.allclose(w[t], want, rtol=2e-6, atol=1e-7), t


def test_sort_kernel_matches_stable_counting_sort(ctx, moe):
    a, m = moe.a, moe.a.moe
    n_tok = 128
    g = np.random.default_rng(11)
    ids = g.integers(0, N_EXPERT, size=(n_tok, N_USED)).astype(np.uint32)
    ids[:4] = 17                            # a crowded expert
    ids[5, :] = np.arange(8) + 120          # top experts
    u = a.u32()
    u[m.ids: m.ids + ids.size] = ids.reshape(-1)
    a.set_ctl(0, 0, n_tok)
    a.buffer.upload()
    _dispatch(ctx, moe.k.sort, [1, 1, 1], [m.ids, m.table, m.list, N_EXPERT, N_USED])
    a.buffer.download()
    table = a.u32()[m.table: m.table + 2 * N_EXPERT].reshape(N_EXPERT, 2)
    lst = a.u32()[m.list: m.list + ids.size]
    want_table, want_list = so.moe_sort(ids.reshape(-1), N_EXPERT)
    assert np.array_equal(table, want_table)
    assert np.array_equal(lst, want_list)
    # brute force: stable argsort by expert
    assert np.array_equal(lst, np.argsort(ids.reshape(-1), kind="stable"))
    # the tile map before the table: every (expert, 32-slot tile) pair in expert order
    counts = np.bincount(ids.reshape(-1), minlength=N_EXPERT)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    entries = [(e | (z << 16), int(starts[e]) | (int(counts[e]) << 16))
               for e in range(N_EXPERT) for z in range(-(-int(counts[e]) // 32))]
    tiles = a.u32()[m.tiles: m.tiles + E.MOE_TILE_MAP]
    assert counts[17] > 32 and tiles[0] == len(entries)
    assert list(tiles[1: 1 + 2 * len(entries)]) == [w for en in entries for w in en]


def test_combine_kernel_bit_exact(ctx, moe):
    a, m = moe.a, moe.a.moe
    n_tok = 3
    g = np.random.default_rng(3)
    x0 = g.standard_normal((n_tok, N_EMBD)).astype(np.float32)
    down = g.standard_normal((n_tok * N_USED, N_EMBD)).astype(np.float32)
    wts = g.random((n_tok, N_USED)).astype(np.float32)
    f = a.f32()
    for t in range(n_tok):
        f[a.x + t * a.s_embd: a.x + t * a.s_embd + N_EMBD] = x0[t]
    for s in range(n_tok * N_USED):
        f[m.down + s * a.s_embd: m.down + s * a.s_embd + N_EMBD] = down[s]
    f[m.weights: m.weights + wts.size] = wts.reshape(-1)
    a.buffer.upload()
    _dispatch(ctx, moe.k.combine, [-(-N_EMBD // 256), n_tok, 1], [a.x, m.down, m.weights, N_EMBD, a.s_embd, N_USED])
    a.buffer.download()
    got = moe.rows(a.x, a.s_embd, n_tok, N_EMBD)
    want = x0.copy()
    for t in range(n_tok):  # ffn.rs:67-74 then model.rs:113-114: out = 0; out += w*y; x += out
        out = np.zeros(N_EMBD, np.float32)
        for s in range(N_USED):
            out = out + wts[t, s] * down[t * N_USED + s]
        want[t] = want[t] + out
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_silu_and_to_half(ctx, moe):
    a = moe.a
    g = np.random.default_rng(5)
    n_tok, n = 4, 64
    gate = (g.standard_normal((n_tok, n)) * 4).astype(np.float32)
    up = g.standard_normal((n_tok, n)).astype(np.float32)
    f = a.f32()
    for t in range(n_tok):
        f[a.gate + t * a.s_ff: a.gate + t * a.s_ff + n] = gate[t]
        f[a.up + t * a.s_ff: a.up + t * a.s_ff + n] = up[t]
    a.set_ctl(0, 0, n_tok - 1)  # the last row is beyond ctl[2] and must stay untouched
    a.buffer.upload()
    _dispatch(ctx, moe.k.silu, [1, n_tok, 1], [a.gate, a.up, n, a.s_ff])
    th = ctx.create_pipeline("to_half", 3, 24, [])   # to_half.metal (used when HALF_INPUTS is set)
    th.bind_buffers([a.buffer, a.buffer, a.buffer])
    _dispatch(ctx, th, [1, n_tok, 1], [a.gate, 2 * a.half, n, a.s_ff, 64, 1])
    th.free()
    a.buffer.download()
    got = moe.rows(a.gate, a.s_ff, n_tok, n)
    want = gate / (1.0 + np.exp(-gate.astype(np.float64))) * up
    assert np.allclose(got[:3], want[:3], rtol=1e-5, atol=1e-6)
    assert np.array_equal(got[3], gate[3])
    h = a.buffer.host().view("<f2")
    half = np.stack([h[2 * a.half + t * 64: 2 * a.half + t * 64 + n] for t in range(3)])
    assert np.array_equal(half.view(np.uint16), got[:3].astype(np.float16).view(np.uint16))


def _oracle_moe(moe, n):
    return so.moe_forward(moe.router, int(E.DType.Q4K), moe.gate, int(E.DType.Q4K), moe.up, int(E.DType.Q4K),
                          moe.down, N_EMBD, N_FF_EXP, N_EXPERT, N_USED, n)


def test_moe_decode_token(ctx, moe):
    n = synth.activations(CFG, "decode-n", (1, N_EMBD))
    x0 = synth.activations(CFG, "decode-x", (1, N_EMBD))
    assert not _near_tie(moe.router, n[0])
    moe.load(n, x0)
    moe.run_moe(batched=False)
    a, m = moe.a, moe.a.moe
    out, ids, w = _oracle_moe(moe, n[0])
    assert list(a.u32()[m.ids: m.ids + N_USED]) == list(ids)
    assert np.allclose(a.f32()[m.weights: m.weights + N_USED], w, rtol=1e-5)
    got = moe.rows(a.x, a.s_embd, 1, N_EMBD)[0] - x0[0]
    assert rel_l2(got, out) <= F32, rel_l2(got, out)  # expert matvecs in f32, as the reference


def test_moe_prefill_chunk(ctx, moe):
    n_tok = 128
    n = synth.activations(CFG, "prefill-n", (n_tok, N_EMBD))
    x0 = synth.activations(CFG, "prefill-x", (n_tok, N_EMBD))
    moe.load(n, x0)
    moe.run_moe(batched=True)
    a, m = moe.a, moe.a.moe
    got = moe.rows(a.x, a.s_embd, n_tok, N_EMBD) - x0
    ids_gpu = a.u32()[m.ids: m.ids + n_tok * N_USED].reshape(n_tok, N_USED)
    table, lst = so.moe_sort(ids_gpu.reshape(-1), N_EXPERT)
    assert np.array_equal(a.u32()[m.table: m.table + 2 * N_EXPERT].reshape(N_EXPERT, 2), table)
    assert np.array_equal(a.u32()[m.list: m.list + n_tok * N_USED], lst)
    checked, errs, outs, gots = 0, [], [], []
    for t in range(n_tok):
        if _near_tie(moe.router, n[t]):
            continue
        out, ids, _ = _oracle_moe(moe, n[t])
        assert list(ids_gpu[t]) == list(ids), t
        assert np.all(np.isfinite(got[t])), (t, "non-finite GPU output")
        assert np.all(np.isfinite(out)), (t, "non-finite oracle output")
        errs.append(rel_l2(got[t], out))
        outs.append(out)
        gots.append(got[t])
        checked += 1
    assert checked >= n_tok - 2
    assert max(errs) <= 5e-3, max(errs)
    assert rel_l2(np.concatenate(gots), np.concatenate(outs)) <= 2e-3


@pytest.mark.parametrize("fuse", ["1", "0"])
@pytest.mark.parametrize("n_tok", [128, 37, 1])
def test_moe_prefill_f16_rows_same_bits(ctx, moe, n_tok, fuse):
    """The expert-group matmuls of a prefill chunk on the f16 row prepass (the tokens' rows
    for gate and up, the slot rows for down; tactic xhalf_moe=1) against the tile's own f32
    staging (xhalf_moe=0): the same bits for every row whose input stays below 2^15 (the
    gate/up outputs; the down rows of slots whose SiLU row does), and for rows past it
    (the prepass scales the whole row by a power of two, the f32 tile each 256-column chunk
    that holds such a value) within the f16 rounding of their inputs; 128, 37, 1 tokens;
    gate and up as one launch of two segments (fuse=1) or two launches (fuse=0)."""
    n = synth.activations(CFG, f"xh-n-{n_tok}", (n_tok, N_EMBD))
    x0 = synth.activations(CFG, f"xh-x-{n_tok}", (n_tok, N_EMBD))
    got = {}
    slots = n_tok * N_USED
    for xh in ("1", "0"):
        with tactics(xhalf_moe=xh, fuse=fuse if xh == "1" else None):
            moe.load(n, x0)
            moe.run_moe(batched=True)
        a, m = moe.a, moe.a.moe
        gate = a.f32()[m.gate: m.gate + slots * m.stride].reshape(slots, m.stride)[:, :N_FF_EXP].copy()
        down = a.f32()[m.down: m.down + slots * a.s_embd].reshape(slots, a.s_embd)[:, :N_EMBD].copy()
        got[xh] = (gate, down)
    (g1, d1), (g0, d0) = got["1"], got["0"]
    assert np.array_equal(g1.view(np.uint32), g0.view(np.uint32))
    small = np.abs(g0).max(axis=1) < 32768.0           # slot rows with no value at 2^15 or above
    assert np.array_equal(d1[small].view(np.uint32), d0[small].view(np.uint32))
    if (~small).any():
        assert rel_l2(d1[~small], d0[~small]) <= 2e-3


@pytest.mark.parametrize("n_tok", [128, 45])
def test_moe_prefill_crowded_experts_same_bits(ctx, moe, n_tok):
    """Every token routed to the same 8 experts (router rows aligned with a component all
    the tokens share), so each expert holds every token and the grouped matmuls walk several
    32-slot tiles of one expert through the tile map (xhalf_moe=1) against the f32-staged
    tile over every expert times every token tile (xhalf_moe=0): the same bits for gate and
    up, and for the down rows whose inputs stay below 2^15."""
    rng = np.random.default_rng(5)
    common = rng.standard_normal(N_EMBD).astype(np.float32)
    n = (common + np.float32(0.3) * rng.standard_normal((n_tok, N_EMBD))).astype(np.float32)
    x0 = synth.activations(CFG, f"crowd-x-{n_tok}", (n_tok, N_EMBD))
    router = moe.router.copy()
    chosen = [3, 9, 20, 33, 64, 90, 111, 127]
    router[chosen] = common / np.float32(np.linalg.norm(common)) * np.float32(0.5)
    s = MoeSetup(ctx, router=router, base=moe)
    slots = n_tok * N_USED
    got = {}
    try:
        for xh in ("1", "0"):
            with tactics(xhalf_moe=xh):
                s.load(n, x0)
                s.run_moe(batched=True)
            a, m = s.a, s.a.moe
            ids = a.u32()[m.ids: m.ids + slots].reshape(n_tok, N_USED)
            assert np.all(np.sort(ids, axis=1) == chosen)
            gate = a.f32()[m.gate: m.gate + slots * m.stride].reshape(slots, m.stride)[:, :N_FF_EXP].copy()
            down = a.f32()[m.down: m.down + slots * a.s_embd].reshape(slots, a.s_embd)[:, :N_EMBD].copy()
            got[xh] = (gate, down, a.u32()[m.tiles])
    finally:
        s.free()
    (g1, d1, t1), (g0, d0, _) = got["1"], got["0"]
    assert t1 == N_USED * -(-n_tok // 32)
    assert np.array_equal(g1.view(np.uint32), g0.view(np.uint32))
    small = np.abs(g0).max(axis=1) < 32768.0
    assert small.any()
    assert np.array_equal(d1[small].view(np.uint32), d0[small].view(np.uint32))
    if (~small).any():
        assert rel_l2(d1[~small], d0[~small]) <= 2e-3


def test_moe_decode_expert_variant_choice(ctx, moe):
    """Expert launches run on the variant the runtime picks for them (four waves, 16 lanes
    per row); the layer output equals the engine-requested variants' up to f32 summation
    order, and the route is the same."""
    n = synth.activations(CFG, "variant-n", (1, N_EMBD))
    x0 = synth.activations(CFG, "variant-x", (1, N_EMBD))
    assert not _near_tie(moe.router, n[0])
    got, ids = {}, {}
    for retile in ("0", "1"):
        with tactics(retile=retile):
            k = E.Kernels(ctx, moe.weights, moe.a.buffer)
        moe.load(n, x0)
        moe.run_moe(batched=False, kernels=k)
        a, m = moe.a, moe.a.moe
        got[retile] = moe.rows(a.x, a.s_embd, 1, N_EMBD)[0].astype(np.float64) - x0[0]
        ids[retile] = list(a.u32()[m.ids: m.ids + N_USED])
    assert ids["1"] == ids["0"]
    assert rel_l2(got["1"], got["0"]) < 1e-5
    out, _, _ = _oracle_moe(moe, n[0])
    assert rel_l2(got["1"], out) <= F32


@pytest.mark.parametrize("forms,n_launch", [("2", 5), ("8", 5), ("10", 4), ("16", 4), ("18", 4), ("24", 3),
                                            ("26", 3)])
@pytest.mark.parametrize("seed", ["fuse-a", "fuse-b"])
def test_moe_decode_fused_forms_equal_six_launches(ctx, moe, seed, forms, n_launch):
    """The runtime's MoE decode forms (bit 2: the experts' gate + up + SiLU, 16: route +
    gate + up + SiLU, 8: down + combine) against the engine's six dispatches launched one
    by one (tactic moe_fuse=0): the same ids, routing weights, logits and residual, bit for
    bit."""
    n = synth.activations(CFG, f"{seed}-n", (1, N_EMBD))
    x0 = synth.activations(CFG, f"{seed}-x", (1, N_EMBD))
    got, launches = {}, {}
    for fuse in (forms, "0"):
        with tactics(moe_fuse=fuse):
            moe.load(n, x0)

            def body(r):
                E.Graph(r, moe.k, moe.a, moe.c, False).moe(moe.qg, moe.qu, moe.qd, moe.router_off)
            rec = ctx.record(False, body)
            launches[fuse] = rec.launches()
            ctx.replay(rec)
            rec.free()
        moe.a.buffer.download()
        a, m = moe.a, moe.a.moe
        got[fuse] = (a.u32()[m.ids: m.ids + N_USED].copy(), a.f32()[m.weights: m.weights + N_USED].copy(),
                     a.f32()[m.logits: m.logits + N_EXPERT].copy(), moe.rows(a.x, a.s_embd, 1, N_EMBD)[0].copy())
    assert (launches[forms], launches["0"]) == (n_launch, 6)
    for g1, g0 in zip(got[forms], got["0"]):
        assert np.array_equal(g1.view(np.uint32), g0.view(np.uint32))
    out, ids, _ = _oracle_moe(moe, n[0])
    if not _near_tie(moe.router, n[0]):
        assert list(got[forms][0]) == list(ids)
        assert rel_l2(got[forms][3] - x0[0], out) <= F32


def _decode_forms(s, n, x0, forms):
    """One decode token through the MoE layer on the launch forms `forms` (tactic moe_fuse):
    launches, ids, routing weights, logits and residual."""
    with tactics(moe_fuse=forms):
        s.load(n, x0)

        def body(r):
            E.Graph(r, s.k, s.a, s.c, False).moe(s.qg, s.qu, s.qd, s.router_off)
        rec = s.ctx.record(False, body)
        launches = rec.launches()
        s.ctx.replay(rec)
        rec.free()
    s.a.buffer.download()
    a, m = s.a, s.a.moe
    return (launches, a.u32()[m.ids: m.ids + N_USED].copy(), a.f32()[m.weights: m.weights + N_USED].copy(),
            a.f32()[m.logits: m.logits + N_EXPERT].copy(), s.rows(a.x, a.s_embd, 1, N_EMBD)[0].copy())


@pytest.mark.parametrize("case", ["top5-and-across-8th", "all-tied"])
def test_moe_decode_fused_route_ties(ctx, moe, case):
    """Exact logit ties through the fused route (form 16: every workgroup of the gate/up
    launch ranks the logits itself) against moe_route's rounds (the six launches): router rows
    copied so that five experts tie at the top and four more tie across the 8th place, or all
    128 tie.  The same ids, routing weights, logits and residual, bit for bit, and the ids are
    the logits' descending order with ties to the lower index."""
    n = synth.activations(CFG, "tie-n", (1, N_EMBD))
    x0 = synth.activations(CFG, "tie-x", (1, N_EMBD))
    router = moe.router.copy()
    unit = n[0] / np.float32(np.linalg.norm(n[0]))
    if case == "all-tied":
        router[:] = router[17]
        want = list(range(N_USED))
    else:  # the other logits are below 2.7
        router[[40, 3, 77, 9, 5]] = unit * np.float32(0.1)     # logit ~4.6
        router[[101, 60, 20, 100]] = unit * np.float32(0.08)   # logit ~3.6
        want = [3, 5, 9, 40, 77, 20, 60, 100]
    s = MoeSetup(ctx, router=router, base=moe)
    try:
        fused = _decode_forms(s, n, x0, "26")
        six = _decode_forms(s, n, x0, "0")
    finally:
        s.free()
    assert (fused[0], six[0]) == (3, 6)
    for g1, g0 in zip(fused[1:], six[1:]):
        assert np.array_equal(g1.view(np.uint32), g0.view(np.uint32))
    logits = fused[3]
    assert list(fused[1]) == sorted(range(N_EXPERT), key=lambda e: (-float(logits[e]), e))[:N_USED] == want
    if case == "all-tied":
        assert np.all(fused[2] == np.float32(1.0 / N_USED))


@pytest.mark.parametrize("n_expert", [256, 160])
def test_route_and_sort_past_128_experts(ctx, moe, n_expert):
    """moe_route and moe_sort with more experts than the 128 of config 4 (the engine takes up to
    256): the route's ranking then counts every expert per thread instead of two halves, and
    the sort's counts span more than half of its LDS rows.  Ids in the logits' descending order
    with ties to the lower index (brute force), weights as the softmax over the chosen,
    the sort's table and list against the oracle, and its tile map against the counts."""
    c = E.Config(n_embd=N_EMBD, n_ff=64, n_expert=n_expert, n_expert_used=N_USED, n_ff_expert=N_FF_EXP)
    arena = E.Arena(ctx, c)
    try:
        k = E.Kernels(ctx, moe.weights, arena.buffer)
        m = arena.moe
        n_tok = 128
        g = np.random.default_rng(n_expert)
        logits = g.standard_normal((n_tok, n_expert)).astype(np.float32)
        logits[0, :] = 1.0                                   # all tied: experts 0..7
        logits[1, [n_expert - 1, 130, 7, 200 % n_expert]] = 9.0  # a tie at the top past expert 128
        logits[2, :] = -1.0
        logits[2, n_expert - 3:] = 2.0                        # the top three are the last experts
        f = arena.f32()
        f[m.logits: m.logits + logits.size] = logits.reshape(-1)
        arena.set_ctl(0, 0, n_tok)
        arena.buffer.upload()
        _dispatch(ctx, k.route, [1, n_tok, 1], [m.logits, m.ids, m.weights, n_expert, N_USED])
        _dispatch(ctx, k.sort, [1, 1, 1], [m.ids, m.table, m.list, n_expert, N_USED])
        arena.buffer.download()
        ids = arena.u32()[m.ids: m.ids + n_tok * N_USED].reshape(n_tok, N_USED).copy()
        w = arena.f32()[m.weights: m.weights + n_tok * N_USED].reshape(n_tok, N_USED)
        for t in range(n_tok):
            order = sorted(range(n_expert), key=lambda e: (-float(logits[t, e]), e))[:N_USED]
            assert list(ids[t]) == order, t
            v = logits[t, order].astype(np.float64)
            want = np.exp(v - v[0]) / np.exp(v - v[0]).sum()
            assert np.allclose(w[t], want, rtol=2e-6, atol=1e-7), t
        table = arena.u32()[m.table: m.table + 2 * n_expert].reshape(n_expert, 2)
        lst = arena.u32()[m.list: m.list + ids.size]
        want_table, want_list = so.moe_sort(ids.reshape(-1), n_expert)
        assert np.array_equal(table, want_table)
        assert np.array_equal(lst, want_list)
        counts = np.bincount(ids.reshape(-1), minlength=n_expert)
        starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
        entries = [(e | (z << 16), int(starts[e]) | (int(counts[e]) << 16))
                   for e in range(n_expert) for z in range(-(-int(counts[e]) // 32))]
        tiles = arena.u32()[m.tiles: m.tiles + E.MOE_TILE_MAP]
        assert tiles[0] == len(entries)
        assert list(tiles[1: 1 + 2 * len(entries)]) == [wd for en in entries for wd in en]
    finally:
        arena.buffer.free()


def test_sort_without_room_for_the_tile_map(ctx, moe):
    """moe_sort with its table within the first 640 words of the arena (a layout of the
    reference's own, no room for the tile map before it): the table and list as the oracle's,
    and no word below the table written (the map is skipped, not written before the arena)."""
    arena = E.Arena(ctx, _cfg())
    try:
        k = E.Kernels(ctx, moe.weights, arena.buffer)
        m = arena.moe
        n_tok, table_off = 100, 64
        g = np.random.default_rng(3)
        ids = np.stack([g.choice(N_EXPERT, N_USED, replace=False) for _ in range(n_tok)]).astype(np.uint32)
        u = arena.u32()
        u[: m.ids] = np.arange(m.ids, dtype=np.uint32) * np.uint32(2654435761)  # a pattern below the table
        u[m.ids: m.ids + ids.size] = ids.reshape(-1)
        arena.set_ctl(0, 0, n_tok)
        before = arena.u32()[:table_off].copy()
        arena.buffer.upload()
        _dispatch(ctx, k.sort, [1, 1, 1], [m.ids, table_off, m.list, N_EXPERT, N_USED])
        arena.buffer.download()
        want_table, want_list = so.moe_sort(ids.reshape(-1), N_EXPERT)
        assert np.array_equal(arena.u32()[table_off: table_off + 2 * N_EXPERT].reshape(N_EXPERT, 2), want_table)
        assert np.array_equal(arena.u32()[m.list: m.list + ids.size], want_list)
        assert np.array_equal(arena.u32()[:table_off], before)
    finally:
        arena.buffer.free()
