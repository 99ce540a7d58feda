"""Host-side bounds check of the K-quant GEMM tile's indexing (matmul.hip,
matmul_tile128_w and its weight loaders) against the sizes the runtime gives its launches
(skyla_hip.cpp: split_of / pack for K-split grids, build_launches for the balanced grid,
bind_workspace for the partial tiles and counters), for the eight-wave and four-wave
tiles at the config-3 shapes and ragged ones, K split 1, 2, 4 and 8 ways.

The index arithmetic below restates the kernel's, statement for statement, and every index
it produces is checked against its buffer: workgroup -> (row tile, token tile, split, slot)
covers every (tile, split) exactly once; partial-tile and counter slots stay inside the
workspace; stage ranges partition the super-blocks; every weight, header, scale and d load
(direct-to-LDS pieces and the register-staged loader) stays inside its planner region; and
every direct-to-LDS piece lands inside its stage buffer.  This is the check for the fault
a four-wave tile split four ways once made: no index of either tile leaves its buffer at
any split of these shapes."""
import numpy as np
import pytest

TM, KC, TN = 128, 256, 128
PART_FLOATS = 128 * 128          # kSplitTileBytes / 4: one f32 partial tile
SLOTS = 512                      # balanced grid: two four-wave workgroups on each of 256 CUs


def split_of(tiles: int, n_in: int, slots: int = 256) -> int:
    """skyla_hip.cpp split_of: launches of at most 128 tiles split their super-blocks."""
    if tiles == 0 or tiles > 128:
        return 1
    s = min(slots // tiles, n_in // 256 // 4, 8)
    return s if s >= 2 else 1


def tile_map(gx: int, gz: int, s: int):
    """matmul_tile128_w, plain grid (HYB = 0, MOE = 0): (rt, tt, sp, kt) of every workgroup
    of grid (gx, 1, gz)."""
    bx, bz = np.meshgrid(np.arange(gx, dtype=np.int64), np.arange(gz, dtype=np.int64), indexing="ij")
    z = gz // s
    lin = bx + gx * bz
    rem = lin % gz
    rt, tt, sp = lin // gz, rem % z, rem // z
    return rt.ravel(), tt.ravel(), sp.ravel(), (rt * z + tt).ravel()


def hyb_map(hf: int, hz: int):
    """matmul_tile128_w, balanced grid (HYB = 1): (rt, tt, S, sp, kt) of workgroups 0..SLOTS."""
    b = np.arange(SLOTS, dtype=np.int64)
    whole = b < hf
    t = np.where(whole, b, hf + ((b - hf) >> 1))
    return t // hz, t % hz, np.where(whole, 1, 2), np.where(whole, 0, (b - hf) & 1), t - hf, whole


def check_partials(kt, sp, s, n_cnt, nw):
    """The partial-tile stores and loads (ws + (kt S + sp) PART + wave (NB 16 64) + (j 16 + i)
    64 + lane) and the counter cnt[kt] of split launches, against bind_workspace's ws of
    n_cnt S kSplitTileBytes and n_cnt counters."""
    nb = 2 if nw == 8 else TN // 32
    part = nw * nb * 16 * 64
    assert part == PART_FLOATS
    assert kt.min() >= 0 and kt.max() < n_cnt
    last = (kt * s + sp) * part + (nw - 1) * (nb * 16 * 64) + (nb * 16 - 1) * 64 + 63
    assert last.max() < n_cnt * s * PART_FLOATS


SHAPES = [  # (type 1 Q4_K / 2 Q6_K, n_in, n_out, tokens)
    (1, 4096, 4096, 512), (1, 4096, 12288, 512), (2, 12288, 4096, 512), (1, 4096, 1024, 128),
    (1, 768, 20000, 200), (2, 768, 9000, 500), (1, 1024, 200, 37), (2, 768, 130, 100), (1, 4096, 6144, 128),
]


@pytest.mark.parametrize("nw", [8, 4])
@pytest.mark.parametrize("s", [1, 2, 4, 8])
@pytest.mark.parametrize("ty,n_in,n_out,m", SHAPES)
def test_split_grid_indices(ty, n_in, n_out, m, s, nw):
    gx, z = -(-n_out // TM), -(-m // TN)
    n_stage = n_in // KC
    if s > n_stage:
        pytest.skip("more splits than super-blocks")
    rt, tt, sp, kt = tile_map(gx, z * s, s)
    # every (row tile, token tile, split) exactly once
    key = (rt * z + tt) * s + sp
    assert np.array_equal(np.sort(key), np.arange(gx * z * s))
    assert rt.max() < gx and tt.max() < z and sp.max() < s
    n_cnt = gx * z                                   # pack: groups[0] * groups[2]
    if s > 1:
        check_partials(kt, sp, s, n_cnt, nw)
    # st0 / st1 = sp n_stage / S .. (sp + 1) n_stage / S partition the super-blocks
    stages = np.concatenate([np.arange(q * n_stage // s, (q + 1) * n_stage // s) for q in range(s)])
    assert np.array_equal(stages, np.arange(n_stage))


@pytest.mark.parametrize("ty,n_in,n_out,m", [(1, 4096, 12288, 512), (1, 768, 20000, 200), (2, 768, 9000, 500),
                                             (1, 4096, 9000, 300), (2, 4096, 16384, 256)])
def test_balanced_grid_indices(ty, n_in, n_out, m):
    """The balanced grid build_launches gives launches of more tiles than CUs and fewer than
    the two-per-CU slots: hf = 2 tiles - 512 whole tiles, the rest in two K halves."""
    gx, hz = -(-n_out // TM), -(-m // TN)
    tiles = gx * hz
    if not (SLOTS // 2 < tiles < SLOTS and n_in >= 2 * 256):
        pytest.skip("not a balanced-grid launch")
    hf = 2 * tiles - SLOTS
    rt, tt, s, sp, kt, whole = hyb_map(hf, hz)
    assert rt.max() < gx and tt.max() < hz
    t = rt * hz + tt
    assert np.array_equal(np.sort(t[whole]), np.arange(hf))              # whole tiles once
    halved = np.sort(t[~whole] * 2 + sp[~whole])
    assert np.array_equal(halved, np.arange(2 * hf, 2 * tiles))          # the rest twice, sp 0 and 1
    check_partials(kt[~whole], sp[~whole], 2, tiles - hf, 4)             # n_cnt = tiles - hf


def regions(ty, n_in, n_out):
    """Planner regions of one matrix at offset 0, in bytes: (start, length) of qs / ql,
    header / qh, scales, d."""
    supers = n_in // 256
    if ty == 1:
        qs = n_out * supers * 128
        return [(0, qs), (qs, n_out * supers * 16)]
    ql, qh, sc = n_out * supers * 128, n_out * supers * 64, n_out * supers * 16
    return [(0, ql), (ql, qh), (ql + qh, sc), (ql + qh + sc, n_out * supers * 2)]


def dl_pieces(ty, n_in, n_out, row0, lane, b):
    """dl_wpiece: byte offset at super-block 0, bytes per super-block, and the region."""
    supers, last = n_in // 256, n_out - 1
    reg = regions(ty, n_in, n_out)
    o = [r[0] // (2 if i == 3 else 16) for i, r in enumerate(reg)]   # region offsets in push units
    R = lambda r: np.minimum(row0 + r, last)  # noqa: E731
    swz = lambda r: (r & 7) ^ ((r >> 3) & 1)  # noqa: E731  (dl_swz)
    swz4 = lambda r: ((r >> 1) ^ (r >> 3)) & 3  # noqa: E731  (dl_swz4)
    if b < 16:
        r = 8 * b + (lane >> 3)
        return 16 * (o[0] + R(r) * supers * 8 + ((lane & 7) ^ swz(r))), 128, 0
    if ty == 1:
        return 16 * (o[1] + R(64 * (b - 16) + lane) * supers), 16, 1
    if b < 24:
        r = 16 * (b - 16) + (lane >> 2)
        return 16 * (o[1] + R(r) * supers * 4 + ((lane & 3) ^ swz4(r))), 64, 1
    if b < 26:
        return 16 * (o[2] + R(64 * (b - 24) + lane) * supers), 16, 2
    return 2 * (o[3] + R(64 * (b - 26) + lane) * supers), 2, 3


@pytest.mark.parametrize("ty,n_in,n_out", [(1, 4096, 4096), (1, 4096, 12288), (2, 12288, 4096), (1, 768, 20000),
                                           (2, 768, 9000), (1, 1024, 200), (2, 768, 130)])
@pytest.mark.parametrize("nw", [8, 4])
def test_direct_to_lds_pieces_in_bounds(ty, n_in, n_out, nw):
    """Every 16 B piece the direct-to-LDS tile loads (dl_issue_w: blocks NW i + wave of
    dl_wblocks, d as the aligned 16 B around it) lies inside its planner region, at every
    row tile and super-block; every piece lands inside its stage buffer."""
    supers = n_in // 256
    nblocks = 18 if ty == 1 else 28
    ws_slots, wmin = -(-nblocks // nw), nblocks // nw
    reg = regions(ty, n_in, n_out)
    lane = np.arange(64)
    for rt in range(-(-n_out // TM)):
        for wv in range(nw):
            for i in range(ws_slots):
                b = nw * i + wv
                if not (i < wmin or b < nblocks):
                    continue
                off, per, k = dl_pieces(ty, n_in, n_out, rt * TM, lane, b)
                start, length = reg[k]
                for sb in (0, supers - 1):
                    if k == 3:   # d: the 16 B-aligned piece around it, within dres's range
                        a = (off + 2 * sb) & ~15
                        assert a.min() >= start & ~15 and (a + 16).max() <= (start + length + 15) & ~15
                    else:
                        a = off + per * sb
                        assert a.min() >= start and (a + 16).max() <= start + length
                assert (b + 1) * 256 <= nblocks * 256      # LDS: 256 u32 per block in a stage


@pytest.mark.parametrize("ty,n_in,n_out", [(1, 4096, 4096), (2, 12288, 4096), (1, 768, 20000), (2, 768, 9000),
                                           (2, 768, 130)])
@pytest.mark.parametrize("nt", [512, 256])
def test_register_loader_in_bounds(ty, n_in, n_out, nt):
    """WLds<TYPE, NT>::load (the register-staged tiles, eight and four waves): every qs / ql,
    header / qh, scale and d index inside its region at every row tile and super-block."""
    supers, last = n_in // 256, n_out - 1
    tid = np.arange(nt)
    reg = regions(ty, n_in, n_out)
    units = lambda k: reg[k][1] // (2 if k == 3 else 16)  # noqa: E731
    for rt in range(-(-n_out // TM)):
        row0 = rt * TM
        for sb in (0, supers - 1):
            if ty == 1:
                qi = TM * 8 // nt
                for i in range(qi):
                    u = tid + nt * i
                    idx = np.minimum(row0 + (u >> 3), last) * (n_in >> 5) + sb * 8 + (u & 7)
                    assert idx.max() < units(0)
                hd = np.minimum(row0 + tid[tid < TM], last) * supers + sb
                assert hd.max() < units(1)
            else:
                li, hi = TM * 8 // nt, TM * 4 // nt
                for i in range(li):
                    u = tid + nt * i
                    assert ((np.minimum(row0 + (u >> 3), last) * supers + sb) * 8 + (u & 7)).max() < units(0)
                for i in range(hi):
                    u = tid + nt * i
                    assert ((np.minimum(row0 + (u >> 2), last) * supers + sb) * 4 + (u & 3)).max() < units(1)
                rs = np.minimum(row0 + (tid & (TM - 1)), last) * supers + sb
                assert rs[tid < TM].max() < units(2)
                if nt > TM:
                    assert rs[(tid >= TM) & (tid < 2 * TM)].max() < units(3)


def test_split_rule_sizes():
    """split_of at the config-3 shapes (M = 512): q and down 128 tiles split 2 ways; gate 384
    tiles unsplit (the balanced grid)."""
    assert split_of(32 * 4, 4096) == 2 and split_of(32 * 4, 12288) == 2 and split_of(96 * 4, 4096) == 1


def test_check_catches_undersized_workspace():
    """The partial-slot check fails for a workspace sized by row tiles only (a counter per
    row tile instead of per tile), and for a grid whose z extent is not tokens x splits."""
    gx, z, s = 32, 4, 2
    rt, tt, sp, kt = tile_map(gx, z * s, s)
    with pytest.raises(AssertionError):
        check_partials(kt, sp, s, gx, 8)
    rt, tt, sp, kt = tile_map(gx, z * s + 1, s)     # one stray z row of workgroups
    with pytest.raises(AssertionError):
        assert np.array_equal(np.sort((rt * z + tt) * s + sp), np.arange(gx * z * s))


@pytest.mark.parametrize("n_tok,used,n_expert", [(128, 8, 128), (1, 8, 128), (37, 2, 16), (128, 4, 64), (100, 8, 8)])
def test_expert_prepass_rows(n_tok, used, n_expert):
    """The f16 row prepass of an expert-group matmul (build_launches: rows = token tiles of
    32 x rows per token, exponents then rows in the workspace) covers every input row the
    expert tiles read: gate and up read token rows slot / used, down the slot rows; the
    engine's grid has BATCH / 32 token tiles and a chunk holds at most BATCH tokens."""
    from skyla_hip import engine as E
    z = E.BATCH // E.MOE_TILE_COLS
    assert n_tok <= z * 32
    rng = np.random.default_rng(n_tok * 1000 + used)
    ids = np.stack([rng.choice(n_expert, used, replace=False) for _ in range(n_tok)]).reshape(-1)
    slots = np.argsort(ids, kind="stable")            # moe_sort's list: slots grouped by expert
    for x_div, per_token in ((used, 1), (1, used)):   # gate / up, then down
        rows = z * 32 * per_token
        h_off = (rows * 4 + 255) // 256 * 256           # bytes of exponents before the rows
        xrow = slots // x_div                             # the tile's input rows
        assert xrow.max() < n_tok * per_token <= rows     # converted (t < ctl[2] x per_token)
        assert xrow.max() * 4 < h_off                      # exponent words
        n_in = 2048
        last = h_off // 2 + int(xrow.max()) * n_in + n_in  # f16 units, end of the last row read
        assert last <= (h_off + rows * n_in * 2) // 2      # inside the workspace region


def expert_grid(rt_n: int, y: int):
    """matmul_tile128_w, MOE = 2 (expert tiles over moe_sort's tile map): (row tile, map entry,
    XCD = linear id mod 8) of every workgroup of grid (rt_n, y, 1)."""
    lin = np.arange(rt_n * y, dtype=np.int64)
    k8 = lin // 8
    return k8 % rt_n, (k8 // rt_n) * 8 + lin % 8, lin % 8


@pytest.mark.parametrize("rt_n", [6, 12, 16, 5])
@pytest.mark.parametrize("bound", [1, 8, 150, 156, 280])
def test_expert_grid_order(rt_n, bound):
    """The runtime's grid.y for expert tiles (the map bound rounded up to a multiple of 8, at
    most 312 entries of the map's 319) and the tile's XCD-aware order: every (row tile,
    entry) exactly once, and all the row tiles of an entry on one XCD (one residue mod 8)."""
    y = min((bound + 7) // 8 * 8, 312)
    assert y % 8 == 0 and y >= min(bound, 312)
    rt, ent, xcd = expert_grid(rt_n, y)
    assert rt.max() < rt_n and ent.max() < y
    assert np.array_equal(np.sort(rt * y + ent), np.arange(rt_n * y))
    for e in range(y):
        assert np.unique(xcd[ent == e]).size == 1, e
