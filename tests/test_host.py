"""CPU tests of the boundary and the host logic: the C-ABI library loads and exports what
include/skyla_hip.h declares, its error paths return codes and messages without a device,
and the engine-side restatement (planner layout, tactics, push words, grids, arena) matches
skyla-engine.  No compute call is made."""
import ctypes as C
import os
import re
import threading

import numpy as np
import pytest

from skyla_hip import abi
from skyla_hip import engine as E
from skyla_hip import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "skyla_hip.h")


def header_functions():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"\b(skyla_hip_[a-z_0-9]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = abi.load_library()
    names = header_functions()
    assert len(names) >= 30
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(s[0] for s in abi.SIGNATURES) == names


def test_code_objects_carry_every_engine_pipeline():
    """Every (name, spec) the engine restatement can request has a gfx950 symbol."""
    blob = open(abi.LIB_PATH, "rb").read()
    wanted = []
    lanes = 64
    for shader in ("matvec_q4k", "matvec_q6k", "matvec_q8_0"):
        for waves, rows in [E.KQUANT_TACTIC, E.Q8_0_TACTIC, (2, 4), (4, 2)]:
            for accum in (0, 1):
                wanted.append(f"{shader}__{waves}_{accum}_{rows}_0_{lanes}")
            for lpr in E.EXPERT_LPR:
                wanted.append(f"{shader}__{waves}_0_{rows}_1_{lpr}")
    for ty in (0, 1, 2):
        for accum in (0, 1):
            for moe in (0, 1):
                wanted += [f"matmul__{ty}_{accum}_{moe}", f"matmul__{ty}_{accum}_{moe}_1"]
    wanted += ["moe_logits", "moe_route", "moe_sort", "moe_combine", "silu_mul", "to_half", "bandwidth__256",
               "dequant__0", "dequant__1", "dequant__2"]
    for sym in wanted:
        assert sym.encode() + b"\0" in blob, sym


def test_error_paths_without_a_device():
    lib = abi.load_library()
    out = C.c_void_p()
    assert lib.skyla_hip_alloc(None, 16, C.byref(out)) == abi.E_ARG
    assert b"alloc" in lib.skyla_hip_last_error()
    assert lib.skyla_hip_pipeline_new(None, b"matmul", 5, 52, None, 0, 1, C.byref(out)) == abi.E_ARG
    assert lib.skyla_hip_record_dispatch(None, None, 0, None, None, 0) == abi.E_ARG
    assert lib.skyla_hip_replay(None, None) == abi.E_ARG
    assert lib.skyla_hip_buffer_upload(None, 0, 0) == abi.E_ARG
    assert lib.skyla_hip_max_buffer(None) == 0
    status = lib.skyla_hip_context_new(0, C.byref(out))
    if status == abi.OK:           # a GPU is present
        lib.skyla_hip_context_free(out.value)
    else:
        assert status == abi.E_DEVICE
        assert lib.skyla_hip_last_error()
        with pytest.raises(abi.SkylaHipError) as e:
            abi.Context.new(0)
        assert e.value.code == abi.E_DEVICE


def test_last_error_is_per_thread():
    lib = abi.load_library()
    lib.skyla_hip_alloc(None, 16, None)
    seen = {}

    def other():
        seen["msg"] = lib.skyla_hip_last_error()
    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == b""
    assert lib.skyla_hip_last_error() != b""


# ---------------------------------------------------------------------------- planner.rs
@pytest.mark.parametrize("dtype,n_in,n_out", [(E.DType.Q4K, 512, 3), (E.DType.Q6K, 256, 5), (E.DType.Q8_0, 96, 7)])
def test_planner_regions_are_a_byte_permutation(dtype, n_in, n_out):
    data = synth.matrix("plan", dtype.name, dtype, n_in, n_out)
    p = E.Planner(1 << 30)
    norm = p.table(np.arange(5, dtype=np.float32))
    m = p.matrix(dtype, n_in, n_out, data)
    out = np.zeros(p.buffer_size(0), np.uint8)
    p.fill(0, out)
    assert np.array_equal(out[norm * 4: norm * 4 + 20].view("<f4"), np.arange(5, dtype=np.float32))
    block, parts = E.LAYOUT[dtype]
    blocks = data.reshape(-1, block)
    rebuilt = np.zeros_like(blocks)
    for i, ((lo, hi), unit) in enumerate(parts):
        start = m.off[i] * unit
        assert start % 16 == 0                     # every region 16-byte aligned
        rebuilt[:, lo:hi] = out[start: start + blocks.shape[0] * (hi - lo)].reshape(-1, hi - lo)
    assert np.array_equal(rebuilt, blocks)


def test_planner_splits_buffers_at_the_cap():
    data = synth.matrix("plan", "big", E.DType.Q4K, 256, 64)   # 9216 bytes
    p = E.Planner(20000)
    ms = [p.matrix(E.DType.Q4K, 256, 64, data) for _ in range(3)]
    assert [m.buf for m in ms] == [0, 0, 1]
    assert all(s <= 20000 for s in p.sizes)


def test_planner_rejects_unsupported():
    p = E.Planner(1 << 20)
    with pytest.raises(ValueError):
        p.matrix(E.DType.Q4K, 100, 1, np.zeros(144, np.uint8))
    with pytest.raises(ValueError):
        p.matrix(E.DType.F16, 256, 1, np.zeros(512, np.uint8))


# ---------------------------------------------------------------------------- kernels.rs / graph.rs
class FakeRecorder:
    def __init__(self):
        self.ops = []

    def dispatch(self, p, groups, push):
        self.ops.append(("dispatch", p, 0, list(groups), list(push)))

    def dispatch_set(self, p, s, groups, push):
        self.ops.append(("dispatch", p, s, list(groups), list(push)))

    def barrier(self):
        self.ops.append(("barrier",))

    def mark(self, label):
        pass


class FakeKernels:
    def __init__(self):
        self.decode = [E.Matvec(["q8a0", "q8a1"], [(l, f"q8e{l}") for l in E.EXPERT_LPR], 64, 8),
                       E.Matvec(["q4a0", "q4a1"], [(l, f"q4e{l}") for l in E.EXPERT_LPR], 64, 8),
                       E.Matvec(["q6a0", "q6a1"], [(l, f"q6e{l}") for l in E.EXPERT_LPR], 64, 8)]
        self.batch = [E.Matvec([f"mm{t}a0", f"mm{t}a1"], [(0, f"mm{t}g")], 64, 128) for t in range(3)]
        self.to_half = "to_half" if E.HALF_INPUTS else None
        self.silu, self.logits, self.route, self.sort, self.combine = "silu", "logits", "route", "sort", "combine"

    matvec = E.Kernels.matvec


def test_experts_lanes_per_row():
    mv = FakeKernels().decode[1]
    assert mv.experts(64) == ("q4e64", 8)
    assert mv.experts(24) == ("q4e32", 16)      # down n_in = 768: 24 units -> 32 lanes per row
    assert mv.experts(12) == ("q4e16", 32)
    assert mv.experts(1000) == ("q4e64", 8)


def test_graph_push_layouts_and_grids():
    r, k = FakeRecorder(), FakeKernels()
    g = E.Graph(r, k, None, None, False)
    q4 = E.QMatrix(E.DType.Q4K, 1, (10, 20, 0, 0), 4096, 1000)
    q6 = E.QMatrix(E.DType.Q6K, 0, (1, 2, 3, 4), 12288, 4096)
    g.matvec(q4, (64, 0), (4160, 0), False, False)
    g.matvec(q6, (64, 0), (128, 0), True, False)
    g.matvec(q4, (64, 4096), (8000, 1024), False, True)
    assert r.ops[0] == ("dispatch", "q4a0", 1, [125, 1, 1], [10, 20, 64, 4160, 4096, 1000, 0, 0, 0])
    assert r.ops[1] == ("dispatch", "q6a1", 0, [512, 1, 1], [1, 2, 3, 4, 64, 128, 12288, 4096, 0, 0, 0])
    assert r.ops[2] == ("dispatch", "mm1a0", 1, [8, 1, E.BATCH // E.MATMUL_TILE_COLS],
                        [10, 20, 0, 0, 64, 8000, 4096, 1000, 4096, 1024, 0, 0, 1])


def test_moe_sequence_decode_and_prefill():
    c = E.Config(n_embd=2048, n_ff=64, n_expert=128, n_expert_used=8, n_ff_expert=768)

    class A:  # arena offsets only
        n, s_embd, x, half = 1000, 2048, 2000, 50000
        moe = E.MoeRegions(logits=3000, ids=4000, weights=4100, gate=5000, up=6000, down=7000, table=8000,
                           list=8300, stride=768)
    gate = E.QMatrix(E.DType.Q4K, 0, (1, 2, 0, 0), 2048, 768)
    down = E.QMatrix(E.DType.Q4K, 0, (5, 6, 0, 0), 768, 2048)
    r = FakeRecorder()
    E.Graph(r, FakeKernels(), A, c, False).moe(gate, gate, down, 77)
    d = [o for o in r.ops if o[0] == "dispatch"]
    assert [o[1] for o in d] == ["logits", "route", "q4e64", "q4e64", "silu", "q4e32", "combine"]
    assert d[0][3:] == ([128, 1, 1], [1000, 77, 3000, 2048, 2048])
    assert d[2][3:] == ([96, 8, 1], [1, 2, 1000, 5000, 2048, 768, 4000, 0, 768])
    assert d[5][3:] == ([128, 8, 1], [5, 6, 5000, 7000, 768, 2048, 4000, 768, 2048])
    assert d[6][3] == [8, 1, 1]
    r = FakeRecorder()
    E.Graph(r, FakeKernels(), A, c, True).moe(gate, gate, down, 77)
    d = [o for o in r.ops if o[0] == "dispatch"]
    half = ["to_half"] if E.HALF_INPUTS else []
    assert [o[1] for o in d] == ["logits", "route", "sort"] + half + ["mm1g", "mm1g", "silu"] + half + [
        "mm1g", "combine"]
    gu = d[3 + len(half)]
    dn = d[6 + 2 * len(half)]
    assert gu[3] == [6, 128, E.BATCH // E.MOE_TILE_COLS]
    assert gu[4][-3:] == [8000, 8300, 8]           # table, list, x_div = n_used for gate/up
    assert dn[4][-1] == 1                          # x_div = 1 for down
    if E.HALF_INPUTS:
        assert d[7][3] == [1, E.BATCH * 8, 1]      # to_half over BATCH * n_used rows
    else:
        assert gu[4][4:6] == [1000, 5000] and dn[4][4] == 5000   # f32 rows read in place


def test_arena_layout_follows_arena_rs():
    class Ctx:
        def alloc_host(self, size):
            return size
    c = E.Config(n_embd=4096, n_ff=12288, n_head=32, n_head_kv=8, head_dim=128, n_vocab=151936)
    a = E.Arena(Ctx(), c, max_ctx=1024)
    assert (a.x, a.s_embd) == (64, 4096)
    assert a.n == 64 + 4096 * E.BATCH
    assert a.s_ff == 12288 and a.s_kv == 1024
    assert a.logits == a.last + 4096
    assert a.buffer == a.size * 4


@pytest.mark.parametrize("n_expert,n_used,msg", [(257, 8, "experts: moe_route"), (128, 17, "per token"),
                                                 (8, 9, "per token"), (64, 0, "per token"),
                                                 (128, 9, "slots")])
def test_arena_rejects_moe_past_kernel_limits(n_expert, n_used, msg):
    """moe_route holds 256 logits and picks at most 16 experts; moe_sort ranks at most 1024
    slots (8 experts x the 128-token chunk): the arena refuses such a model before anything
    is allocated or launched, instead of the kernels clamping silently."""
    c = E.Config(n_embd=256, n_ff=256, n_head=2, n_head_kv=1, n_vocab=64, n_layer=1,
                 n_expert=n_expert, n_expert_used=n_used, n_ff_expert=256)
    with pytest.raises(ValueError, match=msg):
        E.Arena(None, c, 64)
