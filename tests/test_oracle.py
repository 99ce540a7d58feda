"""Pins the CPU oracle (oracle/skyla_oracle.c) before it is trusted as the GPU checker.

The reference ships no tests, fixtures or golden vectors for this path (its checks live in
the absent skyla-platform CLI), and its Rust cannot be built here.  Each oracle function is
therefore pinned by something a plausible mistake would fail:
  * f16 -> f32: all 65,536 patterns against numpy's IEEE binary16 (an independent
    implementation); f32 -> f16 round-to-nearest-even on edge cases and random values;
  * dequantisation: closed-form known-answer blocks built with an independent *packer*
    (the inverse of q4k_scale_min), exhaustive (scale, min) round trips through the 6-bit
    packing, signed Q6_K extremes, all Q8_0 quants, and bit equality with the separate
    numpy restatement (oracle/quant_np.py) on seeded random blocks;
  * the committed golden fixtures in tests/golden (generated from closed forms);
  * matvec: one-hot inputs select a dequantised column exactly; float64 agreement;
    independence from the thread count; linearity;
  * route: brute force over sorted logits with lowest-index tie breaking; softmax in
    float64; moe_sort: numpy's stable argsort; swiglu / moe_forward: float64 compositions.
"""
import json
import os

import numpy as np
import pytest

from oracle import quant_np as qn
from oracle import skyla_oracle as so
from skyla_hip import synth
from skyla_hip.engine import DType

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------------------- f16
def test_f16_to_f32_all_patterns():
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([so.f16_to_f32(int(i)) for i in h], np.float32)
    ref = h.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # NaNs: quiet, sign and payload kept (half 2.7.1 / F16C behaviour)
    gb = got[nan].view(np.uint32)
    hb = h[nan]
    assert np.all(np.isnan(got[nan]))
    assert np.array_equal(gb & 0x80000000, (hb & 0x8000) << 16)
    assert np.array_equal(gb & 0x003FE000, (hb & 0x01FF) << 13)
    assert np.all(gb & 0x00400000)


def test_f32_to_f16_round_to_nearest_even():
    edge = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05, 5.9604645e-08,
                     2.9802322e-08, 2.98023259e-08, 8.940697e-08, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11,
                     np.inf, -np.inf], np.float32)
    rnd = np.random.default_rng(1).standard_normal(20000).astype(np.float32) * np.float32(100)
    tiny = np.random.default_rng(2).uniform(-1e-4, 1e-4, 20000).astype(np.float32)
    for x in np.concatenate([edge, rnd, tiny]):
        assert so.f32_to_f16(float(x)) == int(np.float16(x).view(np.uint16)), x


# ---------------------------------------------------------------------------- packing helpers
def pack_q4k_scales(sc, m):
    """Inverse of q4k_scale_min, from the 6-bit packing definition."""
    s = [0] * 12
    for j in range(4):
        s[j] = sc[j] & 63
        s[j + 4] = m[j] & 63
    for j in range(4, 8):
        k = j - 4
        s[8 + k] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
        s[k] |= (sc[j] >> 4) << 6
        s[k + 4] |= (m[j] >> 4) << 6
    return bytes(s)


def f16le(v: float) -> bytes:
    return np.float16(v).tobytes()


def q4k_block(d, dmin, sc, m, nib_lo, nib_hi) -> bytes:
    qs = bytearray(128)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = (nib_lo[c][l] & 0xF) | ((nib_hi[c][l] & 0xF) << 4)
    return f16le(d) + f16le(dmin) + pack_q4k_scales(sc, m) + bytes(qs)


def test_q4k_scale_min_exhaustive_round_trip():
    for j in range(8):
        for sc in range(64):
            for m in range(0, 64, 3):
                scs = [(sc + 7 * i) % 64 for i in range(8)]
                ms = [(m + 11 * i) % 64 for i in range(8)]
                scs[j], ms[j] = sc, m
                assert so.q4k_scale_min(j, pack_q4k_scales(scs, ms)) == (sc, m)


def test_q4k_known_answer():
    # d = 1, dmin = 0.5, scales j+1, mins j, nibble l%16: value = (j+1) q - 0.5 j
    sc = [j + 1 for j in range(8)]
    mn = [j for j in range(8)]
    nib = [[l % 16 for l in range(32)] for _ in range(4)]
    nib_hi = [[(l * 7 + c) % 16 for l in range(32)] for c in range(4)]
    blk = q4k_block(1.0, 0.5, sc, mn, nib, nib_hi)
    out = so.dequantize(int(DType.Q4K), blk, 256)
    want = np.empty(256, np.float32)
    for c in range(4):
        for l in range(32):
            want[64 * c + l] = (2 * c + 1) * (l % 16) - 0.5 * (2 * c)
            want[64 * c + 32 + l] = (2 * c + 2) * ((l * 7 + c) % 16) - 0.5 * (2 * c + 1)
    assert np.array_equal(out, want)


def test_q4k_high_scale_bits():
    # scales and mins >= 16 exercise the upper 2 bits for j >= 4
    sc = [63, 62, 33, 16, 63, 48, 17, 32]
    mn = [0, 63, 15, 16, 47, 63, 31, 1]
    nib = [[15] * 32 for _ in range(4)]
    blk = q4k_block(0.25, 2.0, sc, mn, nib, nib)
    out = so.dequantize(int(DType.Q4K), blk, 256).reshape(8, 32)
    for j in range(8):
        assert np.all(out[j] == np.float32(0.25 * sc[j] * 15 - 2.0 * mn[j]))


def q6k_block(ql, qh, sc, d) -> bytes:
    return bytes(ql) + bytes(qh) + np.array(sc, np.int8).tobytes() + f16le(d)


def test_q6k_extremes_and_negative_scales():
    # q = 0 everywhere -> -32 * sc * d ; q = 63 -> 31 * sc * d
    for fill, q in ((0x00, -32), (0xFF, 31)):
        sc = [-64, -1, 1, 64, -7, 9, 127, -128, 3, -3, 5, -5, 64, -64, 0, 2]
        blk = q6k_block([fill] * 128, [fill] * 64, sc, 0.5)
        out = so.dequantize(int(DType.Q6K), blk, 256)
        for i in range(256):
            half, r = divmod(i, 128)
            g, l = divmod(r, 32)
            s = sc[8 * half + l // 16 + 2 * g]
            assert out[i] == np.float32(0.5 * s * q), i


def test_q6k_bit_layout():
    # one 6-bit value per (half, group, l): choose q = (i * 37) % 64, pack, dequant with d=1, sc=1
    q = [(i * 37) % 64 for i in range(256)]
    ql, qh = [0] * 128, [0] * 64
    for half in range(2):
        for l in range(32):
            v = [q[128 * half + 32 * g + l] for g in range(4)]
            ql[64 * half + l] = (v[0] & 0xF) | ((v[2] & 0xF) << 4)
            ql[64 * half + 32 + l] = (v[1] & 0xF) | ((v[3] & 0xF) << 4)
            qh[32 * half + l] = (v[0] >> 4) | ((v[1] >> 4) << 2) | ((v[2] >> 4) << 4) | ((v[3] >> 4) << 6)
    out = so.dequantize(int(DType.Q6K), q6k_block(ql, qh, [1] * 16, 1.0), 256)
    assert np.array_equal(out, np.array(q, np.float32) - 32)


def test_q8_0_all_quants():
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8)
    blocks = b"".join(f16le(0.5) + q[i: i + 32].tobytes() for i in range(0, 256, 32))
    out = so.dequantize(int(DType.Q8_0), blocks, 256)
    assert np.array_equal(out, q.astype(np.float32) * np.float32(0.5))


@pytest.mark.parametrize("dtype,n", [(DType.Q4K, 256 * 64), (DType.Q6K, 256 * 64), (DType.Q8_0, 32 * 512)])
def test_c_and_numpy_restatements_agree_bitwise(dtype, n):
    data = synth.matrix("pin", dtype.name, dtype, n, 1)
    a = so.dequantize(int(dtype), data, n)
    b = qn.dequantize(int(dtype), data)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_golden_fixtures():
    with open(os.path.join(GOLDEN, "dequant_known_answers.json")) as fh:
        cases = json.load(fh)
    assert len(cases) >= 6
    for c in cases:
        blk = bytes.fromhex(c["block_hex"])
        out = so.dequantize(c["ggml_type"], blk, len(c["expected_f32_hex"]) // 8)
        want = np.frombuffer(bytes.fromhex(c["expected_f32_hex"]), "<f4")
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), c["name"]


def test_row_bytes_and_errors():
    assert so.row_bytes(int(DType.Q4K), 4096) == 2304
    assert so.row_bytes(int(DType.Q4K), 12288) == 6912
    assert so.row_bytes(int(DType.Q6K), 12288) == 10080
    assert so.row_bytes(int(DType.Q8_0), 1024) == 1088
    assert so.row_bytes(int(DType.Q4K), 100) == -2      # not a multiple of 256
    assert so.row_bytes(7, 256) == -1                    # unsupported ggml type
    with pytest.raises(ValueError):
        so.dequantize(7, b"\0" * 64, 16)


# ---------------------------------------------------------------------------- matvec
@pytest.mark.parametrize("dtype,n_in", [(DType.Q4K, 512), (DType.Q6K, 512), (DType.Q8_0, 96)])
def test_matvec_one_hot_selects_column(dtype, n_in):
    n_out = 9
    data = synth.matrix("pin-mv", dtype.name, dtype, n_in, n_out)
    w = so.dequantize(int(dtype), data, n_in * n_out).reshape(n_out, n_in)
    for k in (0, 1, n_in // 2 + 3, n_in - 1):
        x = np.zeros(n_in, np.float32)
        x[k] = 1.0
        assert np.array_equal(so.matvec(int(dtype), data, n_in, n_out, x), w[:, k])


@pytest.mark.parametrize("dtype,n_in,n_out", [(DType.Q4K, 1024, 33), (DType.Q6K, 768, 17), (DType.Q8_0, 224, 40)])
def test_matvec_float64_threads_linearity(dtype, n_in, n_out):
    data = synth.matrix("pin-mv2", dtype.name, dtype, n_in, n_out)
    w = qn.dequantize(int(dtype), data).reshape(n_out, n_in).astype(np.float64)
    x = synth.activations("pin-mv2", "x", n_in)
    z = synth.activations("pin-mv2", "z", n_in)
    y1 = so.matvec(int(dtype), data, n_in, n_out, x, threads=1)
    y7 = so.matvec(int(dtype), data, n_in, n_out, x, threads=7)
    assert np.array_equal(y1, y7)                          # rows never split across threads
    want = w @ x.astype(np.float64)
    assert np.max(np.abs(y1 - want)) <= 1e-5 * np.max(np.abs(w) @ np.abs(x.astype(np.float64)))
    yz = so.matvec(int(dtype), data, n_in, n_out, z)
    ys = so.matvec(int(dtype), data, n_in, n_out, (x + z).astype(np.float32))
    assert np.allclose(ys, y1 + yz, rtol=1e-4, atol=1e-4)


def test_matvec_sequential_sum_from_negative_zero():
    # all-negative-zero products sum to -0.0 (core's f32 Sum starts at -0.0)
    blk = f16le(-0.0) + bytes(32)
    y = so.matvec(int(DType.Q8_0), blk, 32, 1, np.ones(32, np.float32))
    assert np.signbit(y[0]) and y[0] == 0.0


def test_matmul_is_per_token_matvec():
    dtype, n_in, n_out = DType.Q4K, 512, 24
    data = synth.matrix("pin-mm", "w", dtype, n_in, n_out)
    x = synth.activations("pin-mm", "x", (5, n_in))
    y = so.matmul(int(dtype), data, n_in, n_out, x)
    for t in range(5):
        assert np.array_equal(y[t], so.matvec(int(dtype), data, n_in, n_out, x[t]))


# ---------------------------------------------------------------------------- route, sort, ffn
def test_route_brute_force_and_ties():
    g = np.random.default_rng(9)
    n_embd, n_expert, used = 64, 128, 8
    router = g.standard_normal((n_expert, n_embd)).astype(np.float32)
    n = g.standard_normal(n_embd).astype(np.float32)
    ids, w = so.route(router, n, used)
    logits = np.array([so.dot(router[e], n) for e in range(n_expert)], np.float32)
    order = sorted(range(n_expert), key=lambda e: (-float(logits[e]), e))[:used]
    assert list(ids) == order
    v = logits[order].astype(np.float64)
    assert np.allclose(w, np.exp(v - v.max()) / np.exp(v - v.max()).sum(), rtol=1e-6)
    # exact ties keep expert order (stable sort)
    router_t = np.zeros((n_expert, n_embd), np.float32)
    router_t[[9, 3, 70, 5], 0] = 1.0
    ids, w = so.route(router_t, np.ones(n_embd, np.float32), 6)
    assert list(ids) == [3, 5, 9, 70, 0, 1]
    assert np.allclose(w[:4], w[0]) and np.allclose(w.sum(), 1.0)


def test_moe_sort_is_stable_counting_sort():
    g = np.random.default_rng(4)
    ids = g.integers(0, 128, 1024).astype(np.uint32)
    table, lst = so.moe_sort(ids, 128)
    counts = np.bincount(ids, minlength=128)
    assert np.array_equal(table[:, 0], counts)
    assert np.array_equal(table[:, 1], np.concatenate([[0], np.cumsum(counts)[:-1]]))
    assert np.array_equal(lst, np.argsort(ids, kind="stable"))


def test_swiglu_and_moe_forward_float64():
    n_embd, n_ff, n_expert, used = 256, 256, 8, 2
    t = int(DType.Q4K)
    gate = synth.matrix("pin-ffn", "g", DType.Q4K, n_embd, n_ff, n_expert)
    up = synth.matrix("pin-ffn", "u", DType.Q4K, n_embd, n_ff, n_expert)
    down = synth.matrix("pin-ffn", "d", DType.Q4K, n_ff, n_embd, n_expert)
    router = synth.router("pin-ffn", "r", n_expert, n_embd)
    n = synth.activations("pin-ffn", "n", n_embd)
    G = qn.dequantize(t, gate).reshape(n_expert, n_ff, n_embd).astype(np.float64)
    U = qn.dequantize(t, up).reshape(n_expert, n_ff, n_embd).astype(np.float64)
    D = qn.dequantize(t, down).reshape(n_expert, n_embd, n_ff).astype(np.float64)
    out, ids, w = so.moe_forward(router, t, gate, t, up, t, down, n_embd, n_ff, n_expert, used, n)
    want = np.zeros(n_embd)
    x = n.astype(np.float64)
    for e, wt in zip(ids, w):
        g, u = G[e] @ x, U[e] @ x
        want += wt * (D[e] @ (g / (1 + np.exp(-g)) * u))
    assert np.allclose(out, want, rtol=1e-4, atol=1e-5)
    e0 = int(ids[0])
    sw = so.swiglu(t, gate[e0 * n_ff * 144 * n_embd // 256:], t, up[e0 * n_ff * 144 * n_embd // 256:], t,
                   down[e0 * n_embd * 144 * n_ff // 256:], n_embd, n_ff, n)
    g, u = G[e0] @ x, U[e0] @ x
    assert np.allclose(sw, D[e0] @ (g / (1 + np.exp(-g)) * u), rtol=1e-4, atol=1e-5)


def test_softmax_silu_argmax():
    x = np.array([1.0, 3.0, 3.0, -2.0], np.float32)
    s = so.softmax(x)
    ref = np.exp(x - 3.0) / np.exp(x - 3.0).sum()
    assert np.allclose(s, ref, rtol=1e-6)
    assert so.argmax(x) == 2                      # max_by keeps the last maximum
    assert abs(so.silu(1.5) - 1.5 / (1 + np.exp(-1.5))) < 1e-6


# ---------------------------------------------------------------------------- off-path helpers
def test_rmsnorm_closed_forms():
    """ops.rs:1-16.  Constant x = c with eps = 0 gives r = 1/|c| exactly; a 3-4 pair gives
    mean square 12.5; float64 agreement on random data (catches n-1, missing eps or sqrt)."""
    w = np.linspace(-2, 2, 64).astype(np.float32)
    got = so.rmsnorm(np.full(64, 2.0, np.float32), w, 0.0)
    assert np.array_equal(got, w)                          # 2 * 0.5 * w, exact
    got = so.rmsnorm(np.array([3.0, 4.0], np.float32), np.ones(2, np.float32), 0.0)
    assert np.allclose(got, np.array([3.0, 4.0]) / np.sqrt(12.5), rtol=2e-7)
    x = synth.rng("oracle", "rms").standard_normal(4096).astype(np.float32)
    w = synth.rng("oracle", "rmsw").standard_normal(4096).astype(np.float32)
    want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.allclose(so.rmsnorm(x, w, 1e-6), want, rtol=1e-5, atol=1e-6)


def test_quantize_q8_0_rounding_and_round_trip():
    """quant.rs:91-101: d = amax/127 stored as f16, q = round-half-away(x/d) clamped to
    +-127; ragged tails quantise the values they have; a zero block has d = 0."""
    x = np.zeros(40, np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 2.5, -2.5, 0.49
    x[32:] = [-8.0, 4.0, 0, 0, 0, 0, 0, 1.0]                # second, ragged block: amax 8
    b = so.quantize_q8_0(x)
    assert b.size == 2 * 34
    assert b[:2].view("<f2")[0] == 1.0                     # d = 127/127
    q = b[2:34].view(np.int8)
    assert list(q[:4]) == [127, 3, -3, 0]                  # half away from zero
    d2 = float(b[34:36].view("<f2")[0])
    assert d2 == float(np.float16(8.0 / 127.0))
    q2 = b[36:44].view(np.int8)
    assert q2[0] == -127 and q2[1] == round(4.0 * (127.0 / 8.0))
    assert not b[44:].any()                                # bytes past the tail untouched
    z = so.quantize_q8_0(np.zeros(32, np.float32))
    assert not z.any()
    r = synth.rng("oracle", "q8rt").standard_normal(32 * 64).astype(np.float32)
    back = so.dequantize(int(DType.Q8_0), so.quantize_q8_0(r), r.size)
    d = np.abs(r.reshape(-1, 32)).max(1).astype(np.float64) / 127.0
    d16 = d.astype(np.float16).astype(np.float64)           # the stored scale
    bound = np.repeat(0.5 * d + 127.0 * np.abs(d16 - d), 32) * 1.001 + 1e-7
    assert np.all(np.abs(back.astype(np.float64) - r) <= bound)
