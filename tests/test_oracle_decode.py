"""CPU pins of the oracle's decode-step functions (skyla-ref/src/ops.rs, rope.rs,
model.rs:131-170) and of the engine's KV layout (kv.rs).  Each check is a closed form, an
invariant or a float64 brute force, chosen so that a dropped term, a wrong index (the GQA
head mapping, the RoPE pair) or a transposed operand fails."""
import numpy as np
import pytest

from oracle import skyla_oracle as so
from oracle.model import Model
from skyla_hip import engine as E
from skyla_hip import synth


def test_rope_freqs_closed_form():
    f = so.rope_freqs(128, 1e6)
    assert f.shape == (64,) and f[0] == 1.0
    want = 1e6 ** (-2.0 * np.arange(64) / 128.0)
    assert np.allclose(f, want, rtol=4e-7, atol=0)
    # the product computes the same table on the host for the kernels
    assert np.array_equal(E.rope_frequencies(E.Config(n_embd=128, rope_theta=1e6)), f)


def test_rope_neox_rotation():
    g = np.random.default_rng(1)
    x = g.standard_normal(128).astype(np.float32)
    f = so.rope_freqs(128, 1e6)
    y = x.copy()
    so.rope_neox(y, 0, f, 1.0)
    assert np.array_equal(y, x)                       # position 0 is the identity
    for pos in (1, 17, 1000):
        y = x.copy()
        so.rope_neox(y, pos, f, 1.0)
        ang = pos * f.astype(np.float64)
        a, b = x[:64].astype(np.float64), x[64:].astype(np.float64)
        want = np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)])
        assert np.allclose(y, want, rtol=0, atol=2e-5 * (1 + pos * 1e-3))
        # pairs (i, i + 64) keep their length
        assert np.allclose(np.hypot(y[:64], y[64:]), np.hypot(x[:64], x[64:]), rtol=1e-5)


def test_rmsnorm_inplace_invariants():
    g = np.random.default_rng(2)
    x = g.standard_normal(128).astype(np.float32)
    y = x.copy()
    so.rmsnorm_inplace(y, np.ones(128, np.float32), 0.0)
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 1e-6
    z = (x * np.float32(8.0)).astype(np.float32)      # exact scaling by a power of two
    so.rmsnorm_inplace(z, np.ones(128, np.float32), 0.0)
    assert np.array_equal(z, y)
    w = g.uniform(0.5, 1.5, 128).astype(np.float32)
    v = x.copy()
    so.rmsnorm_inplace(v, w, 1e-6)
    assert np.allclose(v, y * w, rtol=2e-6)


@pytest.mark.parametrize("n_head,n_kv", [(4, 4), (4, 2), (8, 1)])
def test_attention_brute_force_and_special_cases(n_head, n_kv):
    g = np.random.default_rng(3)
    hd, kv_dim = 128, n_kv * 128
    q = g.standard_normal(n_head * hd).astype(np.float32)
    # one position: softmax is exactly 1, so each head returns its kv head's value row
    k1, v1 = g.standard_normal(kv_dim).astype(np.float32), g.standard_normal(kv_dim).astype(np.float32)
    out = so.attention(q, k1, v1, 1, n_head, n_kv, hd).reshape(n_head, hd)
    rep = n_head // n_kv
    for h in range(n_head):
        assert np.array_equal(out[h], v1[(h // rep) * hd:(h // rep + 1) * hd])
    # float64 brute force over 37 positions
    n_pos = 37
    K = g.standard_normal((n_pos, kv_dim)).astype(np.float32)
    V = g.standard_normal((n_pos, kv_dim)).astype(np.float32)
    out = so.attention(q, K.reshape(-1), V.reshape(-1), n_pos, n_head, n_kv, hd).reshape(n_head, hd)
    for h in range(n_head):
        kh = K[:, (h // rep) * hd:(h // rep + 1) * hd].astype(np.float64)
        vh = V[:, (h // rep) * hd:(h // rep + 1) * hd].astype(np.float64)
        s = kh @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        w = np.exp(s - s.max())
        w /= w.sum()
        assert np.allclose(out[h], w @ vh, rtol=0, atol=2e-5)
    # equal keys: uniform weights, the mean value row
    Ke = np.tile(K[:1], (n_pos, 1))
    out = so.attention(q, Ke.reshape(-1), V.reshape(-1), n_pos, n_head, n_kv, hd).reshape(n_head, hd)
    assert np.allclose(out[0], V[:, :hd].astype(np.float64).mean(0), atol=1e-5)


def test_oracle_model_reset_replays():
    c = synth.qwen3_config("tiny")
    c.n_layer = 2
    m = Model(c, synth.qwen3("tiny", c, "q4_k_m", "random"))
    a = [m.forward(t) for t in (3, 9, 27)]
    m.reset()
    b = [m.forward(t) for t in (3, 9, 27)]
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    assert all(np.isfinite(x).all() for x in a)
    assert not np.array_equal(a[1], a[2])


@pytest.mark.parametrize("precision", list(E.KvPrecision))
def test_kv_layout_regions(precision):
    """kv.rs:18-88: per-layer key, value and scale regions tile the buffer without overlap."""
    n_layer, max_ctx, kv_dim = 3, 64, 1024
    kv = E.KvLayout(precision, [True] * n_layer, max_ctx, kv_dim)
    kw = 1 if kv.precision.keys_q8 else 2
    vw = 1 if kv.precision.values_q8 else 2
    spans = []
    for l in range(n_layer):
        spans.append((kv.keys(l) * kw, kv.per_layer * kw))
        spans.append((kv.values(l) * vw, kv.per_layer * vw))
        if kv.precision.keys_q8:
            spans.append((kv.key_scales(l) * 2, kv.per_layer // 32 * 2))
        if kv.precision.values_q8:
            spans.append((kv.value_scales(l) * 2, kv.per_layer // 32 * 2))
    spans.sort()
    assert spans[0][0] == 0
    for (o0, n0), (o1, _) in zip(spans, spans[1:]):
        assert o0 + n0 == o1
    assert spans[-1][0] + spans[-1][1] == kv.bytes()


def test_kv_quantize_q8_closed_forms():
    """qkv_prep.comp:40-65: the block maximum maps to +-127, zero blocks stay zero with a zero
    scale, ties round to even, and a stored row is within half a step (plus the f16 scale's
    rounding) of the value."""
    # max |y| = 127 gives s = 1 exactly: q = rint(y), ties to even
    y = np.zeros(64, np.float32)
    y[:6] = [127.0, -127.0, 2.5, 3.5, -0.5, 1.49]
    q, s = so.kv_quantize_q8(y)
    assert s.dtype == np.float16 and s.shape == (2,)
    assert s[0] == 1.0 and s[1] == 0.0
    assert list(q[:6]) == [127, -127, 2, 4, 0, 1]
    assert not q[32:].any()
    g = np.random.default_rng(5)
    y = (g.standard_normal(4096) * 3).astype(np.float32)
    q, s = so.kv_quantize_q8(y)
    blocks = y.reshape(-1, 32)
    assert np.array_equal(np.abs(q.reshape(-1, 32)).max(1), np.full(128, 127))
    s32 = np.abs(blocks).max(1).astype(np.float64) / 127
    back = so.kv_stored(y, True).reshape(-1, 32).astype(np.float64)
    bound = s32[:, None] / 2 * (1 + 1e-6) + 127 * np.abs(s.astype(np.float64) - s32)[:, None]
    assert (np.abs(back - blocks) <= bound).all()
    # f16 rows: round to nearest even of the f16 format
    assert np.array_equal(so.kv_stored(y, False), y.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("shared", [False, True])
def test_fill_kv_rows_per_layer(shared):
    """synth.fill_kv (the N(0,1) pre-fill): each layer's first n_pos rows hold f16 keys and
    8-bit values whose 32-value blocks reach +-127, about N(0,1); the layers' rows differ
    (each its own seed), or with `shared` every layer holds the same rows."""
    layout = E.KvLayout(E.KvPrecision.F16_KEYS_Q8_VALUES, [True] * 3, 96, 256)
    host = np.zeros(layout.bytes(), np.uint8)
    synth.fill_kv(layout, host, 64, 256, "test-fill", shared=shared)
    n = 64 * 256
    keys = [host.view("<f2")[layout.keys(l): layout.keys(l) + n].astype(np.float32) for l in range(3)]
    vals = [host.view(np.int8)[layout.values(l): layout.values(l) + n] for l in range(3)]
    scl = [host.view("<f2")[layout.value_scales(l): layout.value_scales(l) + n // 32] for l in range(3)]
    for l in (1, 2):
        same = np.array_equal(keys[0], keys[l]) and np.array_equal(vals[0], vals[l])
        assert same == shared, l
    for l in range(3):
        assert np.array_equal(np.abs(vals[l].reshape(-1, 32).astype(np.int32)).max(1), np.full(n // 32, 127))
        v = vals[l].reshape(-1, 32).astype(np.float32) * scl[l].astype(np.float32)[:, None]
        for x in (keys[l], v.reshape(-1)):
            assert abs(float(x.mean())) < 0.05 and abs(float(x.std()) - 1.0) < 0.05
        # rows past n_pos stay untouched
        assert not host.view("<f2")[layout.keys(l) + n: layout.keys(l) + 96 * 256].any()


def test_model_load_cache_per_layer():
    """Model.load_cache with one row set per layer: each layer's attention reads its own
    rows (a forward differs from the one with layer 0's rows in every layer)."""
    from oracle.model import Model
    c = synth.qwen3_config("tiny")
    t = synth.qwen3("test-load-cache", c, "q4_k_m", "random")
    kv_dim = c.n_head_kv * c.head_dim
    g = synth.rng("test-load-cache", "rows")
    rows = [(g.standard_normal((5, kv_dim)).astype(np.float32), g.standard_normal((5, kv_dim)).astype(np.float32))
            for _ in range(c.n_layer)]
    per, same = Model(c, t, (False, False)), Model(c, t, (False, False))
    per.load_cache([k for k, _ in rows], [v for _, v in rows])
    same.load_cache(rows[0][0], rows[0][1])
    assert per.pos == same.pos == 5
    for l in range(c.n_layer):
        assert np.array_equal(per.k_cache[l][0], rows[l][0].reshape(-1))
        assert np.array_equal(same.k_cache[l][0], rows[0][0].reshape(-1))
    assert not np.array_equal(per.forward(1), same.forward(1))


YARN = [(128, 1e6, 4.0, 32768.0, 1.0), (128, 1e6, 8.0, 4096.0, 0.7), (64, 1e4, 2.0, 2048.0, 1.0),
        (128, 5e5, 16.0, 8192.0, 1.2)]


@pytest.mark.parametrize("hd,theta,factor,ctx,attn", YARN)
def test_rope_yarn_closed_form(hd, theta, factor, ctx, attn):
    """The oracle's YaRN table (rope.rs:36-58 in f32) against the method in float64
    (tests/model64.yarn64): pairs below the beta_fast dimension keep theta^(-2i/d), pairs
    above the beta_slow one take 1/factor of it, the ramp between is linear, and the
    magnitude is attn_factor (1 + 0.1 ln factor); within f32 rounding of each."""
    from model64 import yarn64
    f, m = so.rope_freqs_yarn(hd, theta, factor, ctx, attn)
    f64, m64 = yarn64(hd, theta, factor, ctx, attn)
    assert np.allclose(f, f64, rtol=2e-6, atol=0) and abs(m - m64) <= 2e-6 * m64
    base = so.rope_freqs(hd, theta)
    kept = np.isclose(f64, theta ** (-2.0 * np.arange(hd // 2) / hd), rtol=1e-12)
    scaled = np.isclose(f64, theta ** (-2.0 * np.arange(hd // 2) / hd) / factor, rtol=1e-12)
    assert kept.any() and scaled.any() and not (kept & scaled).any()
    assert np.allclose(f[kept], base[kept], rtol=1e-7) and np.allclose(f[scaled], base[scaled] / factor, rtol=2e-7)


def test_rope_yarn_factor_one_is_plain():
    """YaRN with factor 1 leaves every frequency as theta^(-2i/d) and the magnitude at
    attn_factor."""
    f, m = so.rope_freqs_yarn(128, 1e6, 1.0, 32768.0, 1.0)
    assert np.array_equal(f, so.rope_freqs(128, 1e6)) and m == 1.0


@pytest.mark.parametrize("hd,theta,factor,ctx,attn", YARN)
def test_rope_yarn_host_table_equals_oracle(hd, theta, factor, ctx, attn):
    """The engine's host table (engine.rope_table, what the attention kernels read) and its
    magnitude: the oracle's bits."""
    c = E.Config(n_embd=hd, head_dim=hd, rope_theta=theta, rope_scaling=(factor, ctx, attn))
    f, m = E.rope_table(c)
    of, om = so.rope_freqs_yarn(hd, theta, factor, ctx, attn)
    assert np.array_equal(f.view(np.uint32), of.view(np.uint32))
    assert np.float32(m) == np.float32(om) and c.rope_mscale == m
