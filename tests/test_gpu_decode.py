"""GPU parity of the decode step around the weight matvecs, through the C-ABI.

Kernel by kernel against the oracle (rmsnorm, QK-norm + RoPE + KV write, split-K attention
and its merge, the embedding gather), then end to end: the engine's decode of seeded random
Qwen3 models against skyla-ref's Model (oracle/model.py), teacher-forced on the oracle's
greedy tokens, with no top-1 disagreement (north_star).  The oracle stores its KV cache the
way the reference's GPU backend does for the precision under test (qkv_prep.comp:48-65:
f16 rows or q8 blocks).  Every step's top-1 is compared: the tests print the number of
disagreements, the smallest oracle top-2 margin met and the worst logits distance, and
assert that no step disagrees.
"""

import numpy as np
import pytest

from helpers import rel_l2, tactics
from oracle import skyla_oracle as so
from oracle.model import Model
from skyla_hip import engine as E
from skyla_hip import synth

pytestmark = pytest.mark.gpu

P = E.KvPrecision
CFG = "test-decode"


class Bench:
    """Tables + a small embedding matrix, arena with KV cache, and the kernels."""

    def __init__(self, ctx, c, precision, tables, max_ctx=256, embd=None, fuse="none"):
        self.ctx, self.c = ctx, c
        p = E.Planner(ctx.max_buffer())
        self.off = {k: p.table(v) for k, v in tables.items()}
        dt, n_rows, data = embd or (E.DType.Q8_0, 16, synth.matrix(CFG, "embd", E.DType.Q8_0, c.n_embd, 16))
        self.embd = p.matrix(dt, c.n_embd, n_rows, data)
        self.weights = E.upload_weights(ctx, p)
        self.a = E.Arena(ctx, c, max_ctx, precision)
        self.k = E.Kernels(ctx, self.weights, self.a.buffer, kv=self.a.kv, c=c, precision=precision,
                           embd_dtype=dt, fuse=fuse)

    def run(self, body, batched=True):
        rec = self.ctx.record(False, lambda r: body(E.Graph(r, self.k, self.a, self.c, batched)))
        try:
            self.ctx.replay(rec)
        finally:
            rec.free()

    def rows(self, off, stride, n, width):
        f = self.a.f32()
        return np.stack([f[off + t * stride: off + t * stride + width] for t in range(n)])

    def put_rows(self, off, stride, rows):
        f = self.a.f32()
        for t, r in enumerate(rows):
            f[off + t * stride: off + t * stride + r.size] = r

    def free(self):
        for b in self.weights:
            b.free()
        self.a.kv.free()
        self.a.buffer.free()


def _cfg(n_embd=512, n_head=4, n_head_kv=2):
    return E.Config(n_embd=n_embd, n_ff=1024, n_head=n_head, n_head_kv=n_head_kv, head_dim=128, n_vocab=16,
                    n_layer=2)


@pytest.mark.parametrize("n_embd", [512, 1056, 8192])
def test_rmsnorm_matches_oracle(ctx, n_embd):
    """Rows of 512 and 1056 (the float4 path, full and ragged) and 8192 (above the
    registers' 4096) against ops.rs rmsnorm."""
    c = _cfg(n_embd)
    g = np.random.default_rng(1)
    w = g.uniform(0.5, 1.5, c.n_embd).astype(np.float32)
    b = Bench(ctx, c, P.F16, {"w": w})
    try:
        x = (g.standard_normal((3, c.n_embd)) * 7).astype(np.float32)
        a = b.a
        b.put_rows(a.x, a.s_embd, x)
        a.set_ctl(0, 0, 3)
        a.buffer.upload()
        b.run(lambda gr: gr.rmsnorm(a.x, b.off["w"], a.n, E.BATCH))
        a.buffer.download()
        got = b.rows(a.n, a.s_embd, 3, c.n_embd)
        for t in range(3):
            want = so.rmsnorm(x[t], w, c.eps)
            assert np.max(np.abs(got[t] - want)) <= 4e-6 * np.max(np.abs(want)), t
    finally:
        b.free()


def _cache(b, l, n_pos):
    """Dequantised K and V of layer l, positions [0, n_pos), from the host mirror."""
    a, c, kvl = b.a, b.c, b.a.kv_layout
    a.kv.download()
    h = a.kv.host()
    kv_dim = c.n_head_kv * c.head_dim

    def read(off, scales, q8):
        if not q8:
            return h.view("<f2")[off: off + n_pos * kv_dim].astype(np.float32).reshape(n_pos, kv_dim)
        q = h.view(np.int8)[off: off + n_pos * kv_dim].astype(np.float32).reshape(n_pos, kv_dim // 32, 32)
        s = h.view("<f2")[scales: scales + n_pos * kv_dim // 32].astype(np.float32).reshape(n_pos, -1, 1)
        return (q * s).reshape(n_pos, kv_dim)
    pr = kvl.precision
    return (read(kvl.keys(l), kvl.key_scales(l), pr.keys_q8), read(kvl.values(l), kvl.value_scales(l), pr.values_q8))


@pytest.mark.parametrize("precision", list(P))
def test_qkv_prep_matches_oracle(ctx, precision):
    c = _cfg()
    g = np.random.default_rng(2)
    qn, kn = g.uniform(0.5, 1.5, 128).astype(np.float32), g.uniform(0.5, 1.5, 128).astype(np.float32)
    freqs = E.rope_frequencies(c)
    b = Bench(ctx, c, precision, {"qn": qn, "kn": kn, "rope": freqs})
    try:
        a, n_tok, pos0 = b.a, 3, 37
        q = (g.standard_normal((n_tok, c.n_head * 128)) * 3).astype(np.float32)
        k = (g.standard_normal((n_tok, c.n_head_kv * 128)) * 3).astype(np.float32)
        v = g.standard_normal((n_tok, c.n_head_kv * 128)).astype(np.float32)
        b.put_rows(a.q, a.s_q, q)
        b.put_rows(a.k, a.s_kv, k)
        b.put_rows(a.v, a.s_kv, v)
        a.set_ctl(0, pos0, n_tok)
        a.buffer.upload()
        b.run(lambda gr: gr.qk_rope(1, b.off["qn"], b.off["kn"], b.off["rope"]))
        a.buffer.download()
        got_q = b.rows(a.q, a.s_q, n_tok, c.n_head * 128)
        K, V = _cache(b, 1, pos0 + n_tok)
        for t in range(n_tok):
            wq, wk = q[t].copy(), k[t].copy()
            for x, heads, w in ((wq, c.n_head, qn), (wk, c.n_head_kv, kn)):
                for h in range(heads):
                    part = x[h * 128:(h + 1) * 128]
                    so.rmsnorm_inplace(part, w, c.eps)
                    so.rope_neox(part, pos0 + t, freqs, 1.0)
            assert np.max(np.abs(got_q[t] - wq)) < 2e-5 * np.max(np.abs(wq)), t
            for got, want, q8 in ((K[pos0 + t], wk, precision.keys_q8), (V[pos0 + t], v[t], precision.values_q8)):
                if not q8:
                    assert np.allclose(got, want.astype(np.float16).astype(np.float32), rtol=2e-3, atol=1e-4)
                else:
                    qq, ss = so.kv_quantize_q8(want)
                    assert np.max(np.abs(got - (qq.reshape(-1, 32) * ss.astype(np.float32)[:, None]).reshape(-1))) \
                        <= 1e-3 * np.max(np.abs(want))
        # the value quantisation itself, exactly (random data: no exact .5 ties)
        if precision.values_q8:
            kvl, kv_dim = a.kv_layout, c.n_head_kv * 128
            h = a.kv.host()
            raw = h.view(np.int8)[kvl.values(1) + pos0 * kv_dim: kvl.values(1) + (pos0 + n_tok) * kv_dim]
            qq, ss = so.kv_quantize_q8(v)
            assert np.array_equal(raw.reshape(qq.shape), qq)
            sc = h.view("<f2")[kvl.value_scales(1) + pos0 * kv_dim // 32:
                               kvl.value_scales(1) + (pos0 + n_tok) * kv_dim // 32]
            assert np.array_equal(sc.view(np.uint16), ss.reshape(-1).view(np.uint16))
    finally:
        b.free()


@pytest.mark.parametrize("precision", list(P))
@pytest.mark.parametrize("n_pos", [1, 5, 64, 65, 190, 4100])
@pytest.mark.parametrize("heads", [(4, 2), (4, 4), (8, 2), (8, 1)])
def test_attention_matches_oracle(ctx, precision, n_pos, heads):
    """Split-K attention + merge over positions [0, ctl[1] + t] for two tokens, against the
    oracle's attention over the same (dequantised) cache entries; 190 positions span three
    splits, 64 / 65 the split boundary, 4100 sixty-five splits (more than the merge's 16
    split groups); 1, 2, 4 and 8 query heads per kv head."""
    c = _cfg(512, *heads)
    g = np.random.default_rng(3 + n_pos)
    b = Bench(ctx, c, precision, {"one": np.ones(128, np.float32)}, max_ctx=max(256, n_pos))
    try:
        a, kvl, kv_dim = b.a, b.a.kv_layout, c.n_head_kv * 128
        K = (g.standard_normal((n_pos, kv_dim)) * 2).astype(np.float32)
        V = g.standard_normal((n_pos, kv_dim)).astype(np.float32)
        h = a.kv.host()
        for off, scales, data, q8 in ((kvl.keys(0), kvl.key_scales(0), K, precision.keys_q8),
                                      (kvl.values(0), kvl.value_scales(0), V, precision.values_q8)):
            if q8:
                qq, ss = so.kv_quantize_q8(data)
                h.view(np.int8)[off: off + data.size] = qq.reshape(-1)
                h.view("<f2")[scales: scales + data.size // 32] = ss.reshape(-1)
            else:
                h.view("<f2")[off: off + data.size] = data.reshape(-1).astype(np.float16)
        a.kv.upload()
        n_tok = min(2, n_pos)
        q = (g.standard_normal((n_tok, c.n_head * 128)) * 0.3).astype(np.float32)
        b.put_rows(a.q, a.s_q, q)
        a.set_ctl(0, n_pos - n_tok, n_tok)
        a.buffer.upload()
        b.run(lambda gr: gr.attend(0))
        a.buffer.download()
        got = b.rows(a.attn, a.s_attn, n_tok, c.n_head * 128)
        Kd, Vd = _cache(b, 0, n_pos)
        for t in range(n_tok):
            m = n_pos - n_tok + t + 1
            want = so.attention(q[t], Kd[:m].reshape(-1), Vd[:m].reshape(-1), m, c.n_head, c.n_head_kv, 128)
            # both sides round each of m terms in f32: the oracle sequentially, the kernel
            # in split partials, so the allowance grows like sqrt(m) past a few hundred
            assert rel_l2(got[t], want) < 1e-6 * max(2.0, np.sqrt(m) / 16), (t, m)
    finally:
        b.free()


@pytest.mark.parametrize("dt", [E.DType.Q8_0, E.DType.Q4K, E.DType.Q6K])
def test_embed_gathers_rows_bit_exact(ctx, dt):
    c = _cfg()
    rows = 40
    data = synth.matrix(CFG, f"embd-{dt.name}", dt, c.n_embd, rows)
    b = Bench(ctx, c, P.F16, {"one": np.ones(4, np.float32)}, embd=(dt, rows, data))
    try:
        a = b.a
        toks = [0, 17, rows - 1, 17]
        u = a.u32()
        u[a.tokens: a.tokens + len(toks)] = toks
        a.set_ctl(toks[0], 0, len(toks))
        a.buffer.upload()
        b.run(lambda gr: gr.embed(b.embd))
        a.buffer.download()
        got = b.rows(a.x, a.s_embd, len(toks), c.n_embd)
        rb = E.row_bytes(dt, c.n_embd)
        for t, tok in enumerate(toks):
            want = so.dequantize(int(dt), data[tok * rb:(tok + 1) * rb], c.n_embd)
            assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), t
    finally:
        b.free()


class Top1:
    """Top-1 bookkeeping of a teacher-forced decode: disagreements, the smallest oracle top-2
    margin (relative to the logits' std) and the worst logits relative L2."""

    def __init__(self):
        self.flips, self.steps, self.worst, self.margin = 0, 0, 0.0, np.inf
        self.last = None

    def judge(self, gl, ol):
        self.steps += 1
        self.worst = max(self.worst, rel_l2(gl, ol))
        top = np.argsort(ol)[::-1][:2]
        self.margin = min(self.margin, float((ol[top[0]] - ol[top[1]]) / ol.std()))
        self.flips += int(np.argmax(gl)) != so.argmax(ol)
        self.last = so.argmax(ol)

    def report(self, what):
        print(f"{what}: {self.steps} steps, top-1 disagreements {self.flips}, smallest oracle "
              f"top-2 margin {self.margin:.2e} std, worst logits rel-L2 {self.worst:.2e}")



@pytest.mark.parametrize("fuse", ["none", "qkv", "ffn", "all", "auto"])
@pytest.mark.parametrize("quant", ["q8_0", "q4_k_m", "q4_k_m_mixed"])
@pytest.mark.parametrize("precision", [P.F16, P.F16_KEYS_Q8_VALUES])
def test_decode_top1_against_oracle(ctx, quant, precision, fuse):
    """32 greedy steps of a 3-layer model, with each of the decode graph's fusion levels.
    q4_k_m_mixed is the q4_k_m model's seeded weights with attn_v Q6_K in even layers (q, k
    and v of one layer in two types).  Seeded apart, that layout drew an ill-conditioned
    model: FFN activations of 1e6, and 2.5e-4 of noise on its stored k/v rows moved the
    oracle's own logits by up to 97%, so no rounding-level bound could hold."""
    c = synth.qwen3_config("tiny")
    tensors = synth.qwen3(f"{CFG}-{'q4_k_m' if quant == 'q4_k_m_mixed' else quant}", c, quant, "random")
    oracle = Model(c, tensors, (precision.keys_q8, precision.values_q8))
    eng = E.Engine(ctx, tensors, c, 64, precision, fuse=fuse)
    try:
        t = Top1()
        tok = synth.prompt(CFG, 1, c.n_vocab)[0]
        for _ in range(32):                      # 32 greedy steps, teacher-forced
            t.judge(eng.step(tok), oracle.forward(tok))
            tok = t.last
        t.report(f"tiny {quant} {precision.name} fuse={fuse}")
        assert t.flips == 0, t.flips
        assert t.worst < 1e-3, t.worst
    finally:
        eng.free()


def test_prefill_then_decode_against_oracle(ctx):
    """A 150-token prompt through Engine::prefill (a full 128-token chunk, then 22), then greedy
    decode: the batched GEMMs, qkv_prep / attention over many tokens at once and take_last."""
    c = synth.qwen3_config("tiny")
    tensors = synth.qwen3(f"{CFG}-prefill", c, "q4_k_m", "random")
    prompt = synth.prompt(f"{CFG}-prefill", 150, c.n_vocab)
    oracle = Model(c, tensors, (False, True))
    eng = E.Engine(ctx, tensors, c, 192, P.F16_KEYS_Q8_VALUES)
    try:
        gl = eng.prefill(prompt)
        for t in prompt:
            ol = oracle.forward(t)
        assert eng.pos == oracle.pos == 150
        assert rel_l2(gl, ol) < 2e-2
        assert int(np.argmax(gl)) == so.argmax(ol)
        tok = so.argmax(ol)
        for _ in range(8):
            gl, ol = eng.step(tok), oracle.forward(tok)
            assert rel_l2(gl, ol) < 2e-2
            assert int(np.argmax(gl)) == so.argmax(ol)
            tok = so.argmax(ol)
    finally:
        eng.free()


# Oracle top-2 margin (relative to the logits' std) under which a prompt that went through
# the f16-operand prefill GEMM may flip with 8-bit values: fixed, not scaled by the error.
NEAR = 2e-2


@pytest.mark.parametrize("prompt_path", ["step", "prefill"])
@pytest.mark.parametrize("precision", [P.F16, P.F16_KEYS_Q8_VALUES])
def test_config1_qwen3_06b_greedy(ctx, precision, prompt_path):
    """Config 1 (Qwen3-0.6B, Q8_0 weights, tied head, norms 1.0): the 16-token prompt of
    uniform ids, then 64 greedy decode steps, both sides fed the oracle's tokens.

    prompt_path "step": the prompt token by token through the decode graph, as skyla-ref's
    CPU model takes it; every matvec multiplies f32 activations in f32, and no step of the
    65 may disagree.  "prefill": the prompt through Engine::prefill, whose batched GEMM
    multiplies f16 operands as the reference's matmul.comp does (about 1e-3 relative on its
    k/v rows); with f16 keys and values no step may disagree either.  With 8-bit values a
    value that the GEMM's rounding moves across a quantisation step moves by max|v| / 127,
    which puts about 1% relative L2 on the logits: a disagreement is then allowed only at
    a step whose oracle top-2 margin is below NEAR, at most one, and all are reported."""
    c = synth.qwen3_config("qwen3-0.6b")
    tensors = synth.qwen3("qwen3-0.6b-q8_0", c, "q8_0", "ones")
    prompt = synth.prompt("qwen3-0.6b-q8_0", 16, c.n_vocab)
    oracle = Model(c, tensors, (precision.keys_q8, precision.values_q8))
    eng = E.Engine(ctx, tensors, c, 96, precision)
    try:
        t = Top1()
        if prompt_path == "prefill":
            gl = eng.prefill(prompt)
            for tok in prompt:
                ol = oracle.forward(tok)
            t.judge(gl, ol)
        else:
            for tok in prompt[:-1]:
                eng.step(tok)
                oracle.forward(tok)
            t.judge(eng.step(prompt[-1]), oracle.forward(prompt[-1]))
        for _ in range(64):
            t.judge(eng.step(t.last), oracle.forward(t.last))
        t.report(f"config 1 {precision.name} prompt by {prompt_path}")
        assert eng.pos == oracle.pos == 80
        if prompt_path == "prefill" and precision.values_q8:
            assert t.flips <= 1 and (t.flips == 0 or t.margin < NEAR), (t.flips, t.margin)
            assert t.worst < 2e-2, t.worst
        else:
            assert t.flips == 0, (t.flips, t.margin)
            # 8-bit values: a v value the ~1e-6 matvec differences move across a
            # quantisation step moves by max|v| / 127 (a few of 2.3 million per run)
            assert t.worst < (1e-2 if prompt_path == "prefill" else 5e-3 if precision.values_q8 else 1e-3), t.worst
    finally:
        eng.free()


def test_engine_from_gguf_file(ctx, tmp_path):
    """A model written to a GGUF file and loaded back (gguf.py: reader.rs, Config::from_gguf)
    decodes exactly as the same tensors handed over in memory."""
    from skyla_hip import gguf as G
    c = synth.qwen3_config("tiny")
    tensors = synth.qwen3(f"{CFG}-gguf", c, "q4_k_m", "random")
    path = str(tmp_path / "tiny.gguf")
    G.write_model(path, "qwen3", c, tensors)
    g = G.Gguf(path)
    c2, t2 = G.config_from_gguf(g), G.tensors_from_gguf(g)
    e1, e2 = E.Engine(ctx, tensors, c, 32), E.Engine(ctx, t2, c2, 32)
    try:
        for tok in (5, 77, 1999):
            assert np.array_equal(e1.step(tok), e2.step(tok))
    finally:
        e1.free()
        e2.free()


@pytest.mark.parametrize("fuse", ["none", "auto"])
@pytest.mark.parametrize("arch,original_ctx", [("qwen3", 64.0), ("qwen3vl", 32768.0)])
def test_yarn_model_from_gguf_against_oracle(ctx, tmp_path, arch, original_ctx, fuse):
    """A qwen3 model with YaRN RoPE scaling (factor 4; over an original context of 64, so the
    interpolated pairs turn visibly within the test, and 32768 as the R1-0528 Qwen3-8B
    distill declares) written to a GGUF file (and as qwen3vl text), read back
    (RopeScaling::from_gguf, rope.rs:14-58) and decoded through the engine: the host's
    frequency table and magnitude go to the attention kernels.  24 greedy steps
    teacher-forced against the oracle Model (its own C restatement of the table), then a
    40-token prompt through Engine::prefill: no top-1 disagreement."""
    import dataclasses
    from skyla_hip import gguf as G
    c = dataclasses.replace(synth.qwen3_config("tiny"), rope_scaling=(4.0, original_ctx, 1.0))
    tensors = synth.qwen3(f"{CFG}-yarn", c, "q4_k_m", "random")
    path = str(tmp_path / "yarn.gguf")
    G.write_model(path, arch, c, tensors)
    g = G.Gguf(path)
    c2, t2 = G.config_from_gguf(g), G.tensors_from_gguf(g)
    assert c2.rope_scaling == (4.0, original_ctx, 1.0) and abs(c2.rope_mscale - 1.1386294) < 1e-6
    precision = P.F16_KEYS_Q8_VALUES
    oracle = Model(c2, t2, (precision.keys_q8, precision.values_q8))
    eng = E.Engine(ctx, t2, c2, 96, precision, fuse=fuse)
    try:
        top = Top1()
        tok = synth.prompt(f"{CFG}-yarn", 1, c.n_vocab)[0]
        for _ in range(24):
            top.judge(eng.step(tok), oracle.forward(tok))
            tok = top.last
        top.report(f"yarn {arch} {original_ctx:g} {fuse}")
        assert top.flips == 0, (top.flips, top.margin)
        assert top.worst < 5e-3, top.worst
        eng.reset()
        oracle.reset()
        prompt = synth.prompt(f"{CFG}-yarn-prefill", 40, c.n_vocab)
        gl = eng.prefill(prompt)
        for t_ in prompt:
            ol = oracle.forward(t_)
        assert int(np.argmax(gl)) == so.argmax(ol)
        assert rel_l2(gl, ol) < 2e-2, rel_l2(gl, ol)
    finally:
        eng.free()


@pytest.mark.parametrize("precision", list(P))
@pytest.mark.parametrize("pos0", [0, 37, 64, 130])
@pytest.mark.parametrize("heads", [(4, 2), (8, 1), (4, 4)])
def test_attention_prep_equals_qkv_prep_then_attention(ctx, precision, pos0, heads):
    """attention_prep (one token: qkv_prep folded into the attention) leaves the same cache
    bytes and the same attention output, bit for bit, as qkv_prep then attention; the new
    position first in its split (64, 130 - 128 = 2) and alone (0)."""
    c = _cfg(512, *heads)
    g = np.random.default_rng(7 + pos0)
    qn, kn = g.uniform(0.5, 1.5, 128).astype(np.float32), g.uniform(0.5, 1.5, 128).astype(np.float32)
    tables = {"qn": qn, "kn": kn, "rope": E.rope_frequencies(c)}
    b = Bench(ctx, c, precision, tables, fuse="qkv")
    try:
        a = b.a
        kv_host = a.kv.host()
        kv_host[:] = g.integers(0, 256, kv_host.size, dtype=np.uint8)
        kv_host.view("<f2")[:] = g.standard_normal(kv_host.size // 2).astype(np.float16)  # finite rows
        kv0 = kv_host.copy()
        q = (g.standard_normal(c.n_head * 128) * 3).astype(np.float32)
        k = (g.standard_normal(c.n_head_kv * 128) * 3).astype(np.float32)
        v = g.standard_normal(c.n_head_kv * 128).astype(np.float32)
        outs = []
        for fused in (False, True):
            kv_host[:] = kv0
            a.kv.upload()
            b.put_rows(a.q, a.s_q, q[None])
            b.put_rows(a.k, a.s_kv, k[None])
            b.put_rows(a.v, a.s_kv, v[None])
            a.set_ctl(0, pos0, 1)
            a.buffer.upload()
            if fused:
                b.run(lambda gr: gr.attend_prep(1, b.off["qn"], b.off["kn"], b.off["rope"]), batched=False)
            else:
                b.run(lambda gr: (gr.qk_rope(1, b.off["qn"], b.off["kn"], b.off["rope"]), gr.attend(1)),
                      batched=False)
            a.buffer.download()
            a.kv.download()
            outs.append((b.rows(a.attn, a.s_attn, 1, c.n_head * 128)[0].copy(), a.kv.host().copy()))
        (o0, kv_a), (o1, kv_b) = outs
        assert np.array_equal(kv_a, kv_b)
        assert np.isfinite(o1).all()
        assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32))
    finally:
        b.free()


def _stored_rows(kvl, kv_host, n_pos, kv_dim, layer=0):
    """A layer's first n_pos cache rows as the attention reads them back (f16 keys; 8-bit
    values times their f16 scale), from the host mirror synth.fill_kv wrote."""
    pr = kvl.precision
    assert not pr.keys_q8 and pr.values_q8
    k = kv_host.view("<f2")[kvl.keys(layer): kvl.keys(layer) + n_pos * kv_dim].astype(np.float32)
    q = kv_host.view(np.int8)[kvl.values(layer): kvl.values(layer) + n_pos * kv_dim].astype(np.float32)
    sc = kv_host.view("<f2")[kvl.value_scales(layer): kvl.value_scales(layer) + n_pos * kv_dim // 32]
    v = (q.reshape(-1, 32) * sc.astype(np.float32)[:, None]).reshape(n_pos, kv_dim)
    return k.reshape(n_pos, kv_dim), v


def test_config5_qwen3_8b_prefilled_contexts(ctx):
    """Config 5 at full size: the 36-layer Qwen3-8B Q4_K_M decode step (Q6_K head and
    even-layer ffn_down, every layer its own HBM copy of layer 0 / 1's seeded matrices) with
    the f16-key / 8-bit-value cache pre-filled with N(0,1) rows to 16384 positions (256
    splits of 64 merged) and then to 1024, three teacher-forced steps at each, against the
    oracle Model holding the same stored rows: top-1 equal at every step, logits within
    2e-2 relative L2 (engine.rs:137-152, arena.rs:83-181, kv.rs:33-88).  Every layer's
    cache rows are drawn from their own seed and the oracle holds each layer's own rows, so
    a layer reading another layer's cache slot would not match."""
    c = synth.qwen3_config("qwen3-8b")
    t = synth.qwen3("qwen3-8b-q4_k_m", c, "q4_k_m", "ones", shared_layers=True)
    kv_dim = c.n_head_kv * c.head_dim
    eng = E.Engine(ctx, t, c, 16384 + 8, P.F16_KEYS_Q8_VALUES)
    try:
        kvl, kv_host = eng.arena.kv_layout, eng.arena.kv.host()
        synth.fill_kv(kvl, kv_host, 16384, kv_dim, "qwen3-8b-q4_k_m")
        eng.arena.kv.upload()
        rows = [_stored_rows(kvl, kv_host, 16384, kv_dim, l) for l in range(c.n_layer)]
        assert not np.array_equal(rows[0][0][:4], rows[1][0][:4])  # distinct rows per layer
        # 16384 first: the 1024 case's steps overwrite positions 1024..1026 of the fill
        for n_ctx in (16384, 1024):
            oracle = Model(c, t, (False, True))
            oracle.load_cache([k[:n_ctx] for k, _ in rows], [v[:n_ctx] for _, v in rows])
            eng.pos = n_ctx
            top = Top1()
            tok = synth.prompt("qwen3-8b-q4_k_m", 1, c.n_vocab)[0]
            for _ in range(3):
                top.judge(eng.step(tok), oracle.forward(tok))
                tok = top.last
            top.report(f"config 5 at {n_ctx} positions")
            assert eng.pos == oracle.pos == n_ctx + 3
            assert top.flips == 0, (n_ctx, top.flips, top.margin)
            assert top.worst < 2e-2, (n_ctx, top.worst)
    finally:
        eng.free()


@pytest.mark.parametrize("precision", [P.F16, P.F16_KEYS_Q8_VALUES])
def test_moe_model_from_gguf_against_oracle(ctx, tmp_path, precision):
    """A qwen3moe model (16 experts, top 4, expert FFN 256, f32 routers) written to a GGUF
    file, read back (reader.rs, Config::from_gguf) and decoded through the engine's MoE
    layer (graph/moe.rs:42-80 inside graph.rs:158-185) against the oracle Model's Ffn::Moe
    arm (ffn.rs:58-76 from model.rs:113-114): 24 greedy steps teacher-forced, no top-1
    disagreement; then a 40-token prompt through Engine::prefill (the grouped GEMMs)."""
    from skyla_hip import gguf as G
    c = synth.qwen3_config("tiny-moe")
    tensors = synth.qwen3moe(f"{CFG}-moe", c)
    path = str(tmp_path / "tiny-moe.gguf")
    G.write_model(path, "qwen3moe", c, tensors)
    g = G.Gguf(path)
    c2, t2 = G.config_from_gguf(g), G.tensors_from_gguf(g)
    assert (c2.n_expert, c2.n_expert_used, c2.n_ff_expert, c2.n_layer) == (16, 4, 256, 2)
    assert t2["blk.0.ffn_gate_exps.weight"][4] == 16 and t2["blk.1.ffn_gate_inp.weight"].shape == (16, c.n_embd)
    oracle = Model(c2, t2, (precision.keys_q8, precision.values_q8))
    eng = E.Engine(ctx, t2, c2, 96, precision)
    try:
        top = Top1()
        tok = synth.prompt(f"{CFG}-moe", 1, c.n_vocab)[0]
        for _ in range(24):
            top.judge(eng.step(tok), oracle.forward(tok))
            tok = top.last
        top.report(f"qwen3moe {precision.name}")
        assert top.flips == 0, (top.flips, top.margin)
        assert top.worst < 1e-3, top.worst
        eng.reset()
        oracle.reset()
        prompt = synth.prompt(f"{CFG}-moe-prefill", 40, c.n_vocab)
        gl = eng.prefill(prompt)
        for t_ in prompt:
            ol = oracle.forward(t_)
        err = rel_l2(gl, ol)
        print(f"qwen3moe {precision.name} 40-token prefill: logits rel-L2 {err:.2e}")
        assert int(np.argmax(gl)) == so.argmax(ol)
        assert err < 2e-2, err
    finally:
        eng.free()


def test_split_buckets_same_logits(ctx):
    """Recordings over fewer attention splits (Engine.recording picks the smallest bucket
    that covers the positions in play) give the logits of the arena-wide recording bit for
    bit, prefill and decode: the splits past a token's position do no work in either."""
    c = synth.qwen3_config("tiny")
    tensors = synth.qwen3(f"{CFG}-q4_k_m", c, "q4_k_m", "random")
    eng = E.Engine(ctx, tensors, c, 40 * E.ATTENTION_CHUNK, P.F16_KEYS_Q8_VALUES)
    full_p = full_d = None
    try:
        a = eng.arena
        assert a.n_split == 40 and E.SPLIT_BUCKETS[0] < a.n_split
        full_p = E.record(ctx, eng.kernels, eng.weights, a, c, True, False, a.n_split)
        full_d = E.record(ctx, eng.kernels, eng.weights, a, c, False, False, a.n_split)
        prompt = synth.prompt(f"{CFG}-buckets", 150, c.n_vocab)
        got = eng.prefill(prompt)                      # chunks at positions 0 and 128: 2 and 4 splits
        assert eng.recording(True, 128 + E.BATCH) is not full_p
        eng.reset()
        for i in range(0, len(prompt), E.BATCH):
            chunk = prompt[i: i + E.BATCH]
            eng.load(chunk)
            ctx.replay(full_p)
            eng.pos += len(chunk)
        want = eng.logits()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        tok = int(np.argmax(want))
        for _ in range(3):                             # decode from position 150
            pos = eng.pos
            got = eng.step(tok)
            eng.pos = pos
            eng.load([tok], batched=False)
            ctx.replay(full_d)
            eng.pos += 1
            want = eng.logits()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
            tok = int(np.argmax(want))
    finally:
        for rec in (full_p, full_d):
            if rec is not None:
                rec.free()
        eng.free()


def test_single_split_direct_same_logits(ctx):
    """Single-token steps whose positions all lie in the first 64 replay the one-split
    recording, where attention_prep1 writes the merged rows itself (no merge launch): the
    logits of the arena-wide recording (attention_prep over 40 splits, then the merge) bit
    for bit, on both sides of the one-split bound (positions 60..67)."""
    c = synth.qwen3_config("tiny")
    tensors = synth.qwen3(f"{CFG}-q4_k_m", c, "q4_k_m", "random")
    eng = E.Engine(ctx, tensors, c, 40 * E.ATTENTION_CHUNK, P.F16_KEYS_Q8_VALUES)
    full_d = None
    try:
        a = eng.arena
        assert E.SPLIT_BUCKETS[0] == 1 and eng.kernels.attn_prep1 is not None
        full_d = E.record(ctx, eng.kernels, eng.weights, a, c, False, False, a.n_split)
        one = eng.recording(False, 1)
        assert one.launches() < full_d.launches()      # one merge launch fewer per layer
        prompt = synth.prompt(f"{CFG}-direct", 60, c.n_vocab)
        eng.prefill(prompt)
        tok = int(np.argmax(eng.logits()))
        for _ in range(8):                             # positions 60..67
            pos = eng.pos
            got = eng.step(tok)
            eng.pos = pos
            eng.load([tok], batched=False)
            ctx.replay(full_d)
            eng.pos += 1
            want = eng.logits()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos
            tok = int(np.argmax(want))
    finally:
        if full_d is not None:
            full_d.free()
        eng.free()


@pytest.mark.parametrize("ctx_len", [60, 1500])
def test_rope_table_same_logits(ctx, ctx_len):
    """Decode steps whose attention_prep reads the step's rope pairs from rope_table (one
    launch per step) against the same steps with every workgroup computing them: the same
    logits bit for bit, at one split and past the one-split bucket."""
    c = synth.qwen3_config("tiny")
    tensors = synth.qwen3(f"{CFG}-q4_k_m", c, "q4_k_m", "random")
    got = {}
    for table in ("1", "0"):
        with tactics(rope_table=table):
            eng = E.Engine(ctx, tensors, c, 32 * E.ATTENTION_CHUNK, P.F16_KEYS_Q8_VALUES)
        try:
            assert (eng.kernels.rope_table is not None) == (table == "1")
            eng.prefill(synth.prompt(f"{CFG}-rope", ctx_len, c.n_vocab))
            tok = int(np.argmax(eng.logits()))
            rows = []
            for _ in range(3):
                rows.append(eng.step(tok).copy())
                tok = int(np.argmax(rows[-1]))
            got[table] = np.stack(rows)
        finally:
            eng.free()
    assert np.array_equal(got["1"].view(np.uint32), got["0"].view(np.uint32))


@pytest.mark.parametrize("quant", ["q4_k_m", "q4_k_m_mixed"])
def test_prefill_prepass_joined_same_logits(ctx, quant):
    """Prefill with each dense matmul's f16 row prepass joined to the launch that writes its
    rows (rmsnorm_half_rows before q/k/v and before gate/up, silu_half_rows before down)
    against the prepass as a launch of its own (tactic xhalf_join=0): three launches fewer
    per layer in a prefill recording, and the same logits bit for bit, through the prefill
    (two chunks, the second ragged) and the decode steps after it."""
    c = synth.qwen3_config("tiny")
    tensors = synth.qwen3(f"{CFG}-{quant}", c, quant, "random")
    prompt = synth.prompt(f"{CFG}-join", E.BATCH + 22, c.n_vocab)
    got, n_launch = {}, {}
    for join in ("1", "0"):
        with tactics(xhalf_join=join):
            eng = E.Engine(ctx, tensors, c, 8 * E.ATTENTION_CHUNK, P.F16_KEYS_Q8_VALUES)
            try:
                rows = [eng.prefill(prompt).copy()]
                n_launch[join] = eng.recording(True, E.BATCH).launches()
                tok = int(np.argmax(rows[-1]))
                for _ in range(3):
                    rows.append(eng.step(tok).copy())
                    tok = int(np.argmax(rows[-1]))
                got[join] = np.stack(rows)
            finally:
                eng.free()
    assert n_launch["0"] - n_launch["1"] == 3 * c.n_layer, n_launch
    assert np.array_equal(got["1"].view(np.uint32), got["0"].view(np.uint32))
