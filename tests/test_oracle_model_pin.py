"""Pins oracle/model.py's Model (the end-to-end oracle) against an independent float64
forward (tests/model64.py), for the three dense mixes and a qwen3moe model, and shows that
composition mistakes of the kind the pin guards against (swapped norms, a tied head where
the model has its own, a dropped FFN residual, RoPE over adjacent pairs instead of NeoX's
halves, the wrong expert weights) move the logits far past the tolerance."""
import dataclasses

import numpy as np
import pytest

from helpers import rel_l2
from model64 import Model64
from oracle import model as oracle_model
from oracle.model import Model
from skyla_hip import synth

STEPS = 10
TOL = 1e-5


def _setup(kind: str):
    if kind == "moe":
        c = synth.qwen3_config("tiny-moe")
        return c, synth.qwen3moe("pin-moe", c)
    c = dataclasses.replace(synth.qwen3_config("tiny"), n_layer=2)
    return c, synth.qwen3(f"pin-{kind}", c, kind, "random")


def _run(c, oracle_t, ref_t, steps=STEPS):
    m, r = Model(c, oracle_t), Model64(c, ref_t)
    toks = synth.prompt("pin", steps, c.n_vocab)
    errs = [rel_l2(m.forward(t), r.forward(t)) for t in toks]
    return errs, r


@pytest.mark.parametrize("kind", ["q8_0", "q4_k_m", "q4_k_m_mixed", "moe"])
def test_model_matches_float64_forward(kind):
    c, t = _setup(kind)
    errs, r = _run(c, t, t)
    if kind == "moe":   # no routing decision is within f32 noise of a tie
        assert r.route_margin > 1e-3, r.route_margin
    assert max(errs) <= TOL, errs


def test_pin_catches_swapped_norms():
    c, t = _setup("q4_k_m")
    bad = dict(t)
    for l in range(c.n_layer):
        a, f = f"blk.{l}.attn_norm.weight", f"blk.{l}.ffn_norm.weight"
        bad[a], bad[f] = t[f], t[a]
    errs, _ = _run(c, bad, t, 3)
    assert min(errs) > 1e-3, errs


def test_pin_catches_tied_head():
    c, t = _setup("q4_k_m")
    bad = {k: v for k, v in t.items() if k != "output.weight"}   # the oracle ties the head
    errs, _ = _run(c, bad, t, 3)
    assert min(errs) > 1e-1, errs


def test_pin_catches_dropped_ffn_residual(monkeypatch):
    c, t = _setup("q8_0")
    monkeypatch.setattr(oracle_model.so, "swiglu", lambda *a, **k: np.zeros(c.n_embd, np.float32))
    errs, _ = _run(c, t, t, 3)
    assert min(errs) > 1e-2, errs


def test_pin_catches_rope_pairing(monkeypatch):
    """RoPE over adjacent pairs (2i, 2i + 1) instead of NeoX's (i, i + head_dim / 2)."""
    c, t = _setup("q4_k_m")

    def adjacent(x, pos, freqs, mscale):
        a, b = x[0::2].copy(), x[1::2].copy()
        ang = np.float32(pos) * freqs[: a.size]
        x[0::2] = a * np.cos(ang) - b * np.sin(ang)
        x[1::2] = a * np.sin(ang) + b * np.cos(ang)
    monkeypatch.setattr(oracle_model.so, "rope_neox", adjacent)
    errs, _ = _run(c, t, t, 6)
    assert max(errs[1:]) > 10 * TOL, errs   # at position 0 every rotation is the identity


def test_pin_catches_wrong_expert_weights(monkeypatch):
    """Every selected expert weighted 1 / n_used instead of by the softmax of its logit."""
    c, t = _setup("moe")
    moe = oracle_model.so.moe_forward

    def bad(router, gt, g, ut, u, dt, d, n_embd, n_ff, n_expert, used, n, threads=0):
        _, ids, w = moe(router, gt, g, ut, u, dt, d, n_embd, n_ff, n_expert, used, n, threads)
        out = np.zeros(n_embd, np.float32)
        for e in ids:
            rb = len(g) // n_expert
            rd = len(d) // n_expert
            out += oracle_model.so.swiglu(gt, g[e * rb:(e + 1) * rb], ut, u[e * rb:(e + 1) * rb], dt,
                                          d[e * rd:(e + 1) * rd], n_embd, n_ff, n) / used
        return out, ids, w
    monkeypatch.setattr(oracle_model.so, "moe_forward", bad)
    errs, _ = _run(c, t, t, 3)
    assert min(errs) > 1e-3, errs


def _yarn_setup(original_ctx=64.0):
    """YaRN factor 4; an original context of 64 puts the ramp at pairs 0..11, so the
    interpolated pairs turn visibly within the pin's few positions."""
    c = dataclasses.replace(synth.qwen3_config("tiny"), n_layer=2, rope_scaling=(4.0, original_ctx, 1.0))
    return c, synth.qwen3("pin-yarn", c, "q4_k_m", "random")


@pytest.mark.parametrize("original_ctx", [64.0, 32768.0])
def test_model_yarn_matches_float64_forward(original_ctx):
    """Under YaRN scaling (factor 4; over an original context of 64, and of 32768 as the
    reference's R1-0528 Qwen3-8B distill declares) the oracle Model's RoPE (the C
    restatement of rope.rs:36-58) against the float64 forward built from the method."""
    c, t = _yarn_setup(original_ctx)
    errs, _ = _run(c, t, t)
    assert max(errs) <= TOL, errs


def test_pin_catches_yarn_scale_inverted(monkeypatch):
    """The interpolated pairs' frequencies multiplied by the factor instead of divided by it
    (freq_scale inverted) move the logits past three times the pin's tolerance."""
    c, t = _yarn_setup()
    real = oracle_model.so.rope_freqs_yarn

    def inverted(head_dim, theta, factor, original_ctx, attn_factor):
        f, m = real(head_dim, theta, factor, original_ctx, attn_factor)
        base = oracle_model.so.rope_freqs(head_dim, theta)
        return (base * base / f).astype(np.float32), m   # base * (1 / scale) for base * scale
    monkeypatch.setattr(oracle_model.so, "rope_freqs_yarn", inverted)
    errs, _ = _run(c, t, t)
    assert max(errs) > 3 * TOL, errs


def test_pin_catches_yarn_magnitude_dropped(monkeypatch):
    """Dropping YaRN's magnitude (mscale = 1) moves the logits past three times the tolerance."""
    c, t = _yarn_setup()
    real = oracle_model.so.rope_freqs_yarn
    monkeypatch.setattr(oracle_model.so, "rope_freqs_yarn", lambda *a: (real(*a)[0], 1.0))
    errs, _ = _run(c, t, t)
    assert max(errs) > 3 * TOL, errs
