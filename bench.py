#!/usr/bin/env python3
"""Benchmark of Skyla's quantized weight path on one MI355X.

Workload (the config the headline metric is quoted on): the decode
matvecs of Qwen3-8B, per layer Q 4096->4096, K and V 4096->1024, O 4096->4096 (ACCUM),
gate and up 4096->12288 (all Q4_K) and down 12288->4096 (Q6_K, ACCUM), for all 36 layers.
Each layer has its own copy of the weights in HBM (4.37 GB in total, 17x the 256 MB
Infinity Cache), so every step streams the weights from HBM as a real decode token does.
One step = one token's pass over the 36 layers = one replay of a recording of 252
dispatches, issued exactly as skyla-engine's Graph::matvec issues them.

value = algorithmic bytes of the step / step time, where algorithmic bytes per matvec =
weight bytes + 4 n_in + 4 n_out (+ 4 n_out more for ACCUM's read of y).  Inputs are
resident in HBM before timing starts.

Also reported: matvec-only decode tok/s (1 / step time), the dominant kernel's roofline
(matvec_q4k; average launch duration from HIP events on the launch stream), a measured HBM
stream-read probe, the prefill GEMM at M = 512 (config 3) as TFLOP/s, the MoE layer of
config 4 (decode token and 128-token prefill chunk), the end-to-end Qwen3-8B Q4_K_M decode
of config 5 at KV contexts 1024 and 16384 (tok/s), and the CPU oracle (restatement of
skyla-ref Matrix::matvec) timed on this host over a bounded sample.

  python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "skyla-kernel_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from skyla_hip import engine as E  # noqa: E402
from skyla_hip import synth  # noqa: E402
from skyla_hip.abi import Context  # noqa: E402

# Recordings replay as one HIP graph; with --eager they replay as direct launches of the
# same launch list (the runtime's profiled-recording path), for tools that trace launches.
EAGER = False
FUSE = "auto"  # the decode graph's fusion level in the end-to-end runs (Engine fuse)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, vendor peak
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense FP16 MFMA, vendor peak

CONFIG = "qwen3-8b"
N_LAYER = 36
N_EMBD, N_FF, N_KV = 4096, 12288, 1024
# (name, dtype, n_in, n_out, accum)
LAYER = [
    ("q", E.DType.Q4K, N_EMBD, N_EMBD, False),
    ("k", E.DType.Q4K, N_EMBD, N_KV, False),
    ("v", E.DType.Q4K, N_EMBD, N_KV, False),
    ("o", E.DType.Q4K, N_EMBD, N_EMBD, True),
    ("gate", E.DType.Q4K, N_EMBD, N_FF, False),
    ("up", E.DType.Q4K, N_EMBD, N_FF, False),
    ("down", E.DType.Q6K, N_FF, N_EMBD, True),
]


def algo_bytes(dtype, n_in, n_out, accum) -> int:
    return n_out * E.row_bytes(dtype, n_in) + 4 * n_in + 4 * n_out + (4 * n_out if accum else 0)


class DecodeWorkload:
    """36 layers of config-2 matvecs, laid out by the engine's planner."""

    def __init__(self, ctx: Context, n_layer: int = N_LAYER, tactic=None):
        self.ctx = ctx
        self.data = {name: synth.matrix(CONFIG, name, dt, n_in, n_out) for name, dt, n_in, n_out, _ in LAYER}
        planner = E.Planner(ctx.max_buffer())
        self.layers = []
        for _ in range(n_layer):
            self.layers.append({name: planner.matrix(dt, n_in, n_out, self.data[name])
                                for name, dt, n_in, n_out, _ in LAYER})
        self.weights = E.upload_weights(ctx, planner)
        self.weight_bytes = sum(b.size for b in self.weights)
        # activation regions: n (4096), attn (4096), x (4096), q/k/v, gate/up (12288)
        s_e, s_f = N_EMBD, N_FF
        self.off = {}
        o = 64
        for name, width in [("n", s_e), ("attn", s_e), ("x", s_e), ("q", s_e), ("k", N_KV), ("v", N_KV),
                            ("gate", s_f), ("up", s_f)]:
            self.off[name] = o
            o += width
        self.arena = ctx.alloc_host(o * 4)
        f = self.arena.as_f32()
        g = synth.rng(CONFIG, "activations")
        f[64:] = g.standard_normal(o - 64, dtype=np.float32)
        self.arena.as_u32()[2] = 1
        self.arena.upload()
        self.k = E.Kernels(ctx, self.weights, self.arena, kquant_tactic=tactic)
        self.step_bytes = n_layer * sum(algo_bytes(dt, n_in, n_out, acc) for _, dt, n_in, n_out, acc in LAYER)

    def _layer(self, g: E.Graph, lw, only=None):
        a = self.off
        io = {"q": ("n", "q"), "k": ("n", "k"), "v": ("n", "v"), "o": ("attn", "x"),
              "gate": ("n", "gate"), "up": ("n", "up"), "down": ("gate", "x")}
        stages = [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]
        for st in stages:
            for name in st:
                if only is not None and name not in only:
                    continue
                acc = name in ("o", "down")
                xi, yo = io[name]
                g.matvec(lw[name], (a[xi], 0), (a[yo], 0), acc, False)
            g.r.barrier()

    def record(self, only=None, profile=False):
        def body(r):
            g = E.Graph(r, self.k, None, None, False)
            for lw in self.layers:
                self._layer(g, lw, only)
            r.host_barrier()
        return self.ctx.record(profile or EAGER, body)

    def bytes_of(self, only) -> int:
        return len(self.layers) * sum(algo_bytes(dt, n_in, n_out, acc) for name, dt, n_in, n_out, acc in LAYER
                                      if name in only)

    def free(self):
        for b in self.weights:
            b.free()
        self.arena.free()


def time_replays(ctx: Context, rec, warmup: int, steps: int) -> tuple[float, list[float]]:
    """Wall seconds for `steps` synchronous replays, and per-replay device ns (HIP events)."""
    for _ in range(warmup):
        ctx.replay(rec)
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx.replay(rec)
    wall = time.perf_counter() - t0
    dev = [ctx.replay_timed(rec) for _ in range(max(3, min(steps, 10)))]
    return wall, dev


# (threads, loads in flight per lane, non-temporal) of the probe sweep; (256, 4, 0) is the
# reference's bandwidth.comp form
PROBE_FORMS = [(256, 4, 0), (512, 4, 0), (1024, 4, 0), (256, 8, 0), (256, 16, 0), (512, 8, 0),
               (1024, 8, 0), (256, 4, 1), (256, 8, 1), (256, 16, 1), (512, 8, 1), (1024, 8, 1)]


def hbm_probe(ctx: Context, gib: float = 2.0) -> tuple[float, dict]:
    """Stream-read bandwidth of the bandwidth kernel (bandwidth.comp) over `gib` GiB: the
    best over a sweep of workgroup sizes, loads in flight per lane, non-temporal loads and
    grid sizes (workgroups per CU), with the form that reached it."""
    n_bytes = int(gib * (1 << 30)) // 16 * 16
    src = ctx.alloc_host(n_bytes)
    dst = ctx.alloc_host(1 << 25)
    n_vec4 = n_bytes // 16
    best, form = 0.0, {}
    try:
        for t, depth, nt in PROBE_FORMS:
            spec = [t] if (depth, nt) == (4, 0) else [t, depth] + ([1] if nt else [])
            p = ctx.create_pipeline("bandwidth", 2, 4, spec)
            try:
                p.bind_buffers([src, dst])
                for per_cu in (1, 2, 4, 8, 16, 32):
                    groups = 256 * per_cu
                    if groups * t * 4 > dst.size:   # dst holds one word per thread
                        continue
                    ns = ctx.time_dispatch(p, [groups, 1, 1], [n_vec4], 8)
                    gbs = n_bytes / min(ns[2:])  # bytes per ns == GB/s
                    if gbs > best:
                        best, form = gbs, {"threads": t, "depth": depth, "nontemporal": bool(nt),
                                           "workgroups": groups}
            finally:
                p.free()
    finally:
        src.free()
        dst.free()
    return best, form


def calibrate(ctx: Context, mib: int = 1024) -> dict:
    """Known-size traffic for scaling hardware byte counters: one bandwidth-kernel pass that
    reads `mib` MiB (writes nothing), then one device-to-device copy of `mib` / 4 MiB
    (reads and writes that many bytes)."""
    n = mib << 20
    src = ctx.alloc_host(n)
    dst = ctx.alloc_host(1 << 20)
    p = ctx.create_pipeline("bandwidth", 2, 4, [256])
    p.bind_buffers([src, dst])
    ctx.time_dispatch(p, [256 * 8 * 4, 1, 1], [n // 16], 1)
    p.free()
    dst.free()
    m = n // 4
    cdst = ctx.alloc_host(m)
    cdst.copy_from(0, src, 0, m)
    cdst.free()
    src.free()
    return {"bandwidth__256_read_bytes": n, "copy_bytes": m}


def prefill_gemm(ctx: Context, m_tok: int = 512) -> dict:
    """Config 3: Q (Q4_K 4096->4096), gate (Q4_K 4096->12288) and down (Q6_K 12288->4096) at
    M = 512 tokens of f16-valued N(0,1) activations.  The engine's matmul reads f32 rows
    (HALF_INPUTS is off on this backend), so the f16 values are stored widened, exactly.
    Each GEMM's time includes the runtime's f16 row prepass of its input."""
    out = {}
    for name, dt, n_in, n_out in [("q", E.DType.Q4K, N_EMBD, N_EMBD), ("gate", E.DType.Q4K, N_EMBD, N_FF),
                                  ("down", E.DType.Q6K, N_FF, N_EMBD)]:
        data = synth.matrix(CONFIG, name, dt, n_in, n_out)
        planner = E.Planner(ctx.max_buffer())
        copies = 4
        ms = [planner.matrix(dt, n_in, n_out, data) for _ in range(copies)]
        weights = E.upload_weights(ctx, planner)
        s_in, s_out = n_in, n_out
        x_off = 64
        y_off = x_off + s_in * m_tok + 64
        arena = ctx.alloc_host((y_off + s_out * m_tok + 64) * 4)
        x = synth.activations("qwen3-8b-prefill", f"x-{m_tok}-{n_in}", (m_tok, n_in)).astype(np.float16)
        if E.HALF_INPUTS:
            xin = (2 * x_off, s_in)
            arena.host().view("<f2")[2 * x_off: 2 * x_off + x.size] = x.reshape(-1)
        else:
            xin = (x_off, s_in)
            arena.as_f32()[x_off: x_off + x.size] = x.reshape(-1).astype(np.float32)
        arena.as_u32()[2] = m_tok
        arena.upload()
        k = E.Kernels(ctx, weights, arena)
        z = -(-m_tok // E.MATMUL_TILE_COLS)

        def body(r, k=k, ms=ms):  # a barrier after each: no GEMM shares another's f16 row prepass
            g = E.Graph(r, k, None, None, True)
            for i in range(8):
                m = ms[i % copies]
                g.matvec(m, xin, (y_off, s_out), False, True, groups_z=z)
                r.barrier()
        rec = ctx.record(EAGER, body)
        for _ in range(3):
            ctx.replay(rec)
        dev = min(ctx.replay_timed(rec) for _ in range(5)) / 8
        flops = 2.0 * m_tok * n_in * n_out
        out[name] = {"us": round(dev / 1e3, 2), "tflops": round(flops / dev / 1e3, 1),
                     "mfma_frac": round(flops / dev / 1e3 / MFMA_F16_PEAK_TFLOPS, 4)}
        rec.free()
        for b in weights:
            b.free()
        arena.free()
    return out


MOE_CFG = "qwen3-30b-a3b-moe"
MOE_EMBD, MOE_FF, MOE_EXPERT, MOE_USED = 2048, 768, 128, 8


def moe_layers(ctx: Context, n_layer: int = 12, n_tok: int = 128) -> dict:
    """Config 4: Qwen3-30B-A3B-style MoE layer (128 experts, top-8, Q4_K gate/up/down of
    2048x768 / 768x2048 per expert, f32 router), as skyla-engine's Graph::moe sequence
    (graph/moe.rs:42-80), over `n_layer` distinct copies of the layer (4 GB at 12) so the
    selected experts stream from HBM.  Decode: one token through the layers; prefill: one
    128-token chunk.  Bytes per layer = distinct selected experts x 3 expert matrices +
    the 1 MiB router (the algorithmic bytes of the MoE row)."""
    c = E.Config(n_embd=MOE_EMBD, n_ff=64, n_expert=MOE_EXPERT, n_expert_used=MOE_USED, n_ff_expert=MOE_FF)
    router = synth.router(MOE_CFG, "router", MOE_EXPERT, MOE_EMBD)
    data = {name: synth.matrix(MOE_CFG, f"{name}_exps", E.DType.Q4K, n_in, n_out, MOE_EXPERT)
            for name, n_in, n_out in [("gate", MOE_EMBD, MOE_FF), ("up", MOE_EMBD, MOE_FF), ("down", MOE_FF, MOE_EMBD)]}
    p = E.Planner(ctx.max_buffer())
    layers = []
    for _ in range(n_layer):
        layers.append((p.matrix(E.DType.Q4K, MOE_EMBD, MOE_FF, data["gate"]),
                       p.matrix(E.DType.Q4K, MOE_EMBD, MOE_FF, data["up"]),
                       p.matrix(E.DType.Q4K, MOE_FF, MOE_EMBD, data["down"]),
                       p.table(router.reshape(-1))))
    weights = E.upload_weights(ctx, p)
    a = E.Arena(ctx, c)
    k = E.Kernels(ctx, weights, a.buffer)
    expert_bytes = 3 * MOE_FF * E.row_bytes(E.DType.Q4K, MOE_EMBD)  # gate + up + down of one expert
    router_bytes = MOE_EXPERT * MOE_EMBD * 4
    out = {"layers": n_layer, "weight_bytes": sum(b.size for b in weights)}
    for mode, tokens in (("decode", 1), ("prefill", n_tok)):
        f = a.f32()
        g = synth.rng(MOE_CFG, f"bench-{mode}")
        for t in range(tokens):
            f[a.n + t * a.s_embd: a.n + t * a.s_embd + MOE_EMBD] = g.standard_normal(MOE_EMBD, dtype=np.float32)
            f[a.x + t * a.s_embd: a.x + t * a.s_embd + MOE_EMBD] = 0.0
        a.set_ctl(0, 0, tokens)
        a.buffer.upload()

        def body(r, batched=tokens > 1):
            for gq, uq, dq, ro in layers:
                E.Graph(r, k, a, c, batched).moe(gq, uq, dq, ro)
        rec = ctx.record(EAGER, body)
        ctx.replay(rec)
        a.buffer.download()
        ids = a.u32()[a.moe.ids: a.moe.ids + tokens * MOE_USED]
        distinct = len(set(int(i) for i in ids))
        for _ in range(3):
            ctx.replay(rec)
        ns = float(np.median([ctx.replay_timed(rec) for _ in range(7)]))
        per_layer = ns / n_layer
        moved = distinct * expert_bytes + router_bytes
        flops = 2.0 * tokens * MOE_USED * 3 * MOE_EMBD * MOE_FF
        out[mode] = {"tokens": tokens, "us_per_layer": round(per_layer / 1e3, 2), "distinct_experts": distinct,
                     "algorithmic_bytes_per_layer": moved, "gbs": round(moved / per_layer, 1),
                     "tflops": round(flops / per_layer / 1e3, 2), "launches_per_layer": rec.launches() / n_layer}
        rec.free()
    for b in weights:
        b.free()
    a.buffer.free()
    return out


def decode_config5(ctx: Context, contexts=(1024, 16384), steps: int = 20, warmup: int = 3) -> dict:
    """Config 5: the full Qwen3-8B Q4_K_M decode step (embedding gather, 36 layers of
    RMSNorm, q/k/v, QK-norm + RoPE + KV write, attention over the cache, o, gate/up, SiLU,
    down, then the output norm and the 151936-row Q6_K head), with the KV cache (f16 keys,
    8-bit values) pre-filled with N(0,1) rows to each context length.  tok/s is end to end
    as Engine::step runs it: control words up, one graph replay, the logits back and the
    greedy argmax on the host.  Also a 512-token prefill from position 0 (four 128-token
    chunks).  The 36 layers hold copies of one seeded layer (two for ffn_down's Q6_K / Q4_K
    halves), each its own HBM copy."""
    c = synth.qwen3_config("qwen3-8b")
    t = synth.qwen3("qwen3-8b-q4_k_m", c, "q4_k_m", "ones", shared_layers=True)
    max_ctx = max(contexts) + warmup + steps + 8
    eng = E.Engine(ctx, t, c, max_ctx, E.KvPrecision.F16_KEYS_Q8_VALUES, profile=EAGER, fuse=FUSE)
    try:
        a, kvl = eng.arena, eng.arena.kv_layout
        kv_dim = c.n_head_kv * c.head_dim
        synth.fill_kv(kvl, a.kv.host(), max(contexts), kv_dim, "qwen3-8b-q4_k_m", shared=True)
        a.kv.upload()
        mats = [v for k, v in t.items() if isinstance(v, tuple) and k != "token_embd.weight"]
        weight_bytes = sum(m[2] * E.row_bytes(m[0], m[1]) for m in mats) + E.row_bytes(E.DType.Q4K, c.n_embd)
        per_pos = c.n_layer * (kv_dim * 2 + kv_dim + kv_dim // 32 * 2)  # f16 K, i8 V, f16 V scales
        out = {"model": "Qwen3-8B Q4_K_M (36 layers, Q6_K head and even-layer ffn_down)",
               "kv": "f16 keys, 8-bit values", "weight_bytes_per_token": weight_bytes}
        for n_ctx in contexts:
            tok = 0
            eng.pos = n_ctx
            for _ in range(warmup):
                tok = int(np.argmax(eng.step(tok)))
            eng.pos = n_ctx
            t0 = time.perf_counter()
            for _ in range(steps):
                tok = int(np.argmax(eng.step(tok)))
            wall = (time.perf_counter() - t0) / steps
            eng.pos = n_ctx
            eng.load([tok], batched=False)
            dev = float(np.median([ctx.replay_timed(eng.decode) for _ in range(5)])) / 1e9
            nbytes = weight_bytes + n_ctx * per_pos
            out[f"ctx{n_ctx}"] = {"tok_s": round(1.0 / wall, 1), "ms_per_token": round(wall * 1e3, 3),
                                  "device_ms_per_token": round(dev * 1e3, 3),
                                  "launches_per_token": eng.decode.launches(),
                                  "kv_bytes_read": n_ctx * per_pos,
                                  "gbs_device": round(nbytes / dev / 1e9, 1)}
        # prefill: a 512-token prompt from position 0 as Engine::prefill runs it (four
        # 128-token chunks, each one graph replay of the batched recording)
        prompt = [int(v) for v in synth.rng("qwen3-8b-q4_k_m", "prompt").integers(0, c.n_vocab, 512)]
        eng.reset()
        eng.prefill(prompt)  # warm-up: every chunk's recording made
        times = []
        for _ in range(3):
            eng.reset()
            t0 = time.perf_counter()
            eng.prefill(prompt)
            times.append(time.perf_counter() - t0)
        pt = float(np.median(times))
        out["prefill512"] = {"tok_s": round(512 / pt, 1), "ms": round(pt * 1e3, 2), "chunks": 4}
        return out
    finally:
        eng.free()


def decode_config1(ctx: Context, steps: int = 64, warmup: int = 3) -> dict:
    """Config 1: Qwen3-0.6B with every matrix Q8_0 and the output head tied to token_embd
    (28 layers, 151936-row head), KV f16 keys and 8-bit values: the 16-token prompt through
    Engine::prefill, then greedy decode steps timed end to end as Engine::step runs them.
    The 28 layers hold copies of one seeded layer, each its own HBM copy."""
    c = synth.qwen3_config("qwen3-0.6b")
    t = synth.qwen3("qwen3-0.6b-q8_0", c, "q8_0", "ones", shared_layers=True)
    prompt = synth.prompt("qwen3-0.6b-q8_0", 16, c.n_vocab)
    eng = E.Engine(ctx, t, c, len(prompt) + warmup + steps + 8, E.KvPrecision.F16_KEYS_Q8_VALUES, profile=EAGER,
                   fuse=FUSE)
    try:
        mats = [v for v in t.values() if isinstance(v, tuple)]
        weight_bytes = sum(m[2] * E.row_bytes(m[0], m[1]) for m in mats)  # the head is token_embd
        tok = int(np.argmax(eng.prefill(prompt)))
        for _ in range(warmup):
            tok = int(np.argmax(eng.step(tok)))
        t0 = time.perf_counter()
        for _ in range(steps):
            tok = int(np.argmax(eng.step(tok)))
        wall = (time.perf_counter() - t0) / steps
        eng.load([tok], batched=False)
        dev = float(np.median([ctx.replay_timed(eng.decode) for _ in range(5)])) / 1e9
        # launches of the step recording at the last position, and of the one-split recording
        # the steps below 64 positions replay
        first = eng.recording(False, 1).launches()
        return {"model": "Qwen3-0.6B Q8_0 (28 layers, head tied to token_embd)", "kv": "f16 keys, 8-bit values",
                "prompt": len(prompt), "steps": steps, "weight_bytes_per_token": weight_bytes,
                "launches_per_token": eng.decode.launches(), "launches_per_token_below_64": first,
                "tok_s": round(1.0 / wall, 1),
                "ms_per_token": round(wall * 1e3, 3), "device_ms_per_token": round(dev * 1e3, 3),
                "gbs_device": round(weight_bytes / dev / 1e9, 1)}
    finally:
        eng.free()


def cpu_baseline(w: DecodeWorkload, budget_s: float = 15.0) -> dict:
    """skyla-ref Matrix::matvec restated in C (oracle/), timed on this host: layer passes of
    the same 7 matvecs until about budget_s seconds have elapsed."""
    from oracle import skyla_oracle as so

    threads = so.available_parallelism()
    xs = {n_in: synth.activations(CONFIG, f"cpu-x-{n_in}", n_in) for n_in in (N_EMBD, N_FF)}
    layer_bytes = sum(algo_bytes(dt, n_in, n_out, acc) for _, dt, n_in, n_out, acc in LAYER)
    passes, t0 = 0, time.perf_counter()
    while True:
        for name, dt, n_in, n_out, _ in LAYER:
            so.matvec(int(dt), w.data[name], n_in, n_out, xs[n_in], threads)
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    gbs = passes * layer_bytes / el / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{passes} passes over one Qwen3-8B layer's 7 decode matvecs "
                      f"({layer_bytes / 1e6:.1f} MB each), {el:.1f} s; oracle/skyla_oracle.c "
                      f"sk_matvec = skyla-ref Matrix::matvec (one thread per core, row dequant + "
                      f"sequential f32 dot), -O2",
            "tok_s_equiv": round(gbs * 1e9 / w.step_bytes, 3)}


def host_cpu() -> dict:
    """The host the CPU baselines ran on: model name (/proc/cpuinfo), logical CPUs, and the
    threads the oracle uses (available_parallelism, as skyla-ref's Matrix::matvec)."""
    from oracle import skyla_oracle as so

    model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count(), "threads_used": so.available_parallelism()}


def cpu_config1(budget_s: float = 20.0) -> dict:
    """Config 1 on the CPU: skyla-ref's Model::forward (oracle/model.py: Matrix::matvec per
    weight, f32 KV cache) over the Qwen3-0.6B Q8_0 model with 28 distinct seeded layers
    (633 MB of weights streamed per token), the 16-token prompt, then greedy decode steps
    until 64 or about budget_s seconds; tok/s over the decode steps."""
    from oracle import skyla_oracle as so
    from oracle.model import Model

    c = synth.qwen3_config("qwen3-0.6b")
    t = synth.qwen3("qwen3-0.6b-q8_0", c, "q8_0", "ones", shared_layers=False)
    prompt = synth.prompt("qwen3-0.6b-q8_0", 16, c.n_vocab)
    m = Model(c, t)
    t0 = time.perf_counter()
    for tok in prompt:
        logits = m.forward(tok)
    t_prompt = time.perf_counter() - t0
    tok, steps, t1 = so.argmax(logits), 0, time.perf_counter()
    while steps < 64 and time.perf_counter() - t1 < budget_s:
        tok = so.argmax(m.forward(tok))
        steps += 1
    el = time.perf_counter() - t1
    return {"value": round(steps / el, 2), "unit": "tok/s", "cores": so.available_parallelism(), "kind": "port",
            "sample": f"Qwen3-0.6B Q8_0 (28 distinct layers): 16-token prompt ({t_prompt:.1f} s, "
                      f"{16 / t_prompt:.2f} tok/s) then {steps} greedy decode steps ({el:.1f} s); oracle/model.py "
                      f"= skyla-ref Model::forward with Matrix::matvec (one thread per core), f32 KV",
            "prompt_tok_s": round(16 / t_prompt, 2)}


def cpu_config3(budget_s: float = 10.0, n_tok: int = 16) -> dict:
    """Config 3 on the CPU: skyla-ref's f32 GEMM (one Matrix::matvec per token row, the
    oracle's sk_matmul) over the q, gate and down matrices of config 3 on the first n_tok of
    the 512 f16-valued N(0,1) rows, repeated for about budget_s seconds; GFLOP/s, and the
    time M = 512 would take at that rate."""
    from oracle import skyla_oracle as so

    mats = [(name, dt, n_in, n_out, synth.matrix(CONFIG, name, dt, n_in, n_out))
            for name, dt, n_in, n_out in [("q", E.DType.Q4K, N_EMBD, N_EMBD), ("gate", E.DType.Q4K, N_EMBD, N_FF),
                                          ("down", E.DType.Q6K, N_FF, N_EMBD)]]
    xs = {n_in: synth.activations("qwen3-8b-prefill", f"x-512-{n_in}", (512, n_in))[:n_tok]
          .astype(np.float16).astype(np.float32) for n_in in (N_EMBD, N_FF)}
    flops_pass = sum(2.0 * n_tok * n_in * n_out for _, _, n_in, n_out, _ in mats)
    passes, t0 = 0, time.perf_counter()
    while True:
        for _, dt, n_in, n_out, d in mats:
            so.matmul(int(dt), d, n_in, n_out, xs[n_in])
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    gflops = passes * flops_pass / el / 1e9
    m512 = sum(2.0 * 512 * n_in * n_out for _, _, n_in, n_out, _ in mats) / (gflops * 1e9)
    return {"value": round(gflops, 2), "unit": "GFLOP/s", "cores": so.available_parallelism(), "kind": "port",
            "sample": f"{passes} passes of q, gate, down (Q4_K, Q4_K, Q6_K) over {n_tok} of the 512 token rows, "
                      f"{el:.1f} s; oracle sk_matmul = skyla-ref's M x Matrix::matvec",
            "m512_q_gate_down_s": round(m512, 2)}


def cpu_config4(budget_s: float = 10.0) -> dict:
    """Config 4 on the CPU: skyla-ref's Ffn::forward Moe arm (route, then the selected
    experts' swiglu, the oracle's sk_moe_forward) over the config-4 layer, one token at a
    time, for about budget_s seconds; us per token per layer and the GB/s of the experts
    and router it reads."""
    from oracle import skyla_oracle as so

    router = synth.router(MOE_CFG, "router", MOE_EXPERT, MOE_EMBD)
    d = {name: synth.matrix(MOE_CFG, f"{name}_exps", E.DType.Q4K, n_in, n_out, MOE_EXPERT)
         for name, n_in, n_out in [("gate", MOE_EMBD, MOE_FF), ("up", MOE_EMBD, MOE_FF), ("down", MOE_FF, MOE_EMBD)]}
    g = synth.rng(MOE_CFG, "cpu-tokens")
    q = int(E.DType.Q4K)
    tokens, t0 = 0, time.perf_counter()
    while True:
        n = g.standard_normal(MOE_EMBD, dtype=np.float32)
        so.moe_forward(router, q, d["gate"], q, d["up"], q, d["down"], MOE_EMBD, MOE_FF, MOE_EXPERT, MOE_USED, n)
        tokens += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    us = el / tokens * 1e6
    moved = MOE_USED * 3 * MOE_FF * E.row_bytes(E.DType.Q4K, MOE_EMBD) + MOE_EXPERT * MOE_EMBD * 4
    return {"value": round(us, 1), "unit": "us per token per layer", "cores": so.available_parallelism(),
            "kind": "port", "gbs": round(moved / us / 1e3, 2),
            "sample": f"{tokens} single-token MoE layer forwards (route + 8 experts' swiglu), {el:.1f} s; "
                      f"oracle sk_moe_forward = skyla-ref Ffn::forward Moe arm"}


def parity_check(w: DecodeWorkload) -> float:
    """rel-L2 of the GPU q matvec of layer 0 against the oracle (same inputs)."""
    from oracle import skyla_oracle as so

    ctx = w.ctx
    rec = ctx.record(EAGER, lambda r: E.Graph(r, w.k, None, None, False).matvec(
        w.layers[0]["q"], (w.off["n"], 0), (w.off["q"], 0), False, False))
    ctx.replay(rec)
    rec.free()
    w.arena.download()
    f = w.arena.as_f32()
    x = f[w.off["n"]: w.off["n"] + N_EMBD].copy()
    got = f[w.off["q"]: w.off["q"] + N_EMBD].astype(np.float64)
    want = so.matvec(int(E.DType.Q4K), w.data["q"], N_EMBD, N_EMBD, x).astype(np.float64)
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=N_LAYER)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-3 GEMM figures")
    ap.add_argument("--no-moe", action="store_true", help="skip the config-4 MoE figures")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-5 end-to-end decode figures")
    ap.add_argument("--e2e-only", type=str, default=None, metavar="CTX[,CTX]",
                    help="run only the config-5 end-to-end decode at these KV context lengths and print "
                         "its figures (for kernel traces of the whole decode step)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--eager", action="store_true",
                    help="replay recordings as direct launches instead of one HIP graph")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the config-3 prefill GEMMs (for hardware-counter runs)")
    ap.add_argument("--calibrate", action="store_true",
                    help="run only the two known-size kernels that scale rocprofv3 FETCH_SIZE/WRITE_SIZE")
    ap.add_argument("--no-config1", action="store_true",
                    help="with --e2e-only: skip the config-1 decode (kernel traces of config 5 alone)")
    ap.add_argument("--fuse", choices=["none", "qkv", "ffn", "all", "auto"], default="auto",
                    help="the decode graph's fusion level in the end-to-end runs")
    args = ap.parse_args()
    global EAGER, FUSE
    EAGER, FUSE = args.eager, args.fuse
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every box of this build has a single MI355X, and "
              f"the path shards across GPUs only by design (rows of the dense matrices, experts of the MoE); "
              f"got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    def log(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    ctx = Context.new(0)
    if args.calibrate:
        print(json.dumps(calibrate(ctx)))
        ctx.free()
        return 0
    if args.gemm_only:
        print(json.dumps({"prefill_gemm_m512": prefill_gemm(ctx)}))
        ctx.free()
        return 0
    if args.e2e_only:
        e2e = decode_config5(ctx, tuple(int(v) for v in args.e2e_only.split(",")))
        print(json.dumps({"decode_e2e_config5": e2e,
                          "decode_e2e_config1": None if args.no_config1 else decode_config1(ctx)}))
        ctx.free()
        return 0
    log(f"device {ctx.device_name()}; building {args.layers}-layer decode workload")
    w = DecodeWorkload(ctx, args.layers)
    log(f"{w.weight_bytes / 1e9:.2f} GB of weights in {len(w.weights)} buffers")
    step = w.record()
    wall, dev = time_replays(ctx, step, args.warmup, args.steps)
    ms_per_step = wall / args.steps * 1e3
    gbs = w.step_bytes / (wall / args.steps) / 1e9
    dev_ms = float(np.median(dev)) / 1e6
    log(f"step {ms_per_step:.3f} ms wall, {dev_ms:.3f} ms device; {gbs:.0f} GB/s")

    # dominant kernel: matvec_q4k (Q, K, V, O, gate, up); events around its launches only
    q4k_names = ("q", "k", "v", "o", "gate", "up")
    # (a launch may carry several fused dispatches: q/k/v and gate/up each run as one)
    rq = w.record(only=q4k_names)
    _, dq = time_replays(ctx, rq, 3, 5)
    n_launch = rq.launches()
    q4k_ns = float(np.median(dq)) / n_launch
    q4k_bytes = w.bytes_of(q4k_names) / n_launch
    rq.free()
    rd = w.record(only=("down",))
    _, dd = time_replays(ctx, rd, 3, 5)
    q6k_ns = float(np.median(dd)) / rd.launches()
    q6k_bytes = w.bytes_of(("down",)) / rd.launches()
    rd.free()
    achieved = q4k_bytes / q4k_ns  # GB/s
    log(f"matvec_q4k avg {q4k_ns / 1e3:.2f} us/launch, {achieved:.0f} GB/s; "
        f"matvec_q6k avg {q6k_ns / 1e3:.2f} us, {q6k_bytes / q6k_ns:.0f} GB/s")

    parity = parity_check(w)
    log(f"parity (q, layer 0) rel-L2 {parity:.2e}")
    probe, probe_form = hbm_probe(ctx)
    log(f"HBM stream-read probe {probe:.0f} GB/s ({probe_form})")
    prefill = None if args.no_prefill else prefill_gemm(ctx)
    if prefill:
        log(f"prefill GEMM M=512: {prefill}")
    moe = None if args.no_moe else moe_layers(ctx)
    if moe:
        log(f"MoE layer (config 4): {moe}")
    e2e = None if args.no_e2e else decode_config5(ctx)
    e2e1 = None if args.no_e2e else decode_config1(ctx)
    if e2e:
        log(f"end-to-end decode (config 5): {e2e}")
        log(f"end-to-end decode (config 1): {e2e1}")
    cpu = None if args.no_cpu else cpu_baseline(w, args.cpu_seconds)
    cpus = None
    if cpu:
        log(f"cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")
        cpus = {"host": host_cpu(), "config1_decode": cpu_config1(), "config3_gemm": cpu_config3(),
                "config4_moe": cpu_config4()}
        log(f"cpu baselines: {cpus}")

    # HBM bytes of the matvec_q4k launches of one layer, measured with rocprofv3 PMC
    # (FETCH_SIZE / WRITE_SIZE scaled by known-size kernels), spread over this run's launches
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "matvec_q4k_qwen3_8b_decode_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as fh:
            per_layer = json.load(fh).get("bytes_per_layer")
        if per_layer:
            traffic = round(per_layer * args.layers / n_launch)

    line = {
        "metric": "Q4_K matvec HBM GB/s (% of peak) + decode tok/s, Qwen3-8B shapes, 1 GPU",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32: exact integer quants x f32 activations, f32 accumulate (Q4_K/Q6_K blocks)",
        "data": "synthetic: seeded GGUF Q4_K/Q6_K blocks and N(0,1) f32 activations (config 2)",
        "config": {"workload": "config 2: Qwen3-8B decode matvecs x 36 layers (Q,K,V,O,gate,up Q4_K; "
                               "down Q6_K), one HBM copy of the weights per layer",
                   "layers": args.layers, "dispatches_per_step": len(step),
                   "launches_per_step": step.launches(),
                   "replay": "direct launches" if EAGER else "one HIP graph per step",
                   "weight_bytes": w.weight_bytes, "algorithmic_bytes_per_step": w.step_bytes},
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "decode_tok_s_matvec_only": round(1e3 / ms_per_step, 1),
        "device_ms_per_step": round(dev_ms, 4),
        "roofline": {"bound": "hbm", "kernel": "matvec_q4k", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes_per_launch": round(q4k_bytes),
                     "avg_launch_us": round(q4k_ns / 1e3, 3), "launches_per_layer": n_launch / args.layers},
        "matvec_q6k": {"avg_launch_us": round(q6k_ns / 1e3, 3), "gbs": round(q6k_bytes / q6k_ns, 1)},
        "hbm_probe_gbs": round(probe, 1),
        "hbm_probe_form": probe_form,
        "parity_rel_l2": parity,
        "prefill_gemm_m512": prefill,
        "moe_layer_config4": moe,
        "decode_e2e_config5": e2e,
        "decode_e2e_config1": e2e1,
        "cpu_baseline": cpu,
        "cpu_baselines": cpus,
    }
    step.free()
    w.free()
    ctx.free()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
