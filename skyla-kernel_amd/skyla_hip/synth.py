"""Seeded synthetic GGUF blocks and activations for the benchmark configurations.

Every tensor is drawn from numpy's PCG64 generator seeded with the first 8 bytes of
SHA-256("<config>/<tensor name>"), so the GPU box regenerates bit-identical inputs.
f16 fields are drawn as f32 and rounded to f16 with round-to-nearest-even.

  Q4_K (256 values / 144 B): d, dmin ~ U[1e-3, 1e-2]; the 12 scale bytes and 128 quant
       bytes are uniform bytes, i.e. 6-bit scales/mins uniform in 0..63 and nibbles in 0..15.
  Q6_K (256 values / 210 B): ql, qh uniform bytes (6-bit quants uniform in 0..63), int8
       sub-scales ~ U{-64..64}, d ~ U[1e-3, 1e-2].
  Q8_0 (32 values / 34 B): d ~ U[1e-3, 4e-3], quants ~ U{-127..127}.
  activations: f32 N(0, 1).
"""
from __future__ import annotations

import hashlib

import numpy as np

from .engine import DType, row_bytes


def seed_of(config: str, name: str) -> int:
    return int.from_bytes(hashlib.sha256(f"{config}/{name}".encode()).digest()[:8], "little")


def rng(config: str, name: str) -> np.random.Generator:
    return np.random.default_rng(seed_of(config, name))


def _f16_bytes(g: np.random.Generator, n: int, lo: float, hi: float) -> np.ndarray:
    v = g.uniform(lo, hi, size=n).astype(np.float32).astype(np.float16)
    return v.view(np.uint8).reshape(n, 2)


def q4k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    b = g.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(g, n_blocks, 1e-3, 1e-2)
    b[:, 2:4] = _f16_bytes(g, n_blocks, 1e-3, 1e-2)
    return b


def q6k_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    b = g.integers(0, 256, size=(n_blocks, 210), dtype=np.uint8)
    b[:, 192:208] = g.integers(-64, 65, size=(n_blocks, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
    b[:, 208:210] = _f16_bytes(g, n_blocks, 1e-3, 1e-2)
    return b


def q8_0_blocks(g: np.random.Generator, n_blocks: int) -> np.ndarray:
    b = np.empty((n_blocks, 34), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(g, n_blocks, 1e-3, 4e-3)
    b[:, 2:34] = g.integers(-127, 128, size=(n_blocks, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    return b


def matrix(config: str, name: str, dtype: DType, n_in: int, n_out: int, n_expert: int = 1) -> np.ndarray:
    """Raw GGUF bytes of a [n_expert][n_out] x n_in matrix, flat uint8."""
    g = rng(config, name)
    n_blocks = n_expert * n_out * row_bytes(dtype, n_in) // {DType.Q4K: 144, DType.Q6K: 210, DType.Q8_0: 34}[dtype]
    maker = {DType.Q4K: q4k_blocks, DType.Q6K: q6k_blocks, DType.Q8_0: q8_0_blocks}[DType(dtype)]
    return maker(g, n_blocks).reshape(-1)


def activations(config: str, name: str, shape) -> np.ndarray:
    return rng(config, name).standard_normal(size=shape, dtype=np.float32)


def router(config: str, name: str, n_expert: int, n_embd: int) -> np.ndarray:
    return (rng(config, name).standard_normal(size=(n_expert, n_embd), dtype=np.float32) * np.float32(0.02))


# ---- whole models (BASELINE.json configs 1 and 5) ---------------------------------------
def qwen3_config(name: str):
    """Config 1: Qwen3-0.6B (hidden 1024, 28 layers, 16 / 8 heads of 128, FFN 3072, vocab
    151936, RoPE theta 1e6, eps 1e-6).  Config 5: Qwen3-8B (hidden 4096, 36 layers, 32 / 8
    heads, FFN 12288).  "tiny": the same layout at test size."""
    from .engine import Config
    if name == "qwen3-0.6b":
        return Config(n_embd=1024, n_ff=3072, n_head=16, n_head_kv=8, head_dim=128, n_vocab=151936, n_layer=28)
    if name == "qwen3-8b":
        return Config(n_embd=4096, n_ff=12288, n_head=32, n_head_kv=8, head_dim=128, n_vocab=151936, n_layer=36)
    if name == "tiny":
        return Config(n_embd=512, n_ff=1024, n_head=4, n_head_kv=2, head_dim=128, n_vocab=2048, n_layer=3)
    if name == "tiny-moe":  # qwen3moe at test size: 16 experts, top 4, expert FFN 256
        return Config(n_embd=512, n_ff=1024, n_head=4, n_head_kv=2, head_dim=128, n_vocab=2048, n_layer=2,
                      n_expert=16, n_expert_used=4, n_ff_expert=256)
    raise ValueError(f"unknown model {name}")


def qwen3(config: str, c, quant: str = "q8_0", norms: str = "ones", shared_layers: bool = False) -> dict:
    """Tensor map of a dense Qwen3 model with seeded random weights (the names of the GGUF
    tensors, model.rs:33-60, weights.rs:58-144): name -> f32 array for norms, or
    (dtype, n_in, n_out, raw GGUF blocks) for matrices.
      quant "q8_0": every matrix Q8_0 and the head tied to token_embd (config 1).
      quant "q4_k_m": token_embd and attention/gate/up Q4_K, ffn_down Q6_K in even layers and
        Q4_K in odd ones, output head Q6_K (config 5).
      quant "q4_k_m_mixed": as q4_k_m with attn_v also Q6_K in even layers, as llama.cpp's
        Q4_K_M mixes them (q, k and v then differ in type within a layer).
      norms "ones": f32 1.0 (config 1); "random": U[0.5, 1.5], which also exercises the
        norm weights.
    shared_layers: every layer's matrices are the seeded ones of layer 0 (ffn_down: of layer
      0 or 1, by its type), which the loader still lays out as a copy per layer; the bench
      uses it to build a 5 GB model in seconds with the same HBM traffic."""
    def norm(name, n):
        if norms == "ones":
            return np.ones(n, np.float32)
        return rng(config, name).uniform(0.5, 1.5, size=n).astype(np.float32)

    made = {}

    def mat(name, dt, n_in, n_out):
        if shared_layers and name.startswith("blk."):
            i = int(name.split(".")[1])
            name = name.replace(f"blk.{i}.", f"blk.{i % 2 if 'ffn_down' in name else 0}.", 1)
        if name not in made:
            made[name] = (DType(dt), n_in, n_out, matrix(config, name, dt, n_in, n_out))
        return made[name]

    q8 = quant == "q8_0"
    base = DType.Q8_0 if q8 else DType.Q4K
    hd = c.head_dim
    t = {"token_embd.weight": mat("token_embd.weight", base, c.n_embd, c.n_vocab),
         "output_norm.weight": norm("output_norm.weight", c.n_embd)}
    if not q8:
        t["output.weight"] = mat("output.weight", DType.Q6K, c.n_embd, c.n_vocab)
    for i in range(c.n_layer):
        n = lambda s: f"blk.{i}.{s}.weight"  # noqa: E731
        down = base if q8 or i % 2 else DType.Q6K
        v_type = DType.Q6K if quant == "q4_k_m_mixed" and i % 2 == 0 else base
        t.update({
            n("attn_norm"): norm(n("attn_norm"), c.n_embd),
            n("ffn_norm"): norm(n("ffn_norm"), c.n_embd),
            n("attn_q_norm"): norm(n("attn_q_norm"), hd),
            n("attn_k_norm"): norm(n("attn_k_norm"), hd),
            n("attn_q"): mat(n("attn_q"), base, c.n_embd, c.n_head * hd),
            n("attn_k"): mat(n("attn_k"), base, c.n_embd, c.n_head_kv * hd),
            n("attn_v"): mat(n("attn_v"), v_type, c.n_embd, c.n_head_kv * hd),
            n("attn_output"): mat(n("attn_output"), base, c.n_head * hd, c.n_embd),
            n("ffn_gate"): mat(n("ffn_gate"), base, c.n_embd, c.n_ff),
            n("ffn_up"): mat(n("ffn_up"), base, c.n_embd, c.n_ff),
            n("ffn_down"): mat(n("ffn_down"), down, c.n_ff, c.n_embd),
        })
    return t


def qwen3moe(config: str, c, norms: str = "random") -> dict:
    """Tensor map of a qwen3moe model (config 4's layer inside the dense attention layout of
    model.rs): attention and token_embd Q4_K, output head Q6_K, and per layer an f32 router
    ffn_gate_inp ~ N(0, 0.02) of [n_expert][n_embd] with expert tensors ffn_{gate,up,down}_exps
    in Q4_K, (dtype, n_in, n_out per expert, raw blocks of n_expert matrices, n_expert)
    (weights.rs:82-84, ffn.rs:48-54)."""
    def norm(name, n):
        if norms == "ones":
            return np.ones(n, np.float32)
        return rng(config, name).uniform(0.5, 1.5, size=n).astype(np.float32)

    def mat(name, dt, n_in, n_out, n_expert=1):
        entry = (DType(dt), n_in, n_out, matrix(config, name, dt, n_in, n_out, n_expert))
        return entry + (n_expert,) if n_expert > 1 else entry

    hd, e = c.head_dim, c.n_expert
    t = {"token_embd.weight": mat("token_embd.weight", DType.Q4K, c.n_embd, c.n_vocab),
         "output_norm.weight": norm("output_norm.weight", c.n_embd),
         "output.weight": mat("output.weight", DType.Q6K, c.n_embd, c.n_vocab)}
    for i in range(c.n_layer):
        n = lambda s: f"blk.{i}.{s}.weight"  # noqa: E731
        t.update({
            n("attn_norm"): norm(n("attn_norm"), c.n_embd),
            n("ffn_norm"): norm(n("ffn_norm"), c.n_embd),
            n("attn_q_norm"): norm(n("attn_q_norm"), hd),
            n("attn_k_norm"): norm(n("attn_k_norm"), hd),
            n("attn_q"): mat(n("attn_q"), DType.Q4K, c.n_embd, c.n_head * hd),
            n("attn_k"): mat(n("attn_k"), DType.Q4K, c.n_embd, c.n_head_kv * hd),
            n("attn_v"): mat(n("attn_v"), DType.Q4K, c.n_embd, c.n_head_kv * hd),
            n("attn_output"): mat(n("attn_output"), DType.Q4K, c.n_head * hd, c.n_embd),
            n("ffn_gate_inp"): router(config, n("ffn_gate_inp"), e, c.n_embd),
            n("ffn_gate_exps"): mat(n("ffn_gate_exps"), DType.Q4K, c.n_embd, c.n_ff_expert, e),
            n("ffn_up_exps"): mat(n("ffn_up_exps"), DType.Q4K, c.n_embd, c.n_ff_expert, e),
            n("ffn_down_exps"): mat(n("ffn_down_exps"), DType.Q4K, c.n_ff_expert, c.n_embd, e),
        })
    return t


def fill_kv(layout, kv_host: np.ndarray, n_pos: int, kv_dim: int, config: str, shared: bool = False) -> None:
    """Positions [0, n_pos) of every layer's cache, in the host mirror of the KV buffer,
    with seeded N(0,1) keys and values stored at the layout's precision (f16 rows, or 8-bit
    rows with one f16 scale max|y| / 127 per 32 values, as the KV write kernel stores them).
    Layer l's rows come from their own seed, so a layer that read another layer's slot
    would see other values; with `shared` one layer's rows are drawn and copied into every
    layer (cheaper, for timing runs)."""
    pr = layout.precision
    drawn = None
    for l in range(len(layout.slots)):
        if drawn is None or not shared:
            g = rng(config, "kv" if shared else f"kv-{l}")
            drawn = []
            for q8 in (pr.keys_q8, pr.values_q8):
                y = g.standard_normal(size=(n_pos * kv_dim // 32, 32), dtype=np.float32)
                if q8:
                    sc = (np.abs(y).max(1) / np.float32(127.0)).astype(np.float32)
                    drawn.append((np.rint(y / sc[:, None]).astype(np.int8).reshape(-1), sc.astype(np.float16)))
                else:
                    drawn.append((y.reshape(-1).astype(np.float16), None))
        for keys, (rows, scales) in zip((True, False), drawn):
            off = layout.keys(l) if keys else layout.values(l)
            if scales is not None:
                kv_host.view(np.int8)[off: off + rows.size] = rows
                so = layout.key_scales(l) if keys else layout.value_scales(l)
                kv_host.view("<f2")[so: so + scales.size] = scales
            else:
                kv_host.view("<f2")[off: off + rows.size] = rows


def prompt(config: str, n: int, n_vocab: int) -> list[int]:
    """Config 1's prompt: n token ids uniform in [0, n_vocab)."""
    return [int(v) for v in rng(config, "prompt").integers(0, n_vocab, size=n)]
