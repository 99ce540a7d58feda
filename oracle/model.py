"""skyla-ref Model (skyla-ref/src/model.rs:64-170) for the dense Qwen3 layout -- TEST
INFRASTRUCTURE ONLY.

The decode step of the reference's CPU model, composed from the C restatements in
skyla_oracle.c: Matrix::row / matvec, rmsnorm, rmsnorm_inplace, rope_neox, the attention of
model.rs:150-169 and the two arms of Ffn::forward (ffn.rs:58-76: swiglu, or route then the
weighted sum of the selected experts' swiglu for a qwen3moe layer), with the f32 KV cache
the reference keeps.  Element-wise additions are numpy float32 (one IEEE rounding each, as
Rust's).  RoPE with or without YaRN scaling; no output gate, no recurrent layers: the
attention layouts of the Qwen3 decode configurations.

`kv_store` selects the cache the attention reads: None keeps the reference CPU model's f32
rows (model.rs:140-148); a pair (keys_q8, values_q8) stores every key and value row as the
reference's GPU backend does (qkv_prep.comp:48-65): f16, or q8 blocks of 32 with an f16
scale, so the GPU engine is compared with the same rounding of its cache.
"""
from __future__ import annotations

import numpy as np

from . import skyla_oracle as so


class Model:
    def __init__(self, c, tensors: dict, kv_store: tuple[bool, bool] | None = None):
        self.c, self.t, self.kv_store = c, tensors, kv_store
        # Config::from_gguf's (rope_freqs, rope_mscale) (lib.rs:96-97, rope.rs:36-58)
        scaling = getattr(c, "rope_scaling", None)
        if scaling is None:
            self.freqs, self.mscale = so.rope_freqs(c.head_dim, c.rope_theta), 1.0
        else:
            self.freqs, self.mscale = so.rope_freqs_yarn(c.head_dim, c.rope_theta, *scaling)
        self.reset()

    def reset(self) -> None:
        """model.rs:89-98."""
        self.k_cache = [[] for _ in range(self.c.n_layer)]
        self.v_cache = [[] for _ in range(self.c.n_layer)]
        self.pos = 0

    def load_cache(self, keys, values) -> None:
        """A pre-filled context: positions [0, n) of each layer's cache hold the rows
        keys / values (as the attention reads them back), and the next forward runs at
        position n.  keys / values are [n, kv_dim] arrays for every layer, or one such
        array per layer."""
        per_layer = not isinstance(keys, np.ndarray)
        n = (keys[0] if per_layer else keys).shape[0]
        for l in range(self.c.n_layer):
            kl, vl = (keys[l], values[l]) if per_layer else (keys, values)
            assert kl.shape[0] == n and vl.shape[0] == n
            self.k_cache[l] = [np.ascontiguousarray(kl, np.float32).reshape(-1)]
            self.v_cache[l] = [np.ascontiguousarray(vl, np.float32).reshape(-1)]
        self.pos = n

    def _mv(self, name: str, x: np.ndarray) -> np.ndarray:
        dt, n_in, n_out, data = self.t[name][:4]
        return so.matvec(int(dt), data, n_in, n_out, x)

    def _attention(self, l: int, n: np.ndarray) -> np.ndarray:
        """model.rs:131-170."""
        c, hd = self.c, self.c.head_dim
        name = lambda s: f"blk.{l}.{s}.weight"  # noqa: E731
        q, k, v = self._mv(name("attn_q"), n), self._mv(name("attn_k"), n), self._mv(name("attn_v"), n)
        for x, heads, w in ((q, c.n_head, name("attn_q_norm")), (k, c.n_head_kv, name("attn_k_norm"))):
            for h in range(heads):
                part = x[h * hd:(h + 1) * hd]
                so.rmsnorm_inplace(part, self.t[w], c.eps)
                so.rope_neox(part, self.pos, self.freqs, self.mscale)
        if self.kv_store is not None:
            k, v = so.kv_stored(k, self.kv_store[0]), so.kv_stored(v, self.kv_store[1])
        self.k_cache[l].append(k)
        self.v_cache[l].append(v)
        attn = so.attention(q, np.concatenate(self.k_cache[l]), np.concatenate(self.v_cache[l]), self.pos + 1,
                            c.n_head, c.n_head_kv, hd)
        return self._mv(name("attn_output"), attn)

    def forward(self, token: int) -> np.ndarray:
        """model.rs:104-129: the logits after `token` at position self.pos."""
        c = self.c
        dt, n_in, _, data = self.t["token_embd.weight"][:4]
        rb = so.row_bytes(int(dt), n_in)
        x = so.dequantize(int(dt), np.asarray(data)[token * rb:(token + 1) * rb], n_in)
        for l in range(c.n_layer):
            name = lambda s: f"blk.{l}.{s}.weight"  # noqa: E731
            n = so.rmsnorm(x, self.t[name("attn_norm")], c.eps)
            x = x + self._attention(l, n)
            n = so.rmsnorm(x, self.t[name("ffn_norm")], c.eps)
            if c.n_expert:  # Ffn::Moe (ffn.rs:64-75)
                g, u, d = (self.t[name(s)] for s in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"))
                out, _, _ = so.moe_forward(self.t[name("ffn_gate_inp")], int(g[0]), g[3], int(u[0]), u[3],
                                           int(d[0]), d[3], c.n_embd, c.n_ff_expert, c.n_expert,
                                           c.n_expert_used, n)
                x = x + out
            else:           # Ffn::Dense
                g, u, d = (self.t[name(s)] for s in ("ffn_gate", "ffn_up", "ffn_down"))
                x = x + so.swiglu(int(g[0]), g[3], int(u[0]), u[3], int(d[0]), d[3], c.n_embd, c.n_ff, n)
        x = so.rmsnorm(x, self.t["output_norm.weight"], c.eps)
        out = self.t.get("output.weight", self.t["token_embd.weight"])
        self.pos += 1
        return so.matvec(int(out[0]), out[3], out[1], out[2], x)
