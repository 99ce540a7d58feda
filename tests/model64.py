"""An independent float64 restatement of skyla-ref's Model::forward (TEST INFRASTRUCTURE):
the check that pins oracle/model.py's composition of the C oracle functions.

Written from the reference's equations, not from oracle/model.py: weights come from the
numpy dequantisation (oracle/quant_np.py, itself bit-exact against the C oracle), and
every step is float64 numpy:
  x = token_embd row                                          (model.rs:97-100)
  per layer: n = rmsnorm(x) * attn_norm; x += attention(n)     (model.rs:104-112, ops.rs:1-16)
             n = rmsnorm(x) * ffn_norm;  x += ffn(n)           (model.rs:113-114)
  attention: q, k, v = Wq n, Wk n, Wv n; per head rmsnorm * q_norm / k_norm, then NeoX
             RoPE of the (i, i + head_dim/2) pairs by pos * theta^(-2i/head_dim) (under
             YaRN the frequencies of yarn64, every pair scaled by its magnitude); the KV
             cache keeps k, v; head h reads kv head h / (n_head / n_head_kv); softmax of
             q.k / sqrt(head_dim) over the positions so far; Wo of the heads' sums
                                                               (model.rs:131-170, rope.rs:36-67)
  ffn: dense down(silu(gate n) * up n); MoE: router logits R n, the n_used largest (ties to
       the lower index), softmax over them, sum of w_e * expert e's dense ffn
                                                               (ffn.rs:21-37, 58-76)
  logits = W_out (rmsnorm(x) * output_norm), W_out = output.weight, else token_embd
                                                               (model.rs:71-74, 116-121)
"""
from __future__ import annotations

import numpy as np

from oracle import quant_np


def _deq(entry) -> np.ndarray:
    """(dtype, n_in, n_out, blocks[, n_expert]) -> float64 [n_expert,] n_out x n_in."""
    dt, n_in, n_out, data = entry[:4]
    w = quant_np.dequantize(int(dt), data).astype(np.float64)
    return w.reshape(-1, n_out, n_in) if len(entry) > 4 else w.reshape(n_out, n_in)


def _rms(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    return x / np.sqrt(np.mean(x * x) + eps) * w.astype(np.float64)


def _silu(x: np.ndarray) -> np.ndarray:
    return x * 0.5 * (1.0 + np.tanh(0.5 * x))   # x / (1 + e^-x), without overflow


def yarn64(head_dim: int, theta: float, factor: float, original_ctx: float, attn_factor: float):
    """YaRN's RoPE frequencies and magnitude in float64, from the method (Peng et al., "YaRN:
    Efficient Context Window Extension of Large Language Models", 2023): pair i keeps its
    frequency theta^(-2i/d) where it turns more than beta_fast = 32 times over the original
    context, is interpolated by 1/factor where it turns less than beta_slow = 1 time, and
    ramps linearly between the two (whole) dimensions; every rotated pair is scaled by
    attn_factor (1 + 0.1 ln factor)  (rope.rs:4-58)."""
    d = float(head_dim)
    base = theta ** (-2.0 * np.arange(head_dim // 2) / d)

    def dim_of(turns):  # the i at which the wavelength 2 pi / base_i spans original_ctx / turns
        return d * np.log(original_ctx / (turns * 2.0 * np.pi)) / (2.0 * np.log(theta))

    low, high = max(np.floor(dim_of(32.0)), 0.0), min(np.ceil(dim_of(1.0)), d - 1.0)
    keep = 1.0 - np.clip((np.arange(head_dim // 2) - low) / max(high - low, 0.001), 0.0, 1.0)
    return base * (keep + (1.0 - keep) / factor), attn_factor * (1.0 + 0.1 * np.log(factor))


class Model64:
    def __init__(self, c, tensors: dict):
        self.c = c
        self.w = {k: (_deq(v) if isinstance(v, tuple) else np.asarray(v, np.float64)) for k, v in tensors.items()}
        self.head = self.w.get("output.weight", self.w["token_embd.weight"])
        hd = c.head_dim
        self.freqs = c.rope_theta ** (-2.0 * np.arange(hd // 2) / hd)
        self.mscale = 1.0
        if getattr(c, "rope_scaling", None) is not None:
            self.freqs, self.mscale = yarn64(hd, c.rope_theta, *c.rope_scaling)
        self.k_cache = [[] for _ in range(c.n_layer)]
        self.v_cache = [[] for _ in range(c.n_layer)]
        self.pos = 0
        self.route_margin = np.inf   # smallest gap between the n_used-th and next router logit

    def _rope(self, h: np.ndarray) -> np.ndarray:
        half = h.size // 2
        ang = self.pos * self.freqs[:half]
        a, b = h[:half], h[half:]
        cs, sn = self.mscale * np.cos(ang), self.mscale * np.sin(ang)
        return np.concatenate([a * cs - b * sn, a * sn + b * cs])

    def _attention(self, l: int, n: np.ndarray) -> np.ndarray:
        c, hd, w = self.c, self.c.head_dim, self.w
        p = lambda s: w[f"blk.{l}.{s}.weight"]  # noqa: E731
        q = (p("attn_q") @ n).reshape(c.n_head, hd)
        k = (p("attn_k") @ n).reshape(c.n_head_kv, hd)
        v = (p("attn_v") @ n).reshape(c.n_head_kv, hd)
        q = np.stack([self._rope(_rms(h, p("attn_q_norm"), c.eps)) for h in q])
        k = np.stack([self._rope(_rms(h, p("attn_k_norm"), c.eps)) for h in k])
        self.k_cache[l].append(k)
        self.v_cache[l].append(v)
        keys, vals = np.stack(self.k_cache[l]), np.stack(self.v_cache[l])   # [pos, kv head, hd]
        rep = c.n_head // c.n_head_kv
        out = np.empty((c.n_head, hd))
        for h in range(c.n_head):
            s = keys[:, h // rep] @ q[h] / np.sqrt(hd)
            e = np.exp(s - s.max())
            out[h] = (e / e.sum()) @ vals[:, h // rep]
        return p("attn_output") @ out.reshape(-1)

    def _ffn(self, l: int, n: np.ndarray) -> np.ndarray:
        c, w = self.c, self.w
        p = lambda s: w[f"blk.{l}.{s}.weight"]  # noqa: E731
        if not c.n_expert:
            return p("ffn_down") @ (_silu(p("ffn_gate") @ n) * (p("ffn_up") @ n))
        logits = p("ffn_gate_inp") @ n
        order = np.argsort(-logits, kind="stable")
        top = order[:c.n_expert_used]
        self.route_margin = min(self.route_margin, float(logits[order[c.n_expert_used - 1]] - logits[order[c.n_expert_used]]))
        e = np.exp(logits[top] - logits[top].max())
        out = np.zeros(c.n_embd)
        for x, wt in zip(top, e / e.sum()):
            out += wt * (p("ffn_down_exps")[x] @ (_silu(p("ffn_gate_exps")[x] @ n) * (p("ffn_up_exps")[x] @ n)))
        return out

    def forward(self, token: int) -> np.ndarray:
        c, w = self.c, self.w
        x = w["token_embd.weight"][token].copy()
        for l in range(c.n_layer):
            x = x + self._attention(l, _rms(x, w[f"blk.{l}.attn_norm.weight"], c.eps))
            x = x + self._ffn(l, _rms(x, w[f"blk.{l}.ffn_norm.weight"], c.eps))
        self.pos += 1
        return self.head @ _rms(x, w["output_norm.weight"], c.eps)
