"""ctypes wrapper of oracle/libskyla_oracle.so (TEST INFRASTRUCTURE ONLY).

Each function restates the reference function named in its docstring; see skyla_oracle.c
for the file:line citations.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libskyla_oracle.so")

F32, F16, Q8_0, Q4K, Q6K = 0, 1, 8, 12, 14

_lib = None
_f = C.POINTER(C.c_float)
_u8 = C.POINTER(C.c_uint8)
_u32 = C.POINTER(C.c_uint32)


def build() -> str:
    r = subprocess.run(["make", "-s", "-B", "-C", HERE], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = C.CDLL(LIB_PATH)
        l.sk_f16_to_f32.restype = C.c_float
        l.sk_f16_to_f32.argtypes = [C.c_uint16]
        l.sk_f32_to_f16.restype = C.c_uint16
        l.sk_f32_to_f16.argtypes = [C.c_float]
        l.sk_row_bytes.restype = C.c_int64
        l.sk_row_bytes.argtypes = [C.c_uint32, C.c_uint64]
        l.sk_dequantize.restype = C.c_int
        l.sk_dequantize.argtypes = [C.c_uint32, _u8, C.c_uint64, _f, C.c_uint64]
        l.sk_q4k_scale_min.restype = None
        l.sk_q4k_scale_min.argtypes = [C.c_uint32, _u8, _u8, _u8]
        l.sk_quantize_q8_0.restype = None
        l.sk_quantize_q8_0.argtypes = [_f, C.c_uint64, _u8]
        l.sk_matvec.restype = C.c_int
        l.sk_matvec.argtypes = [C.c_uint32, _u8, C.c_uint64, C.c_uint64, _f, _f, C.c_uint32]
        l.sk_matmul.restype = C.c_int
        l.sk_matmul.argtypes = [C.c_uint32, _u8, C.c_uint64, C.c_uint64, C.c_uint64, _f, C.c_uint64,
                                _f, C.c_uint64, C.c_uint32]
        l.sk_rmsnorm.restype = None
        l.sk_rmsnorm.argtypes = [_f, _f, C.c_uint64, C.c_float, _f]
        l.sk_softmax.restype = None
        l.sk_softmax.argtypes = [_f, C.c_uint64]
        l.sk_silu.restype = C.c_float
        l.sk_silu.argtypes = [C.c_float]
        l.sk_dot.restype = C.c_float
        l.sk_dot.argtypes = [_f, _f, C.c_uint64]
        l.sk_argmax.restype = C.c_uint32
        l.sk_argmax.argtypes = [_f, C.c_uint64]
        l.sk_route.restype = C.c_int
        l.sk_route.argtypes = [_f, _f, C.c_uint64, C.c_uint64, C.c_uint64, _u32, _f]
        l.sk_swiglu.restype = C.c_int
        l.sk_swiglu.argtypes = [C.c_uint32, _u8, C.c_uint32, _u8, C.c_uint32, _u8, C.c_uint64, C.c_uint64,
                                _f, _f, C.c_uint32]
        l.sk_moe_forward.restype = C.c_int
        l.sk_moe_forward.argtypes = [_f, C.c_uint32, _u8, C.c_uint32, _u8, C.c_uint32, _u8, C.c_uint64,
                                     C.c_uint64, C.c_uint64, C.c_uint64, _f, _f, _u32, _f, C.c_uint32]
        l.sk_moe_sort.restype = C.c_int
        l.sk_moe_sort.argtypes = [_u32, C.c_uint64, C.c_uint32, _u32, _u32]
        l.sk_rmsnorm_inplace.restype = None
        l.sk_rmsnorm_inplace.argtypes = [_f, _f, C.c_uint64, C.c_float]
        l.sk_rope_freqs.restype = None
        l.sk_rope_freqs.argtypes = [C.c_uint64, C.c_float, _f]
        l.sk_rope_freqs_yarn.restype = C.c_float
        l.sk_rope_freqs_yarn.argtypes = [C.c_uint64, C.c_float, C.c_float, C.c_float, C.c_float, _f]
        l.sk_rope_neox.restype = None
        l.sk_rope_neox.argtypes = [_f, C.c_uint64, C.c_uint64, _f, C.c_float]
        l.sk_attention.restype = None
        l.sk_attention.argtypes = [_f, _f, _f, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, _f, _f]
        l.sk_available_parallelism.restype = C.c_uint32
        l.sk_available_parallelism.argtypes = []
        _lib = l
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _u8a(b) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(b), np.uint8) if isinstance(b, (bytes, bytearray)) else b,
                                dtype=np.uint8)


def _check(s: int, what: str) -> None:
    if s != 0:
        raise ValueError(f"{what}: oracle error {s}")


def f16_to_f32(h: int) -> float:
    """half 2.7.1 f16::to_f32."""
    return lib().sk_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().sk_f32_to_f16(f)


def row_bytes(dtype: int, n: int) -> int:
    """DType::row_bytes (skyla-gguf/src/lib.rs:45-53); negative on error."""
    return lib().sk_row_bytes(dtype, n)


def dequantize(dtype: int, src, n: int) -> np.ndarray:
    """skyla_gguf::dequantize (quant.rs:5-38) into n f32."""
    src = _u8a(src)
    out = np.zeros(n, np.float32)
    _check(lib().sk_dequantize(dtype, _p(src, _u8), src.size, _p(out, _f), n), "dequantize")
    return out


def q4k_scale_min(j: int, scales) -> tuple[int, int]:
    s = _u8a(scales)
    sc, m = C.c_uint8(), C.c_uint8()
    lib().sk_q4k_scale_min(j, _p(s, _u8), C.byref(sc), C.byref(m))
    return sc.value, m.value


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(-(-x.size // 32) * 34, np.uint8)
    lib().sk_quantize_q8_0(_p(x, _f), x.size, _p(out, _u8))
    return out


def matvec(dtype: int, data, n_in: int, n_out: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """Matrix::matvec (skyla-ref/src/matrix.rs:43-58)."""
    data = _u8a(data)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(n_out, np.float32)
    _check(lib().sk_matvec(dtype, _p(data, _u8), n_in, n_out, _p(x, _f), _p(y, _f), threads), "matvec")
    return y


def matmul(dtype: int, data, n_in: int, n_out: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """The oracle's f32 GEMM: one Matrix::matvec per token row of x[n_tok, n_in]."""
    data = _u8a(data)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros((x.shape[0], n_out), np.float32)
    _check(lib().sk_matmul(dtype, _p(data, _u8), n_in, n_out, x.shape[0], _p(x, _f), n_in, _p(y, _f), n_out,
                           threads), "matmul")
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    lib().sk_rmsnorm(_p(x, _f), _p(w, _f), x.size, eps, _p(out, _f))
    return out


def softmax(x):
    x = np.array(x, np.float32)
    lib().sk_softmax(_p(x, _f), x.size)
    return x


def silu(x: float) -> float:
    return lib().sk_silu(x)


def dot(a, b) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().sk_dot(_p(a, _f), _p(b, _f), a.size)


def argmax(x) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return lib().sk_argmax(_p(x, _f), x.size)


def route(router: np.ndarray, n: np.ndarray, used: int):
    """ffn::route (skyla-ref/src/ffn.rs:30-37): [(expert, weight)] in route order."""
    router = np.ascontiguousarray(router, np.float32)
    n = np.ascontiguousarray(n, np.float32)
    n_expert = router.size // n.size
    ids = np.zeros(used, np.uint32)
    w = np.zeros(used, np.float32)
    _check(lib().sk_route(_p(router, _f), _p(n, _f), n.size, n_expert, used, _p(ids, _u32), _p(w, _f)), "route")
    return ids, w


def swiglu(gate_t, gate, up_t, up, down_t, down, n_embd, n_ff, n, threads=0):
    gate, up, down = _u8a(gate), _u8a(up), _u8a(down)
    n = np.ascontiguousarray(n, np.float32)
    out = np.zeros(n_embd, np.float32)
    _check(lib().sk_swiglu(gate_t, _p(gate, _u8), up_t, _p(up, _u8), down_t, _p(down, _u8), n_embd, n_ff,
                           _p(n, _f), _p(out, _f), threads), "swiglu")
    return out


def moe_forward(router, gate_t, gate, up_t, up, down_t, down, n_embd, n_ff, n_expert, used, n, threads=0):
    """Ffn::forward, Moe arm (skyla-ref/src/ffn.rs:58-76): (out, ids, weights)."""
    router = np.ascontiguousarray(router, np.float32)
    gate, up, down = _u8a(gate), _u8a(up), _u8a(down)
    n = np.ascontiguousarray(n, np.float32)
    out = np.zeros(n_embd, np.float32)
    ids = np.zeros(used, np.uint32)
    w = np.zeros(used, np.float32)
    _check(lib().sk_moe_forward(_p(router, _f), gate_t, _p(gate, _u8), up_t, _p(up, _u8), down_t, _p(down, _u8),
                                n_embd, n_ff, n_expert, used, _p(n, _f), _p(out, _f), _p(ids, _u32), _p(w, _f),
                                threads), "moe_forward")
    return out, ids, w


def moe_sort(ids: np.ndarray, n_expert: int):
    """moe_sort.comp:21-55 semantics: (table[n_expert, 2], list[n_slots])."""
    ids = np.ascontiguousarray(ids, np.uint32)
    table = np.zeros(2 * n_expert, np.uint32)
    lst = np.zeros(ids.size, np.uint32)
    _check(lib().sk_moe_sort(_p(ids, _u32), ids.size, n_expert, _p(table, _u32), _p(lst, _u32)), "moe_sort")
    return table.reshape(n_expert, 2), lst


def rmsnorm_inplace(x: np.ndarray, w, eps) -> None:
    """ops.rs:8-16 rmsnorm_inplace (x *= r * w) on a contiguous float32 array."""
    assert x.dtype == np.float32 and x.flags.c_contiguous
    w = np.ascontiguousarray(w, np.float32)
    lib().sk_rmsnorm_inplace(_p(x, _f), _p(w, _f), x.size, eps)


def rope_freqs(head_dim: int, theta: float) -> np.ndarray:
    """rope.rs:36-40 frequencies (no scaling)."""
    out = np.zeros(head_dim // 2, np.float32)
    lib().sk_rope_freqs(head_dim, theta, _p(out, _f))
    return out


def rope_freqs_yarn(head_dim: int, theta: float, factor: float, original_ctx: float,
                    attn_factor: float) -> tuple[np.ndarray, float]:
    """rope.rs:36-58 frequencies with YaRN scaling, and the magnitude scale mscale."""
    out = np.zeros(head_dim // 2, np.float32)
    m = lib().sk_rope_freqs_yarn(head_dim, theta, factor, original_ctx, attn_factor, _p(out, _f))
    return out, float(m)


def rope_neox(x: np.ndarray, pos: int, freqs: np.ndarray, mscale: float = 1.0) -> None:
    """rope.rs:60-68 rope_neox in place on a contiguous float32 array."""
    assert x.dtype == np.float32 and x.flags.c_contiguous
    freqs = np.ascontiguousarray(freqs, np.float32)
    lib().sk_rope_neox(_p(x, _f), x.size, pos, _p(freqs, _f), mscale)


def attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, n_pos: int, n_head: int,
              n_head_kv: int, hd: int) -> np.ndarray:
    """model.rs:150-169: every head's softmax attention over n_pos cached positions."""
    q = np.ascontiguousarray(q, np.float32)
    k_cache = np.ascontiguousarray(k_cache, np.float32)
    v_cache = np.ascontiguousarray(v_cache, np.float32)
    scores = np.zeros(max(n_pos, 1), np.float32)
    out = np.zeros(n_head * hd, np.float32)
    lib().sk_attention(_p(q, _f), _p(k_cache, _f), _p(v_cache, _f), n_pos, n_head, n_head_kv, hd,
                       _p(scores, _f), _p(out, _f))
    return out


def kv_quantize_q8(y: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The GPU backend's q8 KV store (skyla-shaders/shaders/qkv_prep.comp:40-65): per 32
    consecutive values s = max|y| / 127 in f32, q = round(y / s) with the f32 quotient (ties to
    even; GLSL leaves the tie direction to the implementation), 0 where s = 0; the scale is
    stored as f16.  Returns (q int8, scales f16), one scale per 32 values."""
    y = np.ascontiguousarray(y, np.float32)
    blocks = y.reshape(-1, 32)
    s32 = (np.abs(blocks).max(1) / np.float32(127.0)).astype(np.float32)
    safe = np.where(s32 > 0, s32, np.float32(1.0)).astype(np.float32)
    q = np.where(s32[:, None] > 0, np.rint(blocks / safe[:, None]), 0).astype(np.int8)
    return q.reshape(y.shape), s32.astype(np.float16)


def kv_stored(y: np.ndarray, q8: bool) -> np.ndarray:
    """What the attention reads back for a cache row stored by qkv_prep.comp:48-65 (and
    read by attention.comp): f16(y), or q * f16 scale."""
    y = np.ascontiguousarray(y, np.float32)
    if not q8:
        return y.astype(np.float16).astype(np.float32)
    q, s = kv_quantize_q8(y)
    return (q.reshape(-1, 32).astype(np.float32) * s.astype(np.float32)[:, None]).reshape(y.shape)


def available_parallelism() -> int:
    return lib().sk_available_parallelism()
