"""Writes tests/golden/dequant_known_answers.json: GGUF blocks built from their format
definition and the values that definition fixes, computed here in numpy float32 in the
reference's operation order ((d*sc)*q - dmin*m for Q4_K, (d*sc)*q for Q6_K, d*q for Q8_0;
skyla-gguf/src/quant.rs:17-89).  No oracle code is used.

    python tests/golden/make_golden.py
"""
import json
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dequant_known_answers.json")
f32 = np.float32


def f16le(v):
    return np.float16(v).tobytes()


def f16v(v):
    return f32(np.float16(v))


def pack_q4k_scales(sc, m):
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


def q4k(d, dmin, sc, m, lo, hi):
    qs = bytearray(128)
    vals = np.empty(256, f32)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = lo(c, l) | (hi(c, l) << 4)
            vals[64 * c + l] = (f16v(d) * f32(sc[2 * c])) * f32(lo(c, l)) - f16v(dmin) * f32(m[2 * c])
            vals[64 * c + 32 + l] = (f16v(d) * f32(sc[2 * c + 1])) * f32(hi(c, l)) - f16v(dmin) * f32(m[2 * c + 1])
    return f16le(d) + f16le(dmin) + pack_q4k_scales(sc, m) + bytes(qs), vals


def q6k(q, sc, d):
    ql, qh = [0] * 128, [0] * 64
    vals = np.empty(256, f32)
    for half in range(2):
        for l in range(32):
            v = [q[128 * half + 32 * g + l] for g in range(4)]
            ql[64 * half + l] = (v[0] & 0xF) | ((v[2] & 0xF) << 4)
            ql[64 * half + 32 + l] = (v[1] & 0xF) | ((v[3] & 0xF) << 4)
            qh[32 * half + l] = (v[0] >> 4) | ((v[1] >> 4) << 2) | ((v[2] >> 4) << 4) | ((v[3] >> 4) << 6)
            for g in range(4):
                s = sc[8 * half + l // 16 + 2 * g]
                vals[128 * half + 32 * g + l] = (f16v(d) * f32(s)) * f32(v[g] - 32)
    blk = bytes(ql) + bytes(qh) + np.array(sc, np.int8).tobytes() + f16le(d)
    return blk, vals


def q8_0(q, d):
    blk, vals = b"", []
    for i in range(0, len(q), 32):
        blk += f16le(d) + np.array(q[i: i + 32], np.int8).tobytes()
        vals += [f16v(d) * f32(v) for v in q[i: i + 32]]
    return blk, np.array(vals, f32)


def main():
    cases = []

    def add(name, t, blk, vals):
        cases.append({"name": name, "ggml_type": t, "block_hex": blk.hex(),
                      "expected_f32_hex": np.asarray(vals, "<f4").tobytes().hex()})

    add("q4k_closed_form", 12, *q4k(1.0, 0.5, [j + 1 for j in range(8)], list(range(8)),
                                    lambda c, l: l % 16, lambda c, l: (7 * l + c) % 16))
    add("q4k_high_scale_bits", 12, *q4k(0.25, 2.0, [63, 62, 33, 16, 63, 48, 17, 32], [0, 63, 15, 16, 47, 63, 31, 1],
                                        lambda c, l: 15, lambda c, l: 15))
    add("q4k_inexact_scales", 12, *q4k(0.0013, 0.0071, [63, 1, 45, 7, 60, 33, 12, 50], [63, 5, 0, 29, 44, 3, 61, 18],
                                       lambda c, l: (3 * l + c) % 16, lambda c, l: (5 * l + 2 * c) % 16))
    sc6 = [-64, -1, 1, 64, -7, 9, 127, -128, 3, -3, 5, -5, 64, -64, 0, 2]
    add("q6k_all_zero_quants", 14, *q6k([0] * 256, sc6, 0.5))
    add("q6k_all_max_quants", 14, *q6k([63] * 256, sc6, 0.5))
    add("q6k_bit_layout", 14, *q6k([(i * 37) % 64 for i in range(256)], [1] * 16, 1.0))
    add("q6k_inexact", 14, *q6k([(i * 11 + 5) % 64 for i in range(256)], [(k * 29) % 129 - 64 for k in range(16)], 0.0037))
    add("q8_0_all_quants", 8, *q8_0(list(range(-128, 128)), 0.5))
    add("q8_0_inexact", 8, *q8_0([(i * 13) % 255 - 127 for i in range(64)], 0.00317))
    with open(OUT, "w") as fh:
        json.dump(cases, fh, indent=1)
    print(f"wrote {len(cases)} cases to {OUT}")


if __name__ == "__main__":
    main()
