"""Writes tests/golden/k_blocks.json: GGUF Q4_K / Q6_K super-blocks (256 weights) built from
chosen per-weight values, with the values the reference's dequantizers must produce
(crates/tl_runtime/src/quantized.rs:268-415).

The blocks are packed by restating the packing steps of llama.cpp's published block
encoders (ggml-quants.c quantize_row_q4_K_ref / quantize_row_q6_K_ref, MIT), which are the
inverse of the decoders under test:

  Q4_K  bytes 0-1 d, 2-3 dmin (f16 LE), 4-15 the eight (scale, min) 6-bit pairs: for j < 4
        scales[j] = sc_j, scales[j + 4] = m_j; for j >= 4 scales[j + 4] = (sc_j & 15) |
        (m_j & 15) << 4, scales[j - 4] |= (sc_j >> 4) << 6, scales[j] |= (m_j >> 4) << 6;
        bytes 16-143: for each 64-weight group g, byte 32g + l = L[64g + l] | L[64g + 32 + l] << 4.
  Q6_K  for each 128-weight half h (ql += 64, qh += 32): ql[l] = L[l] & 15 | (L[l + 64] & 15) << 4,
        ql[l + 32] = L[l + 32] & 15 | (L[l + 96] & 15) << 4, qh[l] = L[l] >> 4 | (L[l + 32] >> 4) << 2
        | (L[l + 64] >> 4) << 4 | (L[l + 96] >> 4) << 6 (L indexed within the half), then the 16
        int8 scales (one per 16 weights) and f16 d.

Expected values are computed from the chosen values -- never by decoding the bytes:
  Q4_K  w = d * sc_j * q - dmin * m_j,  j = weight / 32
  Q6_K  w = d * sc_s * (L - 32),        s = weight / 16
in float64 IEEE arithmetic (asserted exact against rationals; signed zeros follow the IEEE
rules) and rounded once to float32, stored as bit patterns.  In f32 the
reference's products d * sc, dmin * m, (d * sc) * q are exact, so one rounding is what it
computes too.
"""
import json
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16(bits):
    return float(np.array([bits], dtype=np.uint16).view(np.float16)[0])


def exact_f32(values, values_exact):
    """float64 values (IEEE arithmetic, so signed zeros follow its rules) -> float32, after
    checking each against the exact rational value: one rounding, to float32, is left."""
    for f, v in zip(values, values_exact):
        assert Fraction(f) == v, "float64 not exact for this case"
    return np.array(values, dtype=np.float64).astype(np.float32)


def pack_q4_k(dbits, dminbits, sc, mn, L):
    assert len(sc) == 8 and len(mn) == 8 and len(L) == 256
    scales = [0] * 12
    for j in range(8):
        ls, lm = sc[j], mn[j]
        if j < 4:
            scales[j] = ls
            scales[j + 4] = lm
        else:
            scales[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            scales[j - 4] |= (ls >> 4) << 6
            scales[j] |= (lm >> 4) << 6
    qs = []
    for g in range(4):
        for l in range(32):
            qs.append(L[64 * g + l] | (L[64 * g + 32 + l] << 4))
    blk = bytes([dbits & 0xFF, dbits >> 8, dminbits & 0xFF, dminbits >> 8] + scales + qs)
    assert len(blk) == 144
    d, dmin = f16(dbits), f16(dminbits)
    vals = exact_f32([d * sc[w // 32] * L[w] - dmin * mn[w // 32] for w in range(256)],
                     [Fraction(d) * sc[w // 32] * L[w] - Fraction(dmin) * mn[w // 32] for w in range(256)])
    return blk, vals


def pack_q6_k(dbits, sc, L):
    assert len(sc) == 16 and len(L) == 256
    ql, qh = [0] * 128, [0] * 64
    for h in range(2):
        Lh = L[128 * h:128 * h + 128]
        for l in range(32):
            ql[64 * h + l] = (Lh[l] & 0xF) | ((Lh[l + 64] & 0xF) << 4)
            ql[64 * h + l + 32] = (Lh[l + 32] & 0xF) | ((Lh[l + 96] & 0xF) << 4)
            qh[32 * h + l] = (Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) | ((Lh[l + 96] >> 4) << 6)
    blk = bytes(ql + qh + [s & 0xFF for s in sc] + [dbits & 0xFF, dbits >> 8])
    assert len(blk) == 210
    d = f16(dbits)
    vals = exact_f32([d * float(sc[w // 16]) * float(L[w] - 32) for w in range(256)],
                     [Fraction(d) * sc[w // 16] * (L[w] - 32) for w in range(256)])
    return blk, vals


Q4K_SCALES = [  # (name, d bits, dmin bits)
    ("one_half", 0x3C00, 0x3800), ("typical", 0x1E66, 0x1C1F), ("zero_min", 0x3C00, 0x0000),
    ("neg_d", 0xBC00, 0x4000), ("signed_zeros", 0x8000, 0x8000), ("subnormal_d", 0x0001, 0x3C00),
    ("max_normal", 0x7BFF, 0x7BFF), ("min_normal", 0x0400, 0x03FF),
]
Q6K_SCALES = [("one", 0x3C00), ("typical", 0x1E66), ("neg_half", 0xB800), ("neg_zero", 0x8000),
              ("min_subnormal", 0x0001), ("max_normal", 0x7BFF)]


def main():
    rng = np.random.default_rng(20261202)
    cases = []
    sc_sets = [("distinct_high_bits", [1, 17, 33, 63, 5, 21, 47, 62], [0, 63, 31, 16, 48, 2, 60, 33]),
               ("max", [63] * 8, [63] * 8),
               ("rand", [int(v) for v in rng.integers(0, 64, 8)], [int(v) for v in rng.integers(0, 64, 8)])]
    q_sets = [("ramp", [w % 16 for w in range(256)]), ("rev", [15 - (w * 7) % 16 for w in range(256)]),
              ("rand", [int(v) for v in rng.integers(0, 16, 256)])]
    for name, db, dmb in Q4K_SCALES:
        for scn, sc, mn in sc_sets:
            for qn, L in q_sets:
                blk, vals = pack_q4_k(db, dmb, sc, mn, L)
                cases.append({"type": "Q4_K", "name": f"{name}/{scn}/{qn}", "hex": blk.hex(),
                              "f32_bits": [int(b) for b in vals.view(np.uint32)]})
    s6_sets = [("extremes", [-128, 127, -1, 0, 1, 64, -64, 100, -100, 2, -2, 31, -31, 127, -128, 7]),
               ("rand", [int(v) for v in rng.integers(-128, 128, 16)])]
    l6_sets = [("ramp", [w % 64 for w in range(256)]), ("stride", [(w * 37) % 64 for w in range(256)]),
               ("rand", [int(v) for v in rng.integers(0, 64, 256)])]
    for name, db in Q6K_SCALES:
        for scn, sc in s6_sets:
            for qn, L in l6_sets:
                blk, vals = pack_q6_k(db, sc, L)
                cases.append({"type": "Q6_K", "name": f"{name}/{scn}/{qn}", "hex": blk.hex(),
                              "f32_bits": [int(b) for b in vals.view(np.uint32)]})
    with open(os.path.join(HERE, "k_blocks.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_k_blocks.py", "cases": cases}, f)


if __name__ == "__main__":
    main()
