"""Writes tests/golden/q_blocks.json: hand-built GGUF Q4_0 / Q8_0 blocks with the values
the reference's dequantizers must produce (crates/tl_runtime/src/quantized.rs:182-260).

Expected values come from the closed form alone -- IEEE binary16 decode via numpy's float16
and the exact f32 product d * (q - 8) (Q4_0, low nibble of byte j -> element j, high nibble
-> element j + 16) or d * q (Q8_0) -- computed in float64 and rounded once to float32
(exact: an 11-bit by <= 8-bit significand product).  Values are stored as float32 bit
patterns so signed zeros are pinned too.
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

SCALES = [
    ("one", 0x3C00), ("neg_half", 0xB800), ("pos_zero", 0x0000), ("neg_zero", 0x8000),
    ("min_subnormal", 0x0001), ("max_subnormal", 0x03FF), ("min_normal", 0x0400),
    ("max_normal", 0x7BFF), ("neg_max_normal", 0xFBFF), ("typical", 0x1E66),
]


def f16(bits):
    return float(np.array([bits], dtype=np.uint16).view(np.float16)[0])


def q4_block(dbits, nib):
    qs = bytes((nib[j] & 15) | ((nib[j + 16] & 15) << 4) for j in range(16))
    blk = bytes([dbits & 0xFF, dbits >> 8]) + qs
    d = f16(dbits)
    vals = np.array([d * (q - 8) for q in nib], dtype=np.float64).astype(np.float32)
    return blk, vals


def q8_block(dbits, q):
    blk = bytes([dbits & 0xFF, dbits >> 8]) + bytes(np.array(q, dtype=np.int8).view(np.uint8))
    d = f16(dbits)
    vals = np.array([d * v for v in q], dtype=np.float64).astype(np.float32)
    return blk, vals


def main():
    rng = np.random.default_rng(20261201)
    cases = []
    ramp16 = list(range(16)) + list(range(15, -1, -1))
    for name, dbits in SCALES:
        for pat_name, nib in (("ramp", ramp16), ("all8", [8] * 32), ("rand", list(rng.integers(0, 16, 32)))):
            blk, vals = q4_block(dbits, [int(v) for v in nib])
            cases.append({"type": "Q4_0", "name": f"{name}/{pat_name}", "hex": blk.hex(),
                          "f32_bits": [int(b) for b in vals.view(np.uint32)]})
    ramp8 = list(range(-128, 128, 8))
    for name, dbits in SCALES:
        for pat_name, q in (("ramp", ramp8), ("extremes", [-128, 127, -127, 0, 1, -1] * 5 + [0, 0]),
                            ("rand", list(rng.integers(-127, 128, 32)))):
            blk, vals = q8_block(dbits, [int(v) for v in q])
            cases.append({"type": "Q8_0", "name": f"{name}/{pat_name}", "hex": blk.hex(),
                          "f32_bits": [int(b) for b in vals.view(np.uint32)]})
    with open(os.path.join(HERE, "q_blocks.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_q_blocks.py", "cases": cases}, f, indent=0)


if __name__ == "__main__":
    main()
