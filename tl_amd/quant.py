"""Host-side GGUF Q4_0 / Q8_0 block encoders (numpy).

The reference only dequantizes (crates/tl_runtime/src/quantized.rs:182-260); quantized
files come from llama.cpp.  These encoders restate llama.cpp's published reference
quantizers (ggml-quants.c quantize_row_q4_0_ref / quantize_row_q8_0_ref, MIT) so that
synthetic weights are the blocks a GGUF file would hold:

  Q4_0: per 32 values, m = the value of largest magnitude (first one on ties),
        d = m / -8, id = 1/d (0 if d == 0), q = min(15, trunc(v * id + 8.5)),
        byte j = q[j] | q[j + 16] << 4, block = f16(d) LE + 16 bytes.
  Q8_0: amax = max |v|, d = amax / 127, id = 1/d (0 if d == 0),
        q = roundf(v * id) (half away from zero), block = f16(d) LE + 32 int8.
"""
import numpy as np

QK = 32


def quantize_q4_0(x):
    b = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, QK)
    idx = np.argmax(np.abs(b), axis=1)
    mx = b[np.arange(b.shape[0]), idx]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (b * inv[:, None]).astype(np.float32) + np.float32(8.5)
    q = np.minimum(15, np.trunc(v).astype(np.int32)).astype(np.uint8)
    qs = (q[:, :16] | (q[:, 16:] << 4)).astype(np.uint8)
    out = np.empty((b.shape[0], 18), dtype=np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = qs
    return out.reshape(-1)


def quantize_q8_0(x):
    b = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, QK)
    amax = np.max(np.abs(b), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (b * inv[:, None]).astype(np.float32).astype(np.float64)
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    out = np.empty((b.shape[0], 34), dtype=np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def random_q4_0_blocks(rng, n, k, d_lo=0.001, d_hi=0.02):
    """Q4_0 blocks with d ~ U(d_lo, d_hi) rounded to f16 and q ~ U{0..15} (matvec config)."""
    nb = n * k // QK
    out = np.empty((nb, 18), dtype=np.uint8)
    d = rng.uniform(d_lo, d_hi, nb).astype(np.float16)
    out[:, :2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return out.reshape(-1)


def random_q8_0_blocks(rng, n, k, d_lo=0.001, d_hi=0.02):
    """Q8_0 blocks with d ~ U(d_lo, d_hi) rounded to f16 and q ~ U{-127..127}."""
    nb = n * k // QK
    out = np.empty((nb, 34), dtype=np.uint8)
    d = rng.uniform(d_lo, d_hi, nb).astype(np.float16)
    out[:, :2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    return out.reshape(-1)
