"""Host-side GGUF block encoders (numpy): Q4_0, Q8_0, Q4_K, Q6_K.

The reference only dequantizes (crates/tl_runtime/src/quantized.rs:182-415); quantized
files come from llama.cpp.  The Q4_0 / Q8_0 encoders restate llama.cpp's published reference
quantizers (ggml-quants.c quantize_row_q4_0_ref / quantize_row_q8_0_ref, MIT) so that
synthetic weights are the blocks a GGUF file would hold:

  Q4_0: per 32 values, m = the value of largest magnitude (first one on ties),
        d = m / -8, id = 1/d (0 if d == 0), q = min(15, trunc(v * id + 8.5)),
        byte j = q[j] | q[j + 16] << 4, block = f16(d) LE + 16 bytes.
  Q8_0: amax = max |v|, d = amax / 127, id = 1/d (0 if d == 0),
        q = roundf(v * id) (half away from zero), block = f16(d) LE + 32 int8.

The K-quant encoders use llama.cpp's block packing (quantize_row_q4_K_ref /
quantize_row_q6_K_ref) with a plain min/max choice of the scales instead of llama.cpp's
iterative search (synthetic weights only need valid blocks of the right statistics):

  Q4_K: per 32 values scale s = (max - min') / 15, min' = min(min, 0); d = max(s) / 63,
        dmin = max(-min') / 63 (f16); sc = round(s / d), m = round(-min' / dmin) (6 bits);
        q = clamp(round((v + dmin m) / (d sc)), 0, 15).
  Q6_K: per 16 values s = max|v| / 31 signed toward the extreme; d = max|s| / 127 (f16);
        sc = round(s / d) (int8); q = clamp(round(v / (d sc)), -32, 31) + 32.
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


QK_K = 256


def pack_q4_k(d, dmin, sc, mn, q):
    """Q4_K blocks from f16 d, dmin [nb], 6-bit sc, mn [nb, 8] and q [nb, 256] (0..15)."""
    nb = q.shape[0]
    out = np.zeros((nb, 144), dtype=np.uint8)
    out[:, 0:2] = np.asarray(d, np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = np.asarray(dmin, np.float16).view(np.uint8).reshape(-1, 2)
    sc = np.asarray(sc, np.uint8)
    mn = np.asarray(mn, np.uint8)
    scales = np.zeros((nb, 12), dtype=np.uint8)
    scales[:, 0:4] = sc[:, 0:4]
    scales[:, 4:8] = mn[:, 0:4]
    scales[:, 8:12] = (sc[:, 4:8] & 0xF) | ((mn[:, 4:8] & 0xF) << 4)
    scales[:, 0:4] |= (sc[:, 4:8] >> 4) << 6
    scales[:, 4:8] |= (mn[:, 4:8] >> 4) << 6
    out[:, 4:16] = scales
    q = np.asarray(q, np.uint8).reshape(nb, 4, 2, 32)  # group g, half (low / high nibble), l
    out[:, 16:] = (q[:, :, 0, :] | (q[:, :, 1, :] << 4)).reshape(nb, 128)
    return out.reshape(-1)


def pack_q6_k(d, sc, q):
    """Q6_K blocks from f16 d [nb], int8 sc [nb, 16] and q [nb, 256] (0..63)."""
    nb = q.shape[0]
    out = np.zeros((nb, 210), dtype=np.uint8)
    q = np.asarray(q, np.uint8).reshape(nb, 2, 4, 32)  # half h, quarter a, l
    lo, hi = q & 0xF, q >> 4
    ql = np.zeros((nb, 2, 64), dtype=np.uint8)
    ql[:, :, 0:32] = lo[:, :, 0, :] | (lo[:, :, 2, :] << 4)
    ql[:, :, 32:64] = lo[:, :, 1, :] | (lo[:, :, 3, :] << 4)
    qh = hi[:, :, 0, :] | (hi[:, :, 1, :] << 2) | (hi[:, :, 2, :] << 4) | (hi[:, :, 3, :] << 6)
    out[:, 0:128] = ql.reshape(nb, 128)
    out[:, 128:192] = qh.reshape(nb, 64)
    out[:, 192:208] = np.asarray(sc, np.int8).view(np.uint8)
    out[:, 208:210] = np.asarray(d, np.float16).view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


def quantize_q4_k(x):
    b = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 8, 32).astype(np.float64)
    mx = b.max(axis=2)
    mnv = np.minimum(b.min(axis=2), 0.0)
    s = (mx - mnv) / 15.0
    d = (s.max(axis=1) / 63.0).astype(np.float16)
    dmin = ((-mnv).max(axis=1) / 63.0).astype(np.float16)
    df, dmf = d.astype(np.float64)[:, None], dmin.astype(np.float64)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.clip(np.where(df > 0, np.rint(s / df), 0), 0, 63)
        mn = np.clip(np.where(dmf > 0, np.rint(-mnv / dmf), 0), 0, 63)
        step = (df * sc)[:, :, None]
        q = np.where(step > 0, np.rint((b + (dmf * mn)[:, :, None]) / step), 0)
    q = np.clip(q, 0, 15).reshape(-1, 256)
    return pack_q4_k(d, dmin, sc.astype(np.uint8), mn.astype(np.uint8), q.astype(np.uint8))


def quantize_q6_k(x):
    b = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 16, 16).astype(np.float64)
    idx = np.argmax(np.abs(b), axis=2)
    ext = np.take_along_axis(b, idx[:, :, None], axis=2)[:, :, 0]
    s = ext / -32.0  # the extreme maps to -32 (the wider side of the 6-bit range)
    d = (np.abs(s).max(axis=1) / 127.0).astype(np.float16)
    df = d.astype(np.float64)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.clip(np.where(df > 0, np.rint(s / df), 0), -128, 127)
        step = (df * sc)[:, :, None]
        q = np.where(step != 0, np.rint(b / step), 0)
    q = (np.clip(q, -32, 31) + 32).reshape(-1, 256)
    return pack_q6_k(d, sc.astype(np.int8), q.astype(np.uint8))


def random_q4_k_blocks(rng, n, k, d_lo=0.0005, d_hi=0.002):
    """Q4_K blocks with d, dmin ~ U(d_lo, d_hi) (f16), random 6-bit (scale, min) pairs and
    q ~ U{0..15}."""
    nb = n * k // QK_K
    d = rng.uniform(d_lo, d_hi, nb).astype(np.float16)
    dmin = rng.uniform(d_lo, d_hi, nb).astype(np.float16)
    sc = rng.integers(0, 64, (nb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (nb, 8), dtype=np.uint8)
    q = rng.integers(0, 16, (nb, 256), dtype=np.uint8)
    return pack_q4_k(d, dmin, sc, mn, q)


def random_q6_k_blocks(rng, n, k, d_lo=0.0001, d_hi=0.0005):
    """Q6_K blocks with d ~ U(d_lo, d_hi) (f16), int8 scales ~ U{-128..127}, q ~ U{0..63}."""
    nb = n * k // QK_K
    d = rng.uniform(d_lo, d_hi, nb).astype(np.float16)
    sc = rng.integers(-128, 128, (nb, 16)).astype(np.int8)
    q = rng.integers(0, 64, (nb, 256), dtype=np.uint8)
    return pack_q6_k(d, sc, q)
