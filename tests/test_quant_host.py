"""Host-side GGUF block encoders (tl_amd.quant) against the oracle's decoders and the
published llama.cpp quantizer rules."""
import numpy as np

import oracle
from tl_amd.quant import quantize_q4_0, quantize_q8_0, random_q4_0_blocks, random_q8_0_blocks


def test_q4_0_encoder_roundtrip_error_bound():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    blk = quantize_q4_0(x)
    assert blk.size == 64 * 256 // 32 * 18
    y = oracle.dequantize(2, blk, x.size).reshape(x.shape)
    d = np.abs(blk.reshape(-1, 18)[:, :2].copy().view(np.float16).astype(np.float32)).reshape(64, 8)
    err = np.abs(y - x).reshape(64, 8, 32).max(-1)
    # |x - d(q-8)| <= |d|/2 up to f16 rounding of d, except values of the opposite sign to the
    # block extreme, which the clamp at q = 15 can move by up to |d|
    assert np.all(err <= d * 1.01 + 1e-7)
    assert np.median(err / d) < 0.5


def test_q4_0_encoder_extreme_maps_to_minus_8():
    x = np.zeros(32, np.float32)
    x[5] = -3.0
    x[7] = 1.5
    blk = quantize_q4_0(x)
    y = oracle.dequantize(2, blk, 32)
    assert y[5] == -3.0  # d = m / -8 -> m maps to nibble 0 (value -8 d), exact here
    assert y[7] == 1.5


def test_q8_0_encoder_roundtrip_and_rounding():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((16, 128)).astype(np.float32)
    blk = quantize_q8_0(x)
    y = oracle.dequantize(8, blk, x.size).reshape(x.shape)
    amax = np.abs(x).reshape(16, 4, 32).max(-1)
    # d/2 rounding plus 127 * (f16 rounding of d, <= 2^-11 relative)
    assert np.all(np.abs(y - x).reshape(16, 4, 32).max(-1) <= amax / 127 * (0.5 + 127 * 2.0 ** -11) + 1e-7)
    # roundf: half away from zero
    z = np.zeros(32, np.float32)
    z[0], z[1], z[2] = 127.0, 2.5, -2.5
    q = quantize_q8_0(z).reshape(34)[2:].view(np.int8)
    assert q[0] == 127 and q[1] == 3 and q[2] == -3


def test_random_block_generators():
    rng = np.random.default_rng(13)
    b4 = random_q4_0_blocks(rng, 8, 64).reshape(-1, 18)
    d = b4[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.all((d >= 0.00099) & (d <= 0.0201))
    b8 = random_q8_0_blocks(rng, 8, 64).reshape(-1, 34)
    assert b8[:, 2:].view(np.int8).min() >= -127


def test_k_packers_match_golden_blocks():
    # the vectorised packers used for synthetic models produce the golden generator's bytes
    import importlib.util
    import json
    import os
    from tl_amd.quant import pack_q4_k, pack_q6_k
    here = os.path.dirname(os.path.abspath(__file__))
    spec = importlib.util.spec_from_file_location("mk", os.path.join(here, "golden", "make_k_blocks.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    rng = np.random.default_rng(14)
    for _ in range(5):
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        ref, _ = mk.pack_q4_k(0x3C00, 0x3800, [int(v) for v in sc], [int(v) for v in mn], [int(v) for v in q])
        got = pack_q4_k(np.array([1.0]), np.array([0.5]), sc[None].astype(np.uint8), mn[None].astype(np.uint8),
                        q[None].astype(np.uint8))
        assert bytes(got) == ref
        s6, q6 = rng.integers(-128, 128, 16), rng.integers(0, 64, 256)
        ref, _ = mk.pack_q6_k(0xB800, [int(v) for v in s6], [int(v) for v in q6])
        got = pack_q6_k(np.array([-0.5]), s6[None].astype(np.int8), q6[None].astype(np.uint8))
        assert bytes(got) == ref


def test_k_quantizers_roundtrip():
    from tl_amd.quant import quantize_q4_k, quantize_q6_k, random_q4_k_blocks, random_q6_k_blocks
    rng = np.random.default_rng(15)
    x = (rng.standard_normal((32, 512)) * 0.02).astype(np.float32)
    b4, b6 = quantize_q4_k(x), quantize_q6_k(x)
    assert b4.size == x.size // 256 * 144 and b6.size == x.size // 256 * 210
    e4 = oracle.dequantize(12, b4, x.size).reshape(x.shape) - x
    e6 = oracle.dequantize(14, b6, x.size).reshape(x.shape) - x
    rms = np.sqrt(np.mean(x ** 2))
    # 4-bit and 6-bit grids: relative rms error well under one step of each
    assert np.sqrt(np.mean(e4 ** 2)) < 0.12 * rms
    assert np.sqrt(np.mean(e6 ** 2)) < 0.03 * rms
    assert random_q4_k_blocks(rng, 4, 256).size == 4 * 144
    assert random_q6_k_blocks(rng, 4, 256).size == 4 * 210
