"""GPU parity of the K-quant (Q4_K / Q6_K) residency, dequantization and fused quantized
linear against the CPU oracle (quantized.rs:268-415 restated in oracle/), through the C ABI.

max-rel-err = max_i |a_i - b_i| / max(max_j |b_j|, 1e-30); dequant bit-exact, the quantized
linear 1e-4 on the f32 paths and 1e-2 on the f16-MFMA prefill path (weights dequantized to
f16 operand order, X rounded to f16)."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import oracle
from tl_amd import GGML_Q4_K, GGML_Q6_K, BackendError, QTensor, _lib
from tl_amd.quant import random_q4_k_blocks, random_q6_k_blocks

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
F32_TOL, F16_TOL = 1e-4, 1e-2


def max_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)) if b.size else 0.0


def assert_rel(a, b, tol):
    err = max_rel(a, b)
    if not err <= tol:
        raise AssertionError(f"max-rel-err {err:.3e} > {tol:.0e}")


def blocks(t, rng, n, k):
    return random_q4_k_blocks(rng, n, k) if t == GGML_Q4_K else random_q6_k_blocks(rng, n, k)


def test_dequant_golden_k_blocks(dev):
    with open(os.path.join(HERE, "golden", "k_blocks.json")) as f:
        cases = json.load(f)["cases"]
    for t, name in ((GGML_Q4_K, "Q4_K"), (GGML_Q6_K, "Q6_K")):
        sel = [c for c in cases if c["type"] == name]
        raw = b"".join(bytes.fromhex(c["hex"]) for c in sel)  # one row per golden block
        got = dev.qtensor_dequantize(QTensor(t, raw, (len(sel), 256))).to_numpy()
        for i, c in enumerate(sel):
            assert list(got[i].view(np.uint32)) == c["f32_bits"], c["name"]


@pytest.mark.parametrize("t", [GGML_Q4_K, GGML_Q6_K])
@pytest.mark.parametrize("nk", [(4096, 4096), (11008, 4096), (64, 11008), (32000, 2048)])
def test_dequant_bit_exact(dev, t, nk):
    n, k = nk
    rng = np.random.default_rng(0x71540000 + n + k + t)
    raw = blocks(t, rng, n, k)
    got = dev.qtensor_dequantize(QTensor(t, raw, (n, k))).to_numpy()
    ref = oracle.dequantize(t, raw, n * k).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", [GGML_Q4_K, GGML_Q6_K])
@pytest.mark.parametrize("nk", [(4096, 4096), (11008, 4096), (4096, 11008), (2560, 2048), (256, 2048),
                                (5632, 2048), (2048, 5632), (32000, 2048), (8, 256), (100, 512)])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_kquant_matvec(dev, t, nk, m):
    n, k = nk
    rng = np.random.default_rng(0x71550000 + 7 * n + k + m + t)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = dev.tl_qtensor_matmul(dev.tensor_new(x), QTensor(t, raw, (n, k))).to_numpy()
    assert_rel(y, oracle.qtensor_matmul(x, raw, t, n), F32_TOL)


@pytest.mark.parametrize("t", [GGML_Q4_K, GGML_Q6_K])
@pytest.mark.parametrize("m", [5, 16, 128])
@pytest.mark.parametrize("nk", [(4096, 4096), (1024, 11008), (300, 768), (2048, 5632)])
def test_kquant_gemm(dev, t, m, nk):
    n, k = nk
    rng = np.random.default_rng(0x71560000 + m + n + t)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q = QTensor(t, raw, (n, k))
    xt = dev.tensor_new(x)
    ref = oracle.qtensor_matmul(x, raw, t, n)
    assert_rel(dev.tl_qtensor_matmul(xt, q).to_numpy(), ref, F32_TOL)
    assert_rel(dev.tl_qtensor_matmul_f16(xt, q).to_numpy(), ref, F16_TOL)


@pytest.mark.parametrize("t", [GGML_Q4_K, GGML_Q6_K])
@pytest.mark.parametrize("n", [8192, 11264])
def test_kquant_gemm_f16_wide_tiles(dev, t, n):
    """512 x 8192 and 512 x 11264 outputs on the wide tiles (the shapes above all take the
    128 x 32 tiles): Q4_K straight from its blocks with per-unit scale words, 128 x 64 tiles
    and, at 11264 (704 tiles of 64 > 512 two-per-CU slots), 128 x 96; Q6_K through its f16
    copy on 128 x 64 tiles.  Short K keeps the oracle fast."""
    m, k = 512, 256
    rng = np.random.default_rng(0x71570000 + t + n)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = oracle.qtensor_matmul(x, raw, t, n)
    assert_rel(dev.tl_qtensor_matmul_f16(dev.tensor_new(x), QTensor(t, raw, (n, k))).to_numpy(), ref, F16_TOL)
    v = [C.c_int32() for _ in range(3)]
    assert _lib.load().tl_hip_debug_last_gemm_plan(*[C.byref(x) for x in v]) == 0
    assert (v[0].value, v[1].value) == (128, 96 if t == GGML_Q4_K and n == 11264 else 64)


def test_kquant_upload_errors(dev):
    with pytest.raises(BackendError) as e:  # quantized.rs:347-352
        dev.qtensor_dequantize(QTensor(GGML_Q4_K, bytes(143), (1, 256)))
    assert e.value.variant == "ArgumentError"
    with pytest.raises(BackendError) as e:  # quantized.rs:278-283
        dev.qtensor_dequantize(QTensor(GGML_Q6_K, bytes(211), (1, 256)))
    assert e.value.variant == "ArgumentError"
    with pytest.raises(BackendError) as e:  # rows must hold whole 256-weight blocks
        dev.qtensor_dequantize(QTensor(GGML_Q4_K, bytes(288), (4, 128)))
    assert e.value.variant == "ShapeMismatch"
