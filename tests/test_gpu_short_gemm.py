"""GPU parity of the short-input quantized GEMM (5 <= m <= 16 rows, f16 MFMA, one launch over
f32 X) against the CPU oracle, called through the C ABI (tl_qtensor_matmul_f16 and the raw
launcher).  Tolerance: the f16-path bound 1e-2 (max-rel-err as in test_gpu_kernels).

Covers the configs[2] shapes at M = 5, 8, 9 and 16 for Q4_0 and Q8_0, Q4_K (its per-unit
scale pairs), the launch plan (an M tile of 8 or 16, 16-row sub-tiles per tile, K splits),
run-to-run bit equality and bit equality of the one-launch slice sum (the tile's last split
adds the slices) with the two-launch one, and shapes whose K leaves some wavefronts of a workgroup no 128-k
group (K = 128 .. 896) or whose N is not a multiple of 16."""
import ctypes as C

import numpy as np
import pytest

import oracle
from tl_amd import GGML_Q4_0, GGML_Q4_K, GGML_Q8_0, QTensor, _lib
from tl_amd.quant import random_q4_0_blocks, random_q4_k_blocks, random_q8_0_blocks

pytestmark = pytest.mark.gpu
F16_TOL = 1e-2
GEN = {GGML_Q4_0: random_q4_0_blocks, GGML_Q8_0: random_q8_0_blocks, GGML_Q4_K: random_q4_k_blocks}


def max_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def plan():
    lib = _lib.load()
    v = [C.c_int32() for _ in range(3)]
    assert lib.tl_hip_debug_last_gemm_plan(*[C.byref(x) for x in v]) == 0
    return tuple(x.value for x in v)


def expected_plan(t, m, n, k, cus=256):
    """The launch plan: tiles of 4 wavefronts x 16 NR rows, NR = 2 for the 4-bit types at
    N >= 8192, else 1, and K split until two workgroups per CU run (at most one split per
    128-k group, at most 16)."""
    ng = k // 128
    nr = 2 if t != GGML_Q8_0 and n >= 8192 else 1
    tiles = -(-n // (64 * nr))
    nsp = 1
    if (m * n) % 4 == 0 and tiles < 2 * cus:
        nsp = min(-(-2 * cus // tiles), (ng + 1) // 2, 16)
    return (8 if m <= 8 else 16, 64 * nr, nsp)


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("nk", [(4096, 4096), (11008, 4096), (4096, 11008)])
@pytest.mark.parametrize("m", [5, 8, 9, 16])
def test_short_gemm_configs2(dev, t, nk, m):
    n, k = nk
    rng = np.random.default_rng(0x71570000 + 3 * m + n + t)
    raw = GEN[t](rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q = QTensor(t, raw, (n, k))
    xt = dev.tensor_new(x)
    y = dev.tl_qtensor_matmul_f16(xt, q).to_numpy()
    assert plan() == expected_plan(t, m, n, k)
    ref = oracle.qtensor_matmul(x, raw, t, n)
    err = max_rel(y, ref)
    assert err <= F16_TOL, f"max-rel-err {err:.3e}"
    # the same call again: bitwise equal (the K-split slices are added in slice order) -- and
    # so is the form that adds them in a second kernel instead of the tile's last-arriving split
    y2 = dev.tl_qtensor_matmul_f16(xt, q).to_numpy()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    lib = _lib.load()
    prev = lib.tl_hip_debug_one_launch_merge(0)
    try:
        y3 = dev.tl_qtensor_matmul_f16(xt, q).to_numpy()
    finally:
        lib.tl_hip_debug_one_launch_merge(prev)
    assert np.array_equal(y.view(np.uint32), y3.view(np.uint32))


@pytest.mark.parametrize("nk", [(4096, 4096), (2560, 2048), (32000, 2048)])
@pytest.mark.parametrize("m", [6, 16])
def test_short_gemm_q4_k(dev, nk, m):
    """Q4_K through the same kernel (its (d sc, -dmin m) unit pairs, built on the first f16
    call), up to the 32000-row LM-head shape."""
    n, k = nk
    rng = np.random.default_rng(0x71580000 + m + n)
    raw = random_q4_k_blocks(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = dev.tl_qtensor_matmul_f16(dev.tensor_new(x), QTensor(GGML_Q4_K, raw, (n, k))).to_numpy()
    assert plan() == expected_plan(GGML_Q4_K, m, n, k)
    ref = oracle.qtensor_matmul(x, raw, GGML_Q4_K, n)
    err = max_rel(y, ref)
    assert err <= F16_TOL, f"max-rel-err {err:.3e}"


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("nk", [(100, 128), (37, 384), (250, 896), (16, 1024), (1000, 2176)])
@pytest.mark.parametrize("m", [5, 11, 16])
def test_short_gemm_edges(dev, t, nk, m):
    """N not a multiple of 16 (rows past n read row n - 1 and are not stored) and K of 1-7
    groups of 128 (some of a workgroup's eight wavefronts have no K range and add zeros)."""
    n, k = nk
    rng = np.random.default_rng(0x71590000 + 5 * m + n + k + t)
    raw = GEN[t](rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q = QTensor(t, raw, (n, k))
    lib = _lib.load()
    hw = q.upload(lib)
    xt = dev.tensor_new(x)
    yt = dev.tensor_new(np.full((m, n + 3), np.nan, np.float32))   # 3 guard columns per row
    assert lib.tl_hip_launch_quant_gemm(hw, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), m, 1, None) == 0
    got = yt.to_numpy().reshape(-1)
    y = got[:m * n].reshape(m, n)
    assert np.isnan(got[m * n:]).all(), "stored past y"
    ref = oracle.qtensor_matmul(x, raw, t, n)
    err = max_rel(y, ref)
    assert err <= F16_TOL, f"max-rel-err {err:.3e}"


def test_short_gemm_special_values(dev):
    """An infinite X element reaches exactly the outputs of its row (inf or nan, as the f32
    oracle gives), a zero block scale contributes zero, and the other rows are untouched."""
    n, k, m = 64, 512, 7
    rng = np.random.default_rng(0x715A0000)
    raw = bytearray(random_q4_0_blocks(rng, n, k))
    raw[0:2] = b"\x00\x00"   # row 0, block 0: d = +0
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[3, 5] = np.inf
    y = dev.tl_qtensor_matmul_f16(dev.tensor_new(x), QTensor(GGML_Q4_0, bytes(raw), (n, k))).to_numpy()
    ref = oracle.qtensor_matmul(x, bytes(raw), GGML_Q4_0, n)
    assert np.array_equal(np.isfinite(y), np.isfinite(ref))
    fin = np.isfinite(ref)
    assert float(np.max(np.abs(y[fin] - ref[fin])) / np.max(np.abs(ref[fin]))) <= F16_TOL
