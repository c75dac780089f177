"""GPU parity: every HIP kernel on the path against the CPU oracle on the same seeded inputs,
called through the C ABI (tl_amd binds libtl_hip.so with ctypes).

max-rel-err = max_i |a_i - b_i| / max(max_j |b_j|, 1e-30); bounds from the north star:
bit-exact for dequant, 1e-4 for f32 paths, 1e-2 for f16 paths."""
import ctypes as C
import json
import math
import os

import numpy as np
import pytest

import oracle
from tl_amd import GGML_Q4_0, GGML_Q8_0, BackendError, QTensor, _lib
from tl_amd.quant import random_q4_0_blocks, random_q8_0_blocks

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
F32_TOL, F16_TOL = 1e-4, 1e-2


def max_rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)) if b.size else 0.0


def assert_rel(a, b, tol):
    err = max_rel(a, b)
    if not err <= tol:  # short message: no array dumps
        raise AssertionError(f"max-rel-err {err:.3e} > {tol:.0e}")


def blocks(t, rng, n, k):
    return random_q4_0_blocks(rng, n, k) if t == GGML_Q4_0 else random_q8_0_blocks(rng, n, k)


# ------------------------------------------------------------------ dequant (bit-exact)
def test_dequant_golden_blocks(dev):
    with open(os.path.join(HERE, "golden", "q_blocks.json")) as f:
        cases = json.load(f)["cases"]
    for c in cases:
        t = GGML_Q4_0 if c["type"] == "Q4_0" else GGML_Q8_0
        got = dev.qtensor_dequantize(QTensor(t, bytes.fromhex(c["hex"]), (1, 32))).to_numpy().reshape(-1)
        assert list(got.view(np.uint32)) == c["f32_bits"], c["name"]


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("nk", [(4096, 4096), (11008, 4096), (64, 11008)])
def test_dequant_bit_exact(dev, t, nk):
    n, k = nk
    rng = np.random.default_rng(0x71510000 + n + k + t)
    raw = blocks(t, rng, n, k)
    got = dev.qtensor_dequantize(QTensor(t, raw, (n, k))).to_numpy()
    ref = oracle.dequantize(t, raw, n * k).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------------ quantized linear
@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("nk", [(4096, 4096), (11008, 4096), (4096, 11008), (2560, 2048), (256, 2048),
                                (5632, 2048), (2048, 5632), (32, 32), (100, 96)])
@pytest.mark.parametrize("m", [1, 2, 4])
def test_quant_matvec(dev, t, nk, m):
    n, k = nk
    rng = np.random.default_rng(0x71510000 + 7 * n + k + m + t)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = dev.tl_qtensor_matmul(dev.tensor_new(x), QTensor(t, raw, (n, k))).to_numpy()
    ref = oracle.qtensor_matmul(x, raw, t, n)
    assert_rel(y, ref, F32_TOL)


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("m", [5, 16, 128, 512])
@pytest.mark.parametrize("nk", [(4096, 4096), (11008, 4096), (4096, 11008)])
def test_quant_gemm_f32_and_f16(dev, t, m, nk):
    """Every configs[2] shape at full size on both paths (the oracle's threaded product, bit-
    identical to the faithful loop, takes a few seconds at M = 512 x 11008 x 4096)."""
    n, k = nk
    rng = np.random.default_rng(0x71520000 + m + n + t)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q = QTensor(t, raw, (n, k))
    xt = dev.tensor_new(x)
    ref = oracle.qtensor_matmul(x, raw, t, n)
    y32 = dev.tl_qtensor_matmul(xt, q).to_numpy()
    assert_rel(y32, ref, F32_TOL)
    y16 = dev.tl_qtensor_matmul_f16(xt, q).to_numpy()
    assert_rel(y16, ref, F16_TOL)


def _gemm_plan():
    lib = _lib.load()
    v = [C.c_int32() for _ in range(3)]
    assert lib.tl_hip_debug_last_gemm_plan(*[C.byref(x) for x in v]) == 0
    return tuple(x.value for x in v)


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("nk", [(11008, 4096), (4096, 11008), (4096, 4096)])
def test_quant_gemm_f16_full_size_m512(dev, t, nk):
    """The prefill GEMMs bench.py times, at their full configs[2] size (M = 512, every row of
    W): the f16 MFMA path against the oracle's threaded f32 product (bit-identical to the
    faithful loop) within the f16 tolerance, and the launch plan that ran: 128 x 64 tiles (at
    least 256 of them in each shape), 128 x 96 for Q4_0 at N = 11008 (688 tiles of 64 would
    overflow the 512 two-per-CU slots, 460 of 96 do not), and for Q4_0 at K = 11008 the K
    range split in two (256 tiles, two workgroups per CU) with the partial sums added after."""
    n, k = nk
    m = 512
    rng = np.random.default_rng(0x71550000 + n + t)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y16 = dev.tl_qtensor_matmul_f16(dev.tensor_new(x), QTensor(t, raw, (n, k))).to_numpy()
    q4 = t == GGML_Q4_0
    assert _gemm_plan() == (128, 96 if q4 and n == 11008 else 64, 2 if q4 and k == 11008 else 1)
    ref = oracle.qtensor_matmul(x, raw, t, n, fast=True)
    assert_rel(y16, ref, F16_TOL)


@pytest.mark.parametrize("k,m", [(17408, 2), (17408, 4), (34816, 1)])
def test_qtensor_matmul_long_rows_take_the_gemm(dev, k, m):
    """Rows too long for the LDS-staged matvec (k >= 17408 at 2-4 rows, >= 34816 at one):
    tl_qtensor_matmul takes the tiled f32 GEMM instead of returning an error, as the
    reference accepts any [n, k] weight (system.rs:180-382)."""
    n = 96
    rng = np.random.default_rng(0x71560000 + k + m)
    raw = blocks(GGML_Q4_0, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = dev.tl_qtensor_matmul(dev.tensor_new(x), QTensor(GGML_Q4_0, raw, (n, k))).to_numpy()
    assert_rel(y, oracle.qtensor_matmul(x, raw, GGML_Q4_0, n), F32_TOL)


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("m", [33, 64, 65])
@pytest.mark.parametrize("nk", [(1000, 2176), (4096, 1152)])
def test_quant_gemm_f16_split_k(dev, t, m, nk):
    """Short inputs on the f16 GEMM: 64-row tiles (33, 64 rows) or 128-row tiles (65), the K
    range split over workgroup rows (17 and 9 iterations of 128: uneven splits) with the
    partial tiles added in order by a second kernel; within the f16 tolerance of the oracle."""
    n, k = nk
    rng = np.random.default_rng(0x71540000 + m + n + t)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = oracle.qtensor_matmul(x, raw, t, n)
    assert_rel(dev.tl_qtensor_matmul_f16(dev.tensor_new(x), QTensor(t, raw, (n, k))).to_numpy(), ref, F16_TOL)


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("m,n", [(512, 8192), (300, 8160), (300, 4096), (512, 11264), (300, 12008)])
def test_quant_gemm_f16_tile_widths(dev, t, m, n):
    """The f16 MFMA GEMM's tile widths: 128 x 64 tiles when they give >= 256 workgroups
    (512 x 8192, and 300 x 8160 with row and column counts off the tile), 128 x 32 below
    that (300 x 4096: 3 x 64 wide tiles), and for Q4_0 128 x 96 when more than 512 tiles of
    64 but at most 512 of 96 (512 x 11264; 300 x 12008 with a last tile of 8 columns and a
    last row tile of 44 rows); short K keeps the oracle fast."""
    k = 256
    rng = np.random.default_rng(0x71530000 + m + n + t)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = oracle.qtensor_matmul(x, raw, t, n)
    assert_rel(dev.tl_qtensor_matmul_f16(dev.tensor_new(x), QTensor(t, raw, (n, k))).to_numpy(), ref, F16_TOL)
    want = 32 if n == 4096 else 96 if t == GGML_Q4_0 and n > 8192 else 64
    assert _gemm_plan()[:2] == (128, want)


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
@pytest.mark.parametrize("m", [5, 16, 32, 33, 64])
def test_quant_gemm_f16_short_tiles_split_k(dev, t, m):
    """Op calls with 32- or 64-row tiles and K split over workgroup rows (17 iterations of 128:
    an uneven last range) -- or, up to 16 rows, the one-launch short-input kernel: the row
    tile that ran, the oracle within the f16 tolerance, and the same bits from the
    allocation-free entry on the same inputs."""
    n, k = 2048, 2176
    rng = np.random.default_rng(0x71570000 + m + t)
    raw = blocks(t, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q = QTensor(t, raw, (n, k))
    y16 = dev.tl_qtensor_matmul_f16(dev.tensor_new(x), q).to_numpy()
    plan = _gemm_plan()
    if m <= 16:
        assert plan[0] == (8 if m <= 8 else 16)
    else:
        assert plan[0] == (32 if m <= 32 else 64) and plan[2] > 1
    assert_rel(y16, oracle.qtensor_matmul(x, raw, t, n), F16_TOL)
    lib = _lib.load()
    hw = q.upload(lib)
    xt, yt = dev.tensor_new(x), dev.tensor_zeros((m, n))
    assert lib.tl_hip_launch_quant_gemm_noalloc(hw, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), m, 1, None) == 0
    assert np.array_equal(yt.to_numpy(), y16)


def test_qtensor_matmul_shapes_and_errors(dev):
    rng = np.random.default_rng(5)
    raw = random_q4_0_blocks(rng, 64, 128)
    q = QTensor(GGML_Q4_0, raw, (64, 128))
    x3 = rng.standard_normal((2, 3, 128)).astype(np.float32)  # leading dims are kept
    y = dev.tl_qtensor_matmul(dev.tensor_new(x3), q)
    assert y.shape == (2, 3, 64)
    np.testing.assert_allclose(y.to_numpy().reshape(6, 64), oracle.qtensor_matmul(x3.reshape(6, 128), raw, 2, 64),
                               rtol=1e-4, atol=1e-5)
    with pytest.raises(BackendError) as e:
        dev.tl_qtensor_matmul(dev.tensor_new(np.zeros((2, 96), np.float32)), q)
    assert e.value.variant == "ShapeMismatch"


# ------------------------------------------------------------------ fused row ops (config 1)
def test_rms_norm(dev):
    rng = np.random.default_rng(0x71510001)
    x = rng.standard_normal((512, 4096)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    got = dev.tensor_rms_norm(dev.tensor_new(x), dev.tensor_new(w), 1e-5).to_numpy()
    assert_rel(got, oracle.rms_norm(x, w, 1e-5), F32_TOL)
    x2 = rng.standard_normal((3, 2050)).astype(np.float32)  # odd width: generic kernel
    assert_rel(dev.tensor_rms_norm(dev.tensor_new(x2), None, 1e-5).to_numpy(), oracle.rms_norm(x2, None, 1e-5),
               F32_TOL)
    r = rng.standard_normal((512, 4096)).astype(np.float32)
    xt, rt, wt = dev.tensor_new(x), dev.tensor_new(r), dev.tensor_new(w)
    assert_rel(dev.fused_rms_norm(xt, wt, 1e-5).to_numpy(), oracle.fused_rms_norm(x, w, 1e-5), F32_TOL)
    assert_rel(dev.fused_add_rms_norm(xt, rt, wt, 1e-5).to_numpy(), oracle.fused_add_rms_norm(x, r, w, 1e-5),
               F32_TOL)


def test_fused_tier2_ops(dev):
    """fused_rotary_emb / fused_add_relu / fused_bias_gelu against the oracle (tl_cpu
    semantics): one head vector and a [16, 32, 64] input (the reference's overlapping pair
    indexing past the first vector), NaN in add_relu, bias broadcast, error paths."""
    rng = np.random.default_rng(0x71510002)
    f = rng.uniform(-4, 4, 32).astype(np.float32)
    for shape in ((64,), (16, 32, 64), (5, 64)):
        x = rng.standard_normal(shape).astype(np.float32)
        got = dev.fused_rotary_emb(dev.tensor_new(x), dev.tensor_new(f), 64).to_numpy()
        assert got.shape == shape
        assert_rel(got, oracle.fused_rotary_emb(x, f, 64), F32_TOL)
    a = rng.standard_normal((512, 4096)).astype(np.float32)
    b = rng.standard_normal((512, 4096)).astype(np.float32)
    a[0, :3] = [np.nan, -1.0, 1.0]
    got = dev.fused_add_relu(dev.tensor_new(a), dev.tensor_new(b)).to_numpy()
    np.testing.assert_array_equal(got, oracle.fused_add_relu(a, b))  # add and max are exact
    bias = rng.standard_normal(4096).astype(np.float32)
    assert_rel(dev.fused_bias_gelu(dev.tensor_new(a[1:]), dev.tensor_new(bias)).to_numpy(),
               oracle.fused_bias_gelu(a[1:], bias), F32_TOL)
    with pytest.raises(BackendError) as e:
        dev.fused_add_relu(dev.tensor_new(a), dev.tensor_new(b[:1]))
    assert e.value.variant == "ShapeMismatch"
    with pytest.raises(BackendError) as e:  # fewer than head_dim / 2 freqs
        dev.fused_rotary_emb(dev.tensor_new(a[0, :64]), dev.tensor_new(f[:8]), 64)
    assert e.value.variant == "ArgumentError"
    with pytest.raises(BackendError) as e:
        dev.fused_bias_gelu(dev.tensor_new(a), dev.tensor_new(np.zeros(0, np.float32)))
    assert e.value.variant == "ArgumentError"


def test_rope(dev):
    rng = np.random.default_rng(0x71510001)
    x = rng.standard_normal((512, 32, 128)).astype(np.float32)
    cos_d, sin_d = dev.tensor_rope_new_cos(128, 512, 10000.0), dev.tensor_rope_new_sin(128, 512, 10000.0)
    cos_h, sin_h = oracle.rope_table(512, 128, 10000.0), oracle.rope_table(512, 128, 10000.0, sin=True)
    assert_rel(cos_d.to_numpy(), cos_h, 1e-5)
    assert_rel(sin_d.to_numpy(), sin_h, 1e-5)
    xt = dev.tensor_new(x)
    # tl_cpu semantics: the (narrowed) table's first row for every vector
    for start in (0, 7, 300):
        cs = dev.tensor_narrow(cos_d, 0, start, 5)
        ss = dev.tensor_narrow(sin_d, 0, start, 5)
        got = dev.tensor_apply_rope(xt, cs, ss).to_numpy()
        assert_rel(got, oracle.apply_rope(x, cos_h[start:start + 5], sin_h[start:start + 5]), F32_TOL)
    # position-aware: token t rotated by row t, equal to per-token tl_cpu calls
    got = dev.tensor_apply_rope_pos(xt, cos_d, sin_d, 0, 32).to_numpy()
    ref = np.stack([oracle.apply_rope(x[t], cos_h[t:t + 1], sin_h[t:t + 1]) for t in range(512)])
    assert_rel(got, ref, F32_TOL)


def test_row_ops_kernel_shapes(dev):
    """The one-wavefront-per-row RMSNorm (widths up to 4096, multiple of 4) and the float4 RoPE
    (head sizes 4 .. 1024 floats with hd / 4 a power of two) next to their general kernels:
    widths 100, 2048, 4096 and 8192 with and without a weight or a residual; RoPE head sizes 4,
    64 and 96 (general kernel), tl_cpu's fixed row and per-token rows from pos0 = 5, and a table
    shorter than the positions (identity past its end, as tl_cpu's row bounds give)."""
    rng = np.random.default_rng(0x71510003)
    for rows, n in ((7, 100), (33, 2048), (5, 4096), (3, 8192)):
        x = rng.standard_normal((rows, n)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        r = rng.standard_normal((rows, n)).astype(np.float32)
        xt, wt, rt = dev.tensor_new(x), dev.tensor_new(w), dev.tensor_new(r)
        assert_rel(dev.tensor_rms_norm(xt, wt, 1e-5).to_numpy(), oracle.rms_norm(x, w, 1e-5), F32_TOL)
        assert_rel(dev.tensor_rms_norm(xt, None, 1e-5).to_numpy(), oracle.rms_norm(x, None, 1e-5), F32_TOL)
        assert_rel(dev.fused_add_rms_norm(xt, rt, wt, 1e-5).to_numpy(), oracle.fused_add_rms_norm(x, r, w, 1e-5),
                   F32_TOL)
    for tokens, heads, hd in ((9, 4, 64), (6, 3, 96), (11, 8, 4), (4, 2, 1024)):
        x = rng.standard_normal((tokens, heads, hd)).astype(np.float32)
        cos_d, sin_d = dev.tensor_rope_new_cos(hd, 12, 10000.0), dev.tensor_rope_new_sin(hd, 12, 10000.0)
        cos_h, sin_h = oracle.rope_table(12, hd, 10000.0), oracle.rope_table(12, hd, 10000.0, sin=True)
        xt = dev.tensor_new(x)
        got = dev.tensor_apply_rope(xt, dev.tensor_narrow(cos_d, 0, 3, 2), dev.tensor_narrow(sin_d, 0, 3, 2))
        assert_rel(got.to_numpy(), oracle.apply_rope(x, cos_h[3:5], sin_h[3:5]), F32_TOL)
        got = dev.tensor_apply_rope_pos(xt, cos_d, sin_d, 5, heads).to_numpy()
        for t in range(tokens):
            p = 5 + t
            if p < 12:
                want = oracle.apply_rope(x[t], cos_h[p:p + 1], sin_h[p:p + 1])
            else:  # past the table: cos 1, sin 0
                want = x[t]
            assert_rel(got[t], want, F32_TOL)


def test_swiglu(dev):
    rng = np.random.default_rng(0x71510001)
    g = rng.standard_normal((512, 11008)).astype(np.float32)
    u = rng.standard_normal((512, 11008)).astype(np.float32)
    gt, ut = dev.tensor_new(g), dev.tensor_new(u)
    unfused = dev.tensor_mul(dev.tensor_silu(gt), ut).to_numpy()
    ref = oracle.binop("mul", oracle.silu(g), u)
    assert_rel(unfused, ref, F32_TOL)
    assert_rel(dev.fused_silu_mul(gt, ut).to_numpy(), oracle.fused_silu_mul(g, u), F32_TOL)


def test_softmax(dev):
    rng = np.random.default_rng(0x71510001)
    x = (rng.standard_normal((512, 32000)) * 3).astype(np.float32)
    got = dev.tensor_softmax(dev.tensor_new(x), -1).to_numpy()
    assert_rel(got, oracle.softmax(x, -1), F32_TOL)
    np.testing.assert_allclose(got.sum(-1), 1.0, rtol=1e-4)
    y = (rng.standard_normal((4, 33, 6)) * 3).astype(np.float32)  # middle axis, odd size
    assert_rel(dev.tensor_softmax(dev.tensor_new(y), 1).to_numpy(), oracle.softmax(y, 1), F32_TOL)
    # causal-mask rows (the chatbot adds -inf above the diagonal): masked entries exactly 0
    z = (rng.standard_normal((64, 4096)) * 3).astype(np.float32)
    z[np.triu_indices(64, 1, 4096)] = -np.inf
    gz = dev.tensor_softmax(dev.tensor_new(z), -1).to_numpy()
    assert_rel(gz, oracle.softmax(z, -1), F32_TOL)
    assert np.all(gz[np.triu_indices(64, 1, 4096)] == 0.0)


# ------------------------------------------------------------------ decode attention (config 3)
@pytest.mark.parametrize("L", [512, 2048, 8192])
@pytest.mark.parametrize("B", [1, 8])
def test_attention_decode_f16_kv(dev, L, B):
    rng = np.random.default_rng(0x71530000 + L + B)
    hq, hkv, d = 32, 8, 128
    q = rng.standard_normal((B, hq, d)).astype(np.float16)
    k = rng.standard_normal((B, hkv, L, d)).astype(np.float16)
    v = rng.standard_normal((B, hkv, L, d)).astype(np.float16)
    got = dev.attention_decode(dev.tensor_new(q.astype(np.float32)), dev.tensor_new_f16(k),
                               dev.tensor_new_f16(v), L, 1.0 / np.sqrt(128.0)).to_numpy()
    bsel = range(B) if L * B <= 4096 else [0, B - 1]  # oracle time: check first and last batch
    for b in bsel:
        ref = oracle.attention(q[b][None].astype(np.float32), k[b].astype(np.float32), v[b].astype(np.float32),
                               np.float32(1.0 / np.sqrt(128.0)), False).reshape(hq, d)
        assert_rel(got[b], ref, F32_TOL)


@pytest.mark.parametrize("d,hq,hkv,lmax,L,B", [(64, 32, 4, 2000, 1500, 2), (128, 32, 4, 1100, 1031, 1),
                                               (64, 16, 4, 1400, 1025, 3), (128, 64, 8, 4096, 4096, 1)])
def test_attention_grouped_split_lengths(dev, d, hq, hkv, lmax, L, B):
    # caches longer than 1024 positions take the grouped-query split kernel: lengths that end
    # inside a 128-position split, 4 and 8 query heads per KV head, head_dim 64 and 128
    rng = np.random.default_rng(0x71570000 + L + d + B)
    q = rng.standard_normal((B, hq, d)).astype(np.float32)
    k = rng.standard_normal((B, hkv, lmax, d)).astype(np.float16)
    v = rng.standard_normal((B, hkv, lmax, d)).astype(np.float16)
    got = dev.attention_decode(dev.tensor_new(q), dev.tensor_new_f16(k), dev.tensor_new_f16(v), L,
                               1.0 / np.sqrt(d)).to_numpy()
    for b in range(B):
        ref = oracle.attention(q[b][None], k[b, :, :L].astype(np.float32), v[b, :, :L].astype(np.float32),
                               np.float32(1.0 / np.sqrt(d)), False).reshape(hq, d)
        assert_rel(got[b], ref, F32_TOL)


@pytest.mark.parametrize("d,hq,hkv,lmax,L,B", [(128, 32, 8, 512, 512, 1), (128, 32, 8, 512, 512, 8),
                                               (128, 32, 8, 300, 65, 2), (64, 64, 8, 500, 449, 2),
                                               (128, 32, 4, 256, 200, 3), (128, 32, 8, 2048, 2048, 1),
                                               (64, 64, 8, 4096, 4001, 1)])
def test_attention_one_launch_and_two_launch(dev, d, hq, hkv, lmax, L, B):
    """The grouped split form with its records merged by the last-arriving workgroup of each
    (batch item, KV head) -- one launch, taken for up to 8 splits: the first five cases, with
    lengths ending inside a split -- and with the separate merge kernel: both within the f32
    tolerance of the oracle, and the one-launch form bitwise equal over repeated calls (its
    arrival counters return to zero after every call).  The last two cases have more splits
    and take the merge kernel either way."""
    rng = np.random.default_rng(0x715B0000 + L + d + B + hkv)
    q = rng.standard_normal((B, hq, d)).astype(np.float32)
    k = rng.standard_normal((B, hkv, lmax, d)).astype(np.float16)
    v = rng.standard_normal((B, hkv, lmax, d)).astype(np.float16)
    qt, kt, vt = dev.tensor_new(q), dev.tensor_new_f16(k), dev.tensor_new_f16(v)
    scale = 1.0 / np.sqrt(d)
    lib = dev.lib
    prev = lib.tl_hip_debug_one_launch_merge(1)
    try:
        one = [dev.attention_decode(qt, kt, vt, L, scale).to_numpy() for _ in range(3)]
        lib.tl_hip_debug_one_launch_merge(0)
        two = dev.attention_decode(qt, kt, vt, L, scale).to_numpy()
    finally:
        lib.tl_hip_debug_one_launch_merge(prev)
    for r in one[1:]:
        assert np.array_equal(r.view(np.uint32), one[0].view(np.uint32))
    for b in sorted({0, B - 1}):
        ref = oracle.attention(q[b][None], k[b, :, :L].astype(np.float32), v[b, :, :L].astype(np.float32),
                               np.float32(scale), False).reshape(hq, d)
        assert_rel(one[0][b], ref, F32_TOL)
        assert_rel(two[b], ref, F32_TOL)


@pytest.mark.parametrize("d,hq,hkv,lmax,pos0,n", [(64, 32, 4, 600, 0, 512), (64, 16, 2, 300, 0, 37),
                                                  (128, 32, 8, 1100, 0, 1031), (128, 16, 4, 700, 333, 250),
                                                  (64, 8, 1, 200, 45, 1), (128, 16, 2, 256, 100, 100)])
def test_attention_prefill_causal(dev, d, hq, hkv, lmax, pos0, n):
    """The f16-MFMA causal prefill against the oracle's chatbot attention: at pos0 = 0 the
    masked form (chatbot.tl:76-81); later starts (chunked prompts) as one unmasked row per
    query over the positions it sees.  Query counts off the kernel's 16 / 32-query block,
    cache rows past the last query hold NaN (masked rows must not leak into the output)."""
    rng = np.random.default_rng(0x71590000 + d + hq + pos0 + n)
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    k = rng.standard_normal((hkv, lmax, d)).astype(np.float16)
    v = rng.standard_normal((hkv, lmax, d)).astype(np.float16)
    k[:, pos0 + n:] = np.nan
    v[:, pos0 + n:] = np.nan
    scale = np.float32(1.0 / np.sqrt(d))
    got = dev.attention_prefill(dev.tensor_new(q), dev.tensor_new_f16(k), dev.tensor_new_f16(v), pos0,
                                scale).to_numpy()
    assert got.shape == (n, hq, d) and np.isfinite(got).all()
    kf, vf = k.astype(np.float32), v.astype(np.float32)
    if pos0 == 0:
        ref = oracle.attention(q, kf[:, :n], vf[:, :n], scale, n > 1).reshape(n, hq, d)
        assert_rel(got, ref, F16_TOL)
    else:
        for i in sorted({0, 1, n // 2, n - 2, n - 1} & set(range(n))):
            L = pos0 + i + 1
            ref = oracle.attention(q[i][None], kf[:, :L], vf[:, :L], scale, False).reshape(hq, d)
            assert_rel(got[i], ref, F16_TOL)


def test_attention_prefill_errors(dev):
    q = dev.tensor_new(np.zeros((4, 8, 64), np.float32))
    kv = dev.tensor_new_f16(np.zeros((2, 16, 64), np.float16))
    with pytest.raises(BackendError) as e:  # 4 query heads per KV head: fine; 13 + 4 > 16 rows
        dev.attention_prefill(q, kv, kv, 13, 0.125)
    assert e.value.variant == "ArgumentError"
    kv4 = dev.tensor_new_f16(np.zeros((4, 16, 64), np.float16))
    with pytest.raises(BackendError) as e:  # 2 query heads per KV head: not covered
        dev.attention_prefill(q, kv4, kv4, 0, 0.125)
    assert e.value.variant == "ArgumentError"
    with pytest.raises(BackendError) as e:
        dev.attention_prefill(q, dev.tensor_new(np.zeros((2, 16, 64), np.float32)), kv, 0, 0.125)
    assert e.value.variant == "TypeMismatch"
    assert dev.attention_prefill(q, kv, kv, 12, 0.125).to_numpy().shape == (4, 8, 64)


def test_attention_decode_partial_length_and_f32_cache(dev):
    rng = np.random.default_rng(17)
    q = rng.standard_normal((2, 32, 64)).astype(np.float32)
    k = rng.standard_normal((2, 4, 300, 64)).astype(np.float32)
    v = rng.standard_normal((2, 4, 300, 64)).astype(np.float32)
    got = dev.attention_decode(dev.tensor_new(q), dev.tensor_new(k), dev.tensor_new(v), 129, 0.125).to_numpy()
    for b in range(2):
        ref = oracle.attention(q[b][None], k[b, :, :129], v[b, :, :129], 0.125, False).reshape(32, 64)
        assert_rel(got[b], ref, F32_TOL)
    # L = 1: the output is the first V row of each query head's KV head (h // 8)
    one = dev.attention_decode(dev.tensor_new(q), dev.tensor_new(k), dev.tensor_new(v), 1, 0.125).to_numpy()
    assert_rel(one[0], np.repeat(v[0, :, 0], 8, axis=0), 1e-6)


# ------------------------------------------------------------------ glue ops
def test_glue_ops(dev):
    rng = np.random.default_rng(21)
    x = rng.standard_normal((1, 5, 4, 16)).astype(np.float32)
    xt = dev.tensor_new(x)
    assert np.array_equal(dev.tensor_transpose(xt, 1, 2).to_numpy(), oracle.transpose(x, 1, 2))
    assert np.array_equal(dev.tensor_repeat_interleave(xt, 8, 2).to_numpy(), oracle.repeat_interleave(x, 8, 2))
    y = rng.standard_normal((1, 3, 4, 16)).astype(np.float32)
    assert np.array_equal(dev.tensor_cat(xt, dev.tensor_new(y), 1).to_numpy(), oracle.cat(x, y, 1))
    assert np.array_equal(dev.tensor_narrow(xt, 1, 2, 3).to_numpy(), oracle.narrow(x, 1, 2, 3))
    a2 = rng.standard_normal((300, 77)).astype(np.float32)
    assert np.array_equal(dev.tensor_transpose_2d(dev.tensor_new(a2)).to_numpy(), a2.T)
    assert np.array_equal(dev.tensor_new_causal_mask(6).to_numpy(), oracle.causal_mask(6))
    assert np.array_equal(dev.tensor_scale(xt, 0.125).to_numpy(), oracle.scale(x, 0.125))
    b = rng.standard_normal(16).astype(np.float32)
    bt = dev.tensor_new(b)
    for op, fn in (("add", dev.tensor_add), ("mul", dev.tensor_mul), ("sub", dev.tensor_sub), ("div", dev.tensor_div)):
        assert np.array_equal(fn(xt, bt).to_numpy(), oracle.binop(op, x, b)), op
    with pytest.raises(BackendError) as e:
        dev.tensor_add(xt, dev.tensor_new(np.ones(3, np.float32)))
    assert e.value.variant == "ShapeMismatch"


def test_matmul_batched(dev):
    rng = np.random.default_rng(22)
    a = rng.standard_normal((1, 32, 7, 64)).astype(np.float32)
    b = rng.standard_normal((1, 32, 64, 130)).astype(np.float32)
    got = dev.tensor_matmul(dev.tensor_new(a), dev.tensor_new(b)).to_numpy()
    assert_rel(got, oracle.matmul(a, b), F32_TOL)
    b2 = rng.standard_normal((64, 5)).astype(np.float32)
    assert_rel(dev.tensor_matmul(dev.tensor_new(a), dev.tensor_new(b2)).to_numpy(), oracle.matmul(a, b2), F32_TOL)
    v = rng.standard_normal(64).astype(np.float32)
    got = dev.tensor_matmul(dev.tensor_new(a[0, 0]), dev.tensor_new(v))
    assert got.shape == (7,)
    assert_rel(got.to_numpy(), oracle.matmul(a[0, 0], v), F32_TOL)


def test_embedding_argmax_penalty(dev):
    rng = np.random.default_rng(23)
    table = rng.standard_normal((1000, 64)).astype(np.float32)
    ids = np.array([3, 999, 0, 3], np.float32)
    tt = dev.tensor_new(table)
    assert np.array_equal(dev.tensor_embedding(tt, dev.tensor_new(ids)).to_numpy(), oracle.embedding(table, ids))
    with pytest.raises(BackendError) as e:
        dev.tensor_embedding(tt, dev.tensor_new(np.array([1000], np.float32)))
    assert e.value.variant == "IndexOutOfBounds"
    for arr in ([1, 5, 3, 5, 2], [7, 7, 7], [5, np.nan, 3], [1, 9, np.nan], list(rng.standard_normal(32000))):
        a = np.array(arr, np.float32)
        assert dev.tensor_argmax_all(dev.tensor_new(a)) == oracle.argmax_last(a)
    ties = np.zeros(32000, np.float32)
    ties[[5, 17000, 31999 - 3]] = 2.0
    assert dev.tensor_argmax_all(dev.tensor_new(ties)) == 31996
    s = dev.tensor_sample(dev.tensor_new(ties), 0.0, 0.9).to_numpy()
    assert s.shape == (1,) and s[0] == 31996.0
    lg = rng.standard_normal((2, 500)).astype(np.float32)
    tok = np.array([3, 3, 499, 17, -1], np.float32)
    got = dev.tensor_repetition_penalty(dev.tensor_new(lg), dev.tensor_new(tok), 1.1).to_numpy()
    assert np.array_equal(got, oracle.repetition_penalty(lg, tok, 1.1))


# ------------------------------------------------------------------ top-p sampling
def _choice(dev, t, temp, top_p, u):
    out = dev.tensor_sample_uniform(t, temp, top_p, float(u)).to_numpy()
    assert out.shape == (1,) and out[0] == int(out[0])
    return int(out[0])


@pytest.mark.parametrize("temp", [0.1, 0.7, 1.0, 2.5])
def test_sample_top_p_matches_oracle(dev, temp):
    """tl_hip_tensor_sample_uniform against sample_impl (tensor.rs:1641-1679): vocab-sized
    logits ~ N(0, 3) (32000, a ragged 131075, 7).  Every choice sits where the definition
    puts it in the float64 order (running sums bracket r within 4e-6); where top_p and r are
    clear of every summation's rounding the choice equals the oracle's and the float64
    restatement's.  The chatbot samples at temp 0.1, top_p 0.9 (chatbot.tl:189)."""
    from sampling_f64 import bracketed, decided, sample_f64
    rng = np.random.default_rng(0x5A40 + int(temp * 10))
    checked = total = 0
    for n in (32000, 131075, 7):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        t = dev.tensor_new(x)
        for top_p in (0.9, 0.5, 0.0, 0.75):
            for u in rng.random(6):
                got = _choice(dev, t, temp, top_p, u)
                assert bracketed(x, temp, top_p, u, got), (n, top_p, u, got)
                sel, margin, drift = sample_f64(x, temp, top_p, u)
                total += 1
                if decided(margin, drift):
                    checked += 1
                    assert got == sel == oracle.sample(x, temp, top_p, u), (n, top_p, u, got, sel)
    assert checked >= 0.5 * total, (checked, total)


def test_sample_top_p_ties_and_specials(dev):
    """Equal probabilities in index order, the cut and the choice by exact running sums;
    NaN / infinite inputs, temp <= 0, [1, V] logits, sizes 1 and 2, errors."""
    n = 32000
    t = dev.tensor_new(np.full(n, 0.5, np.float32))
    # every prob q = f32(1 / n); the running sum after j elements is j * v, v = q in 2^-47 units
    q = np.float32(1.0) / np.float32(n)
    v = int(float(q) * 2.0 ** 47)
    for top_p in (0.9, 0.3, 1.0):
        for u in (0.0, 0.25, 0.5, 0.999):
            tt = int(math.floor(float(np.float32(top_p)) * 2.0 ** 47))
            j_cut = min(tt // v + 1, n)  # n: the sum never exceeds top_p
            cutoff = np.float32(j_cut * v * 2.0 ** -47)
            r = np.float32(u) * cutoff
            j = max(1, -(-int(math.ceil(float(r) * 2.0 ** 47)) // v))
            want = j - 1 if j <= j_cut else 0  # past the cut: order[0]
            got = _choice(dev, t, 1.0, top_p, u)
            assert got == want, (top_p, u, got, want)
            # the reference's f32 running sums drift from j * q by a few places at most
            assert abs(oracle.sample(np.full(n, 0.5, np.float32), 1.0, top_p, u) - got) <= 64
    # two levels of ties: the four 3.0s first (indices 5, 9, 100, 999), then the rest in order
    x = np.zeros(1000, np.float32)
    x[[5, 9, 100, 999]] = 3.0
    for u in (0.0, 0.3, 0.6, 0.95):
        got = _choice(dev, dev.tensor_new(x), 1.0, 0.9, u)
        assert got == oracle.sample(x, 1.0, 0.9, u)
    # NaN / infinite logits or temp: index 0; temp <= 0: the greedy choice
    for arr, temp in (([1.0, np.nan, 3.0], 1.0), ([1.0, np.inf, 3.0], 1.0), ([-np.inf] * 5, 1.0),
                      ([1.0, 2.0, 3.0], float("nan"))):
        assert _choice(dev, dev.tensor_new(np.array(arr, np.float32)), temp, 0.9, 0.5) == 0
    g = np.array([1, 7, 3, 7, 2], np.float32)
    assert _choice(dev, dev.tensor_new(g), 0.0, 0.9, 0.5) == 3
    assert _choice(dev, dev.tensor_new(g), -2.0, 0.9, 0.5) == 3
    # [1, V] logits (the chatbot's narrowed row) are taken whole; n = 1 and n = 2
    rng = np.random.default_rng(99)
    row = (rng.standard_normal((1, 32000)) * 3).astype(np.float32)
    assert _choice(dev, dev.tensor_new(row), 0.1, 0.9, 0.3) == oracle.sample(row, 0.1, 0.9, 0.3)
    assert _choice(dev, dev.tensor_new(np.array([4.0], np.float32)), 1.0, 0.9, 0.7) == 0
    ln3 = np.float32(math.log(3.0))
    two = dev.tensor_new(np.array([0.0, ln3], np.float32))
    assert [_choice(dev, two, 1.0, 0.9, u) for u in (0.0, 0.5, 0.8)] == [1, 1, 0]
    assert _choice(dev, two, 1.0, 0.5, 0.99) == 1
    for tp in (float("nan"), 1e6):  # never exceeded: no cut (the kernel skips the cut's descent)
        assert [_choice(dev, two, 1.0, tp, u) for u in (0.0, 0.5, 0.8)] == [1, 1, 0]
        assert _choice(dev, t, 1.0, tp, 0.999) == oracle.sample(np.full(n, 0.5, np.float32), 1.0, tp, 0.999)
    with pytest.raises(BackendError) as e:
        dev.tensor_sample_uniform(dev.tensor_new(np.zeros(0, np.float32)), 1.0, 0.9, 0.5)
    assert e.value.variant == "InternalError"
    for bad_u in (-0.1, 1.0, float("nan")):
        with pytest.raises(BackendError) as e:
            dev.tensor_sample_uniform(two, 1.0, 0.9, bad_u)
        assert e.value.variant == "ArgumentError"


def test_sample_seeded_draws(dev):
    """tl_hip_tensor_sample draws u from the calling thread's splitmix64 generator: after
    tl_hip_sample_seed its choices equal sample_uniform at the replayed draws."""
    from sampling_f64 import splitmix64_uniforms
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(32000) * 3).astype(np.float32)
    t = dev.tensor_new(x)
    for temp, top_p in ((0.1, 0.9), (1.0, 0.95)):
        dev.sample_seed(1234)
        got = [int(dev.tensor_sample(t, temp, top_p).to_numpy()[0]) for _ in range(12)]
        want = [_choice(dev, t, temp, top_p, u) for u in splitmix64_uniforms(1234, 12)]
        assert got == want
    assert len(set(got)) > 1  # temp 1: the draws spread over several tokens


# ------------------------------------------------------ scaled dot-product attention
@pytest.mark.parametrize("qshape,sk,dv,mask", [
    ((2, 4, 33, 64), 33, 64, "causal"),      # 4-D, causal ones mask (the chatbot's case)
    ((2, 4, 1, 128), 700, 128, None),        # decode-like: one query, many keys
    ((8, 17, 32), 129, 48, "random"),        # 3-D, d_v != d_k, zeros drop keys
    ((5, 16), 3, 7, "rowzero"),              # 2-D, a fully masked row
    ((3, 300, 64), 300, 64, "short"),        # mask shorter than seq_q * seq_k
])
def test_scaled_dot_product_attention(dev, qshape, sk, dv, mask):
    """tensor_scaled_dot_product_attention against the oracle's restatement of tl_cpu
    (device_impl.rs:775-872) within the f32 tolerance: scale 1/sqrt(d_k), mask == 0 -> -1e9,
    other mask values ignored, ranks 2-4."""
    rng = np.random.default_rng(0x71570000 + sk + dv)
    q = rng.standard_normal(qshape).astype(np.float32)
    k = rng.standard_normal(qshape[:-2] + (sk, qshape[-1])).astype(np.float32)
    v = rng.standard_normal(qshape[:-2] + (sk, dv)).astype(np.float32)
    sq = qshape[-2]
    m = None
    if mask == "causal":
        m = np.tril(np.ones((sq, sk), np.float32))
    elif mask == "random":
        keep = rng.random((sq, sk)) > 0.5
        m = np.where(keep, rng.choice([1.0, -np.inf, 3.0], (sq, sk)), 0.0).astype(np.float32)
    elif mask == "rowzero":
        m = np.ones((sq, sk), np.float32)
        m[2] = 0.0
    elif mask == "short":
        m = (rng.random(sq * sk // 3) > 0.3).astype(np.float32)
    ref = oracle.sdpa(q, k, v, m)
    got = dev.tensor_scaled_dot_product_attention(dev.tensor_new(q), dev.tensor_new(k), dev.tensor_new(v),
                                                  dev.tensor_new(m) if m is not None else None).to_numpy()
    assert got.shape == ref.shape
    assert_rel(got, ref, F32_TOL)


def test_scaled_dot_product_attention_errors(dev):
    t = dev.tensor_new
    q = t(np.zeros((2, 3, 8), np.float32))
    with pytest.raises(BackendError) as e:   # head dims differ
        dev.tensor_scaled_dot_product_attention(q, t(np.zeros((2, 3, 4), np.float32)), t(np.zeros((2, 3, 4), np.float32)))
    assert e.value.variant == "ShapeMismatch"
    with pytest.raises(BackendError) as e:   # batch / heads differ
        dev.tensor_scaled_dot_product_attention(q, t(np.zeros((3, 3, 8), np.float32)), t(np.zeros((3, 3, 8), np.float32)))
    assert e.value.variant == "ShapeMismatch"
    with pytest.raises(BackendError) as e:   # rank 1
        v1 = t(np.zeros(8, np.float32))
        dev.tensor_scaled_dot_product_attention(v1, v1, v1)
    assert e.value.variant == "ShapeMismatch"
    # no keys: zeros of [.., seq_q, d_v]
    out = dev.tensor_scaled_dot_product_attention(q, t(np.zeros((2, 0, 8), np.float32)),
                                                  t(np.zeros((2, 0, 5), np.float32))).to_numpy()
    assert out.shape == (2, 3, 5) and np.all(out == 0)
