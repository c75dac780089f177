"""Pins the CPU oracle (oracle/) against golden vectors, reference known-answer tests and
closed forms.  CPU only."""
import json
import math
import os

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))


def test_f16_decode_all_patterns():
    # half 2.7.1 f16::to_f32 (quantized.rs:176) = IEEE binary16 decode; numpy float16 is an
    # independent implementation of the same standard
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    lib = oracle.lib()
    got = np.array([lib.tlo_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def _golden():
    with open(os.path.join(HERE, "golden", "q_blocks.json")) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden(), ids=lambda c: f"{c['type']}:{c['name']}")
def test_dequant_golden_blocks(case):
    t = 2 if case["type"] == "Q4_0" else 8
    got = oracle.dequantize(t, bytes.fromhex(case["hex"]), 32)
    assert list(got.view(np.uint32)) == case["f32_bits"]


def test_dequant_errors():
    # quantized.rs:190-200: numel % 32 and byte-count checks
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(2, bytes(18), 31)
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(2, bytes(17), 32)
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(8, bytes(33), 32)


def _k_golden():
    with open(os.path.join(HERE, "golden", "k_blocks.json")) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _k_golden(), ids=lambda c: f"{c['type']}:{c['name']}")
def test_dequant_k_golden_blocks(case):
    # blocks packed from chosen values by llama.cpp's encoders; expected values from those
    # values, so a wrong nibble, high-bit or scale index in the decoder fails here
    t = 12 if case["type"] == "Q4_K" else 14
    got = oracle.dequantize(t, bytes.fromhex(case["hex"]), 256)
    assert list(got.view(np.uint32)) == case["f32_bits"]


def test_dequant_k_errors():
    # quantized.rs:273-283 (Q6_K), 342-352 (Q4_K): numel % 256 and byte-count checks
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(12, bytes(144), 255)
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(12, bytes(143), 256)
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(14, bytes(210), 128)
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(14, bytes(211), 256)


def test_q4_layout_low_then_high_nibble():
    # a block whose byte 0 = 0x1F: element 0 = d*(0xF-8) = 7, element 16 = d*(1-8) = -7
    blk = bytes([0x00, 0x3C, 0x1F] + [0x88] * 15)
    v = oracle.dequantize(2, blk, 32)
    assert v[0] == 7.0 and v[16] == -7.0 and v[1] == 0.0


def test_matmul_reference_kat():
    # crates/tl_cpu/tests/cpu_tensor_tests.rs:488-497
    a = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], dtype=np.float32)
    assert np.array_equal(oracle.matmul(a, b), np.array([[58, 64], [139, 154]], dtype=np.float32))


def test_matmul_sequential_sum_and_fast_variant():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((5, 67)).astype(np.float32)
    b = rng.standard_normal((67, 9)).astype(np.float32)
    got = oracle.matmul(a, b)
    # left-to-right f32 sum with separately rounded products, restated in numpy
    ref = np.zeros((5, 9), dtype=np.float32)
    for p in range(67):
        ref = (ref + (a[:, p:p + 1] * b[p:p + 1, :]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(got, ref)
    assert np.array_equal(oracle.matmul_fast(a, b), got)
    # and close to the float64 product
    np.testing.assert_allclose(got, a.astype(np.float64) @ b.astype(np.float64), rtol=1e-5, atol=1e-5)


def test_matmul_batched_and_vector():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    b = rng.standard_normal((2, 3, 5, 6)).astype(np.float32)
    np.testing.assert_allclose(oracle.matmul(a, b), a @ b, rtol=1e-5, atol=1e-5)
    b2 = rng.standard_normal((5, 6)).astype(np.float32)   # rank-2 rhs is shared by all batches
    np.testing.assert_allclose(oracle.matmul(a, b2), a @ b2, rtol=1e-5, atol=1e-5)
    v = rng.standard_normal(5).astype(np.float32)         # 1-D rhs: column vector, no n dim
    np.testing.assert_allclose(oracle.matmul(a[0, 0], v), a[0, 0] @ v, rtol=1e-5, atol=1e-5)


def test_qtensor_matmul_is_dequant_transpose_matmul():
    from tl_amd.quant import random_q4_0_blocks
    rng = np.random.default_rng(3)
    n, k = 48, 96
    w = random_q4_0_blocks(rng, n, k)
    x = rng.standard_normal((3, k)).astype(np.float32)
    wf = oracle.dequantize(2, w, n * k).reshape(n, k)
    assert np.array_equal(oracle.qtensor_matmul(x, w, 2, n, fast=False), oracle.matmul(x, wf.T.copy()))
    assert np.array_equal(oracle.qtensor_matmul(x, w, 2, n, fast=True), oracle.qtensor_matmul(x, w, 2, n, fast=False))


def test_rms_norm_closed_form():
    # tl_cuda nn_llm_test.rs:123-132: x = [1,2,3,4], w = 1 -> x / sqrt(7.5 + eps)
    x = np.array([[1, 2, 3, 4]], dtype=np.float32)
    got = oracle.rms_norm(x, np.ones(4, np.float32), 1e-5)
    ref = x / np.float32(math.sqrt(7.5 + 1e-5))
    np.testing.assert_allclose(got, ref, rtol=1e-6)
    # divide then multiply (ffi.rs:2470 + mul_impl), each rounded
    w = np.array([0.5, 1.5, 2.0, 0.25], dtype=np.float32)
    rms = np.float32(np.sqrt(np.float32(np.float32(30.0) / np.float32(4.0)) + np.float32(1e-5)))
    assert np.array_equal(oracle.rms_norm(x, w, 1e-5), (x / rms) * w)
    # unit RMS before weighting
    rng = np.random.default_rng(4)
    y = oracle.rms_norm(rng.standard_normal((7, 300)).astype(np.float32), None, 0.0)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(axis=1)), 1.0, rtol=1e-5)


def test_fused_rms_norm_variants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    r = rng.standard_normal((4, 64)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-5) * w
    np.testing.assert_allclose(oracle.fused_rms_norm(x, w, 1e-5), ref, rtol=1e-5, atol=1e-6)
    xr = (x + r).astype(np.float32)
    np.testing.assert_allclose(oracle.fused_add_rms_norm(x, r, w, 1e-5), oracle.fused_rms_norm(xr, w, 1e-5),
                               rtol=0, atol=0)


def test_rope_tables():
    # nn_llm_test.rs:151-169: row 0 is cos 1 / sin 0; pairs share a value
    c = oracle.rope_table(16, 8, 10000.0)
    s = oracle.rope_table(16, 8, 10000.0, sin=True)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert np.array_equal(c[:, 0::2], c[:, 1::2]) and np.array_equal(s[:, 0::2], s[:, 1::2])
    pos = np.arange(16)[:, None].astype(np.float64)
    freq = 1.0 / 10000.0 ** (2 * np.arange(4) / 8.0)
    np.testing.assert_allclose(c[:, 0::2], np.cos(pos * freq), atol=2e-6)
    np.testing.assert_allclose(s[:, 0::2], np.sin(pos * freq), atol=2e-6)


def test_apply_rope_identity_rotation_and_row0():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 4, 8)).astype(np.float32)
    c = oracle.rope_table(10, 8, 10000.0)
    s = oracle.rope_table(10, 8, 10000.0, sin=True)
    # cuda_shader_test.rs:332-355: position 0 is the identity
    assert np.array_equal(oracle.apply_rope(x, c, s), x)
    # the narrowed table's FIRST row rotates every vector (ffi.rs:2662-2676)
    y = oracle.apply_rope(x, c[5:8], s[5:8])
    th = c[5, 0::2], s[5, 0::2]
    x0, x1 = x[..., 0::2], x[..., 1::2]
    np.testing.assert_allclose(y[..., 0::2], x0 * th[0] - x1 * th[1], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(y[..., 1::2], x0 * th[1] + x1 * th[0], rtol=1e-6, atol=1e-6)
    # rotation keeps each pair's norm
    n0 = x0 ** 2 + x1 ** 2
    n1 = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    np.testing.assert_allclose(n0, n1, rtol=1e-5)
    # entries past the table read as cos 1 / sin 0
    assert np.array_equal(oracle.apply_rope(x, c[:1, :4], s[:1, :4])[..., 4:], x[..., 4:])


def test_silu_softmax_closed_forms():
    x = np.array([-3, -1, 0, 0.5, 2, 10], dtype=np.float32)
    np.testing.assert_allclose(oracle.silu(x), x / (1 + np.exp(-x.astype(np.float64))), rtol=1e-6)
    assert oracle.silu(np.zeros(1, np.float32))[0] == 0.0
    rng = np.random.default_rng(7)
    z = (rng.standard_normal((5, 37)) * 3).astype(np.float32)
    p = oracle.softmax(z, -1)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-5)
    order = np.argsort(z, axis=-1)
    assert np.all(np.diff(np.take_along_axis(p, order, -1), axis=-1) >= 0)  # monotone
    e = np.exp(z.astype(np.float64) - z.max(-1, keepdims=True))
    np.testing.assert_allclose(p, e / e.sum(-1, keepdims=True), rtol=1e-5)
    # softmax over a middle axis
    np.testing.assert_allclose(oracle.softmax(z.reshape(5, 37, 1), 1)[..., 0], p, rtol=1e-6)


def test_argmax_last_among_ties_and_nan():
    assert oracle.argmax_last(np.array([1, 5, 3, 5, 2], np.float32)) == 3
    assert oracle.argmax_last(np.array([7, 7, 7], np.float32)) == 2
    assert oracle.argmax_last(np.array([-np.inf, -np.inf], np.float32)) == 1
    # a NaN compares Equal, so the fold moves to it and then to the next element
    assert oracle.argmax_last(np.array([5, np.nan, 3], np.float32)) == 2
    assert oracle.argmax_last(np.array([1, 9, np.nan], np.float32)) == 2


def test_sample_top_p_closed_forms():
    """sample_impl (tensor.rs:1626-1680) on distributions whose cutoff and choice follow by
    hand."""
    ln3 = math.log(3.0)
    # probs (1/4, 3/4): order [1, 0], running sums 3/4, 1
    assert oracle.sample([0.0, ln3], 1.0, 0.9, 0.5) == 1   # cut after both; r = 0.5 <= 3/4
    assert oracle.sample([0.0, ln3], 1.0, 0.9, 0.8) == 0   # r = 0.8 > 3/4: the second place
    assert oracle.sample([0.0, ln3], 1.0, 0.9, 0.0) == 1   # r = 0: the first place
    assert oracle.sample([0.0, ln3], 1.0, 0.5, 0.99) == 1  # 3/4 > 0.5: cut after the first
    assert oracle.sample([0.0, ln3], 2.0, 0.9, 0.8) == 0   # probs (0.366, 0.634): r = 0.8
    # four equal probs stay in index order: sums 0.25, 0.5, 0.75 > 0.6 -> cutoff 0.75
    assert oracle.sample([1.0, 1.0, 1.0, 1.0], 1.0, 0.6, 0.5) == 1    # r = 0.375
    assert oracle.sample([1.0, 1.0, 1.0, 1.0], 1.0, 0.6, 0.9) == 2    # r = 0.675
    assert oracle.sample([1.0, 1.0, 1.0, 1.0], 1.0, 0.6, 0.0) == 0
    assert oracle.sample([1.0, 1.0, 1.0, 1.0], 1.0, 1.5, 0.99) == 3   # never exceeds: all four
    assert oracle.sample([1.0, 1.0, 1.0, 1.0], 1.0, -1.0, 0.99) == 0  # cut after the first
    # a NaN top_p is never exceeded (cum_prob > NaN is false): no cut, as with top_p 1e6
    for tp in (float("nan"), 1e6):
        assert [oracle.sample([0.0, ln3], 1.0, tp, u) for u in (0.0, 0.5, 0.8)] == [1, 1, 0]
    # the top-probability element first, then ties in index order: [3, 1, 1, 3] -> 0, 3, 1, 2
    assert oracle.sample([3.0, 1.0, 1.0, 3.0], 1.0, 1.5, 0.6) == 3
    # a NaN or infinite logit, or a NaN temp, makes every prob NaN: index 0
    for x, t in (([1.0, np.nan, 3.0], 1.0), ([1.0, np.inf, 3.0], 1.0), ([-np.inf, -np.inf], 1.0),
                 ([1.0, 2.0, 3.0], np.nan)):
        assert oracle.sample(x, t, 0.6, 0.5) == 0
    # temp <= 0: the greedy choice, last index among equal maxima
    assert oracle.sample([1.0, 3.0, 3.0], 0.0, 0.6, 0.5) == 2
    assert oracle.sample([1.0, 3.0, 3.0], -1.0, 0.6, 0.5) == 2
    assert oracle.sample([], 1.0, 0.9, 0.5) == -1


@pytest.mark.parametrize("temp", [0.1, 0.7, 1.0, 2.5])
def test_sample_top_p_against_float64(temp):
    """The oracle's choice equals the float64 restatement (numpy stable argsort, cumulative
    sums) wherever top_p and r are clear of the f32 rounding of every running sum."""
    from sampling_f64 import bracketed, decided, sample_f64
    rng = np.random.default_rng(int(temp * 1000))
    checked = total = 0
    for n in (2, 17, 300, 4000):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        for top_p in (0.9, 0.5, 0.99, 0.0, 0.75):  # (top_p 1.0 sits on the last running sums)
            for u in rng.random(6):
                sel, margin, drift = sample_f64(x, temp, top_p, u)
                got = oracle.sample(x, temp, top_p, u)
                assert bracketed(x, temp, top_p, u, got, tol=4e-6 + 4 * drift), (n, top_p, u)
                total += 1
                if decided(margin, drift):
                    checked += 1
                    assert got == sel, (n, top_p, u)
    assert checked >= 0.9 * total


def test_glue_ops_match_numpy():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    assert np.array_equal(oracle.transpose(x, 1, 2), x.transpose(0, 2, 1, 3))
    assert np.array_equal(oracle.repeat_interleave(x, 3, 1), np.repeat(x, 3, axis=1))
    y = rng.standard_normal((2, 3, 2, 5)).astype(np.float32)
    assert np.array_equal(oracle.cat(x, y, 2), np.concatenate([x, y], 2))
    assert np.array_equal(oracle.narrow(x, 2, 1, 2), x[:, :, 1:3])
    m = oracle.causal_mask(4)
    assert np.array_equal(np.isinf(m), np.triu(np.ones((4, 4), bool), 1)) and np.all(m[np.tril_indices(4)] == 0)
    b = rng.standard_normal(5).astype(np.float32)
    assert np.array_equal(oracle.binop("mul", x, b), x * b)
    assert np.array_equal(oracle.binop("add", x, x), x + x)
    assert np.array_equal(oracle.scale(x, 0.125), x * np.float32(0.125))
    table = rng.standard_normal((10, 4)).astype(np.float32)
    assert np.array_equal(oracle.embedding(table, np.array([3, 0, 9], np.float32)), table[[3, 0, 9]])
    with pytest.raises(oracle.OracleError):
        oracle.embedding(table, np.array([10], np.float32))


def test_repetition_penalty():
    lg = np.array([[2.0, -2.0, 1.0, 0.0]], np.float32)
    out = oracle.repetition_penalty(lg, np.array([0, 1, 1, 7], np.float32), 2.0)
    assert np.array_equal(out, np.array([[1.0, -4.0, 1.0, 0.0]], np.float32))


def test_attention_direct_equals_op_chain():
    # tlo_attention restates chatbot.tl:63-87 directly; the literal op chain
    # (transpose / repeat_interleave / matmul_4d / scale / +mask / softmax / matmul_4d)
    # must give the same bits
    rng = np.random.default_rng(9)
    sl, nh, nkv, hd = 5, 4, 2, 8
    for causal, L in ((True, 5), (False, 9)):
        q = rng.standard_normal((sl if causal else 1, nh, hd)).astype(np.float32)
        kc = rng.standard_normal((nkv, L, hd)).astype(np.float32)
        vc = rng.standard_normal((nkv, L, hd)).astype(np.float32)
        got = oracle.attention(q, kc, vc, 0.125, causal)
        s = q.shape[0]
        qt = oracle.transpose(q[None], 1, 2)                        # [1, nh, s, hd]
        kw = oracle.repeat_interleave(kc[None], nh // nkv, 1)       # [1, nh, L, hd]
        vw = oracle.repeat_interleave(vc[None], nh // nkv, 1)
        mm = oracle.matmul(qt, oracle.transpose(kw, 2, 3))
        sc = oracle.scale(mm, 0.125)
        if causal:
            sc = oracle.binop("add", sc, oracle.causal_mask(s).reshape(1, 1, s, s))
        sm = oracle.softmax(sc, 3)
        ao = oracle.transpose(oracle.matmul(sm, vw), 1, 2).reshape(s, nh * hd)
        assert np.array_equal(got, ao)


def test_fused_add_relu_pins():
    # known answer of the reference (tl_cuda new_ops_comprehensive_test.rs:624-632)
    a = np.array([-1.0, 2.0, -3.0, 4.0], np.float32)
    b = np.array([0.5, -3.0, 5.0, -1.0], np.float32)
    np.testing.assert_array_equal(oracle.fused_add_relu(a, b), [0.0, 0.0, 2.0, 3.0])
    # f32::max(NaN, 0) is 0
    assert oracle.fused_add_relu(np.array([np.nan], np.float32), np.array([1.0], np.float32))[0] == 0.0


def test_fused_bias_gelu_pins():
    # gelu(0 + 0) = 0 (new_ops_comprehensive_test.rs:687-693)
    np.testing.assert_array_equal(oracle.fused_bias_gelu(np.zeros((2, 2), np.float32), np.zeros(2, np.float32)), 0)
    # signs at +-1.1 (tl_metal fused_ops_test.rs:60-75)
    y = oracle.fused_bias_gelu(np.array([1.0, -1.0], np.float32), np.array([0.1, -0.1], np.float32))
    assert y[0] > 0.9 and y[1] < 0.0
    # limits: gelu(v) -> v for large v, -> 0 for very negative v
    np.testing.assert_allclose(oracle.fused_bias_gelu(np.array([20.0, -20.0], np.float32), np.zeros(1, np.float32)),
                               [20.0, 0.0], atol=1e-6)
    # bias broadcast i % len(bias): the same as adding the tiled bias first
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 7)).astype(np.float32)
    bias = rng.standard_normal(7).astype(np.float32)
    np.testing.assert_array_equal(oracle.fused_bias_gelu(x, bias),
                                  oracle.fused_bias_gelu((x + bias).astype(np.float32), np.zeros(1, np.float32)))
    # the reference's constant is 2/sqrt(pi): gelu(1) = 0.5 (1 + tanh(2/sqrt(pi) 1.044715)),
    # not the textbook sqrt(2/pi) value 0.8412
    g1 = oracle.fused_bias_gelu(np.array([1.0], np.float32), np.zeros(1, np.float32))[0]
    assert abs(g1 - 0.5 * (1 + np.tanh(2 / np.sqrt(np.pi) * 1.044715))) < 1e-6
    assert abs(g1 - 0.8412) > 0.05


def _rotary_replay(x, f, hd):
    # the reference loop (tl_cpu fused_ops.rs:87-108), element by element in float64
    half, out = hd // 2, np.zeros(x.size, np.float64)
    for i in range(x.size // 2):
        p = i % half
        base = i - p
        c, s = np.cos(np.float64(f[p])), np.sin(np.float64(f[p]))
        x0, x1 = float(x[base + p]), float(x[base + p + half])
        out[base + p] = x0 * c - x1 * s
        out[base + p + half] = x0 * s + x1 * c
    return out


def test_fused_rotary_emb_pins():
    rng = np.random.default_rng(6)
    hd = 8
    x = rng.standard_normal(hd).astype(np.float32)
    f = rng.uniform(-3, 3, hd // 2).astype(np.float32)
    y = oracle.fused_rotary_emb(x, f, hd)
    # one head vector: each (x_p, x_{p+half}) pair rotated, norms kept
    np.testing.assert_allclose(y[:4] ** 2 + y[4:] ** 2, x[:4] ** 2 + x[4:] ** 2, rtol=1e-5)
    np.testing.assert_array_equal(oracle.fused_rotary_emb(x, np.zeros(4, np.float32), hd), x)
    q = oracle.fused_rotary_emb(x, np.full(4, np.pi / 2, np.float32), hd)
    np.testing.assert_allclose(q, np.concatenate([-x[4:], x[:4]]), atol=1e-6)
    # several vectors: the reference loop replayed (pairs of consecutive vectors overlap)
    x3 = rng.standard_normal(3 * hd + 4).astype(np.float32)
    np.testing.assert_allclose(oracle.fused_rotary_emb(x3, f, hd), _rotary_replay(x3, f, hd), rtol=2e-6, atol=2e-6)
