"""Pins the oracle's whole-model composition (tlo_llama_forward, oracle/tl_llama_oracle.c)
against a literal replay of the reference chatbot's op chain, and its remaining small
functions (fused_silu_mul, binop sub / div, the Q4_K_M type plan).  CPU only.

The replay issues the tl_cpu ops one by one, in the order and with the arguments
examples/apps/tinyllama/chatbot.tl writes them (Linear / RMSNorm / MLP / Attention / Block at
10-112, the decode loop at 174-190), each op through the oracle function that restates it and
that tests/test_oracle.py pins on its own.  The quantized linear is the TL_DEVICE=cpu route of
tl_qtensor_matmul (dequantize, transpose, matmul_impl: system.rs:193-222) with the faithful
matmul loop order.  The direct form in tlo_llama_forward (cached transposed weights, threaded
matmul, fused attention loop, KV cache written in place, LM head on the last row only) must
give the same bits at every step.
"""
import numpy as np
import pytest

import oracle
from tl_amd.quant import quantize_q4_0, quantize_q4_k, quantize_q6_k, quantize_q8_0


class _Cfg:
    def __init__(self, n_layers, d_model, n_heads, n_kv_heads, ffn_dim, vocab, max_seq):
        self.n_layers, self.d_model, self.n_heads, self.n_kv_heads = n_layers, d_model, n_heads, n_kv_heads
        self.ffn_dim, self.vocab, self.max_seq = ffn_dim, vocab, max_seq
        self.eps, self.rope_theta = 1e-5, 10000.0


_ENC = {2: quantize_q4_0, 8: quantize_q8_0, 12: quantize_q4_k, 14: quantize_q6_k}


def _toy_model(cfg, plan, seed):
    """(kind, layer, which, payload) tuples of a random model; head_dim 64 as the chatbot's
    hard-coded scale 0.125 = 1/sqrt(64) assumes (chatbot.tl:78, 83)."""
    rng = np.random.default_rng(seed)
    out = [("embedding", -1, 0, rng.standard_normal((cfg.vocab, cfg.d_model)).astype(np.float32))]
    for layer in range(cfg.n_layers):
        for which, name in enumerate(oracle.LINEAR_SLOTS):
            n, k = oracle.linear_shape(cfg, name)
            w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
            out.append(("linear", layer, which, _ENC[oracle.weight_type(plan, cfg, layer, name)](w)))
        for which in (0, 1):
            out.append(("norm", layer, which, rng.uniform(0.5, 1.5, cfg.d_model).astype(np.float32)))
    out.append(("norm", -1, 0, rng.uniform(0.5, 1.5, cfg.d_model).astype(np.float32)))
    n, k = oracle.linear_shape(cfg, "output")
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    out.append(("linear", -1, 0, _ENC[oracle.weight_type(plan, cfg, -1, "output")](w)))
    return out


class _LiteralChatbot:
    """chatbot.tl's model, one tl_cpu op per line of the program."""

    def __init__(self, cfg, tensors, plan):
        self.cfg = cfg
        self.lin, self.norm = {}, {}
        for kind, layer, which, payload in tensors:
            if kind == "embedding":
                self.emb = payload
            elif kind == "norm":
                self.norm[(layer, which)] = payload
            else:
                name = oracle.LINEAR_SLOTS[which] if layer >= 0 else "output"
                self.lin[(layer, which)] = (payload, oracle.weight_type(plan, cfg, layer, name),
                                            oracle.linear_shape(cfg, name)[0])
        hd = cfg.d_model // cfg.n_heads
        # chatbot.tl:151-152 Tensor::rope_new_cos(64, 2048, 10000.0): [seq_len, dim]
        self.cos = oracle.rope_table(cfg.max_seq, hd, cfg.rope_theta)
        self.sin = oracle.rope_table(cfg.max_seq, hd, cfg.rope_theta, sin=True)
        self.cache = {}

    def linear(self, layer, which, x):
        # Linear::forward: x.matmul_quantized(w) -> tl_qtensor_matmul, CPU route (chatbot.tl:12-14)
        w, t, n = self.lin[(layer, which)]
        return oracle.qtensor_matmul(x, w, t, n, fast=False)

    def rmsnorm(self, layer, which, x):
        # RMSNorm::forward: x.rms_norm(w, 0.00001) (chatbot.tl:17-19)
        return oracle.rms_norm(x, self.norm[(layer, which)], np.float32(0.00001))

    def attention(self, li, x, sl, sp):
        c = self.cfg
        H, KV, hd = c.n_heads, c.n_kv_heads, c.d_model // c.n_heads
        q_4d = self.linear(li, 0, x).reshape(1, sl, H, hd)                # chatbot.tl:52
        k_4d = self.linear(li, 1, x).reshape(1, sl, KV, hd)               # :53
        v_4d = self.linear(li, 2, x).reshape(1, sl, KV, hd)               # :54
        cs = oracle.narrow(self.cos, 0, sp, sl)                           # :56
        ss = oracle.narrow(self.sin, 0, sp, sl)                           # :57
        qr = oracle.apply_rope(q_4d, cs, ss)                              # :60
        kr = oracle.apply_rope(k_4d, cs, ss)                              # :61
        kt = oracle.transpose(kr, 1, 2)                                   # :63
        vt = oracle.transpose(v_4d, 1, 2)                                 # :64
        k_tot = kt if sp == 0 else oracle.cat(self.cache[li][0], kt, 2)   # :66
        v_tot = vt if sp == 0 else oracle.cat(self.cache[li][1], vt, 2)   # :67
        self.cache[li] = (k_tot, v_tot)                                   # :69
        qt = oracle.transpose(qr, 1, 2)                                   # :71
        kw = oracle.repeat_interleave(k_tot, H // KV, 1)                  # :73
        vw = oracle.repeat_interleave(v_tot, H // KV, 1)                  # :74
        mm = oracle.matmul(qt, oracle.transpose(kw, 2, 3))                # :77 / :82
        sm = oracle.scale(mm, 0.125)                                      # :78 / :83
        if sl > 1:
            mask = oracle.causal_mask(sl).reshape(1, 1, sl, sl)           # :79
            sm = oracle.binop("add", sm, mask)                            # :80
        sm_soft = oracle.softmax(sm, 3)                                   # :86
        ao = oracle.transpose(oracle.matmul(sm_soft, vw), 1, 2)           # :87
        return self.linear(li, 3, ao.reshape(sl, c.d_model))              # :89

    def mlp(self, li, x):
        gx = self.linear(li, 4, x)                                        # chatbot.tl:34
        sx = oracle.silu(gx)                                              # :35
        ux = self.linear(li, 5, x)                                        # :36
        mu = oracle.binop("mul", sx, ux)                                  # :37
        return self.linear(li, 6, mu)                                     # :38

    def block(self, li, x, sl, sp):
        attn_out = self.attention(li, self.rmsnorm(li, 0, x), sl, sp)     # chatbot.tl:108
        x2 = oracle.binop("add", x, attn_out)                             # :109
        ffn_out = self.mlp(li, self.rmsnorm(li, 1, x2))                   # :110
        return oracle.binop("add", x2, ffn_out)                           # :111

    def step(self, tokens, cur_tokens, penalty):
        """One pass of the decode loop body (chatbot.tl:175-190) with sample(temp <= 0);
        returns (logits row the sample reads, chosen id)."""
        total_len, batch_len = len(tokens), len(cur_tokens)
        start_pos = total_len - batch_len                                 # :175-177
        x = oracle.embedding(self.emb, np.asarray(cur_tokens, np.float32))  # :178
        for l in range(self.cfg.n_layers):                                # :181-185
            x = self.block(l, x, batch_len, start_pos)
        lo = self.linear(-1, 0, self.rmsnorm(-1, 0, x))                   # :186
        if penalty != 1.0:                                                # :188
            lo = oracle.repetition_penalty(lo, np.asarray(tokens, np.float32), penalty)
        row = oracle.narrow(lo, 0, batch_len - 1, 1)                      # :189
        return row[0], oracle.argmax_last(row)


@pytest.mark.parametrize("plan,penalty", [(2, 1.0), (2, 1.1), ("Q4_K_M", 1.1), (8, 1.0)])
def test_llama_forward_equals_literal_chatbot_chain(plan, penalty):
    """Prefill at start position 0 (causal mask) plus three decode steps: logits and greedy
    ids of tlo_llama_forward bit-equal to the literal op chain, with and without the
    chatbot's repetition penalty 1.1."""
    d_model = 256 if plan == "Q4_K_M" else 128   # K-quant rows hold whole 256-weight blocks
    cfg = _Cfg(2, d_model, d_model // 64, 1 if plan == 2 else 2, 2 * d_model if plan == "Q4_K_M" else 160,
               96, 32)
    tensors = _toy_model(cfg, plan, seed=11)
    lit = _LiteralChatbot(cfg, tensors, plan)
    model = oracle.Llama(cfg)
    model.load(tensors, ggml_type=plan)
    try:
        prompt = list(np.random.default_rng(12).integers(0, cfg.vocab, 6))
        tokens, cur = list(prompt), list(prompt)
        model.reset()
        for step in range(4):
            want_row, want_id = lit.step(tokens, cur, penalty)
            got = model.forward(cur)
            if penalty != 1.0:
                got = oracle.repetition_penalty(got[None, :], np.asarray(tokens, np.float32), penalty)[0]
            assert np.array_equal(got.view(np.uint32), want_row.view(np.uint32)), f"logits differ at step {step}"
            assert oracle.argmax_last(got) == want_id
            tokens.append(want_id)
            cur = [want_id]
        # the same ids from the oracle's own greedy loop (the golden-token generator)
        assert list(model.greedy(prompt, 4, penalty)) == tokens[len(prompt):]
    finally:
        model.close()


def test_literal_chain_first_layer_by_hand():
    """The replay itself, checked in float64 for one token at position 0: embedding row,
    RMSNorm, and a single-token attention whose softmax over one position is 1 (so the
    attention output is the v projection, repeated per query head) -- a closed form of
    chatbot.tl:52-89 at sl = 1, sp = 0."""
    cfg = _Cfg(1, 128, 2, 1, 160, 40, 8)
    tensors = _toy_model(cfg, 2, seed=3)
    lit = _LiteralChatbot(cfg, tensors, 2)
    x = lit.emb[[5]].astype(np.float64)
    h = x / np.sqrt((x * x).mean() + 1e-5) * lit.norm[(0, 0)]
    W = {w: oracle.dequantize(2, lit.lin[(0, w)][0], lit.lin[(0, w)][2] * cfg.d_model).reshape(-1, cfg.d_model)
         for w in (2, 3)}
    v = h @ W[2].T.astype(np.float64)                      # [1, 64]: one KV head
    ao = np.concatenate([v, v], axis=1)                    # two query heads read KV head 0
    want = ao @ W[3].T.astype(np.float64)
    got = lit.attention(0, lit.rmsnorm(0, 0, lit.emb[[5]]), 1, 0)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_fused_silu_mul_pins():
    # known answers of the reference (tl_cuda new_ops_comprehensive_test.rs:635-645)
    v = oracle.fused_silu_mul(np.array([0.0, 1.0, -1.0, 2.0], np.float32), np.ones(4, np.float32))
    assert abs(v[0]) < 1e-5 and abs(v[1] - 0.7311) < 1e-3
    # fused vs unfused silu(gate) * up within 1e-4 (tl_metal fused_ops_test.rs:42-56)
    g = np.array([1.0, -1.0, 2.0, 0.0], np.float32)
    u = np.array([2.0, 3.0, 1.0, 5.0], np.float32)
    np.testing.assert_allclose(oracle.fused_silu_mul(g, u), oracle.binop("mul", oracle.silu(g), u), atol=1e-4)
    # float64 closed form g / (1 + e^-g) * u over a wide range, and the tl_cpu order of
    # operations g / (1 + exp(-g)) then * u (fused_ops.rs:15-17, 28-30) restated in numpy f32
    rng = np.random.default_rng(21)
    g = (rng.standard_normal(4096) * 6).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    g64 = g.astype(np.float64)
    np.testing.assert_allclose(oracle.fused_silu_mul(g, u), g64 / (1 + np.exp(-g64)) * u, rtol=2e-6, atol=1e-30)
    e = np.exp(-g).astype(np.float32)            # numpy's f32 exp may differ from glibc expf by 1 ulp
    np.testing.assert_allclose(oracle.fused_silu_mul(g, u), (g / (np.float32(1) + e)) * u, rtol=3e-7, atol=1e-30)
    # exact special values: silu(0) = 0; large negative gate -> -0 or a tiny value; large positive -> g * u
    assert oracle.fused_silu_mul(np.array([0.0], np.float32), np.array([7.0], np.float32))[0] == 0.0
    assert oracle.fused_silu_mul(np.array([100.0], np.float32), np.array([3.0], np.float32))[0] == 300.0
    assert abs(oracle.fused_silu_mul(np.array([-100.0], np.float32), np.array([3.0], np.float32))[0]) < 1e-38


def test_binop_sub_div_match_numpy():
    # CpuTensor elementwise sub / div with broadcasting (tensor.rs:549-609): one IEEE op per
    # element, so numpy's float32 arithmetic is the same function
    rng = np.random.default_rng(22)
    a = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    for bshape in [(5,), (4, 1), (3, 1, 5), (2, 3, 4, 5), (1,)]:
        b = (rng.standard_normal(bshape) + 0.1).astype(np.float32)
        assert np.array_equal(oracle.binop("sub", a, b), a - b)
        assert np.array_equal(oracle.binop("div", a, b), a / b)
        assert np.array_equal(oracle.binop("sub", b, a), b - a)
        assert np.array_equal(oracle.binop("div", b, a), b / a)
    # division by zero and signed zeros follow IEEE
    z = oracle.binop("div", np.array([1.0, -1.0, 0.0], np.float32), np.zeros(3, np.float32))
    assert z[0] == np.inf and z[1] == -np.inf and np.isnan(z[2])
    assert np.signbit(oracle.binop("sub", np.zeros(1, np.float32), np.zeros(1, np.float32))[0]) == np.False_
    with pytest.raises((oracle.OracleError, ValueError)):
        oracle.binop("sub", a, np.ones((3,), np.float32))
    # the C restatement's own broadcast check (tensor.rs:568-577 ShapeMismatch)
    ash, bsh = (oracle.C.c_int64 * 2)(2, 5), (oracle.C.c_int64 * 1)(3)
    out, osh = np.empty(10, np.float32), (oracle.C.c_int64 * 2)()
    assert oracle.lib().tlo_binop(2, oracle._p(a.reshape(-1)[:10].copy()), ash, 2, oracle._p(np.ones(3, np.float32)),
                                  bsh, 1, oracle._p(out), osh) < 0


def test_q4_k_m_type_plan_for_tinyllama():
    # llama.cpp's use_more_bits for 22 layers: i < 2, i >= 19, or (i - 2) % 3 == 2
    more = {0, 1, 4, 7, 10, 13, 16, 19, 20, 21}
    for layer in range(22):
        for name in oracle.LINEAR_SLOTS:
            want = 14 if name in ("attn_v", "ffn_down") and layer in more else 12
            assert oracle.q4_k_m_type(22, layer, name) == want, (layer, name)
    assert oracle.q4_k_m_type(22, -1, "output") == 14
    # the 4-layer toy models of the GPU tests: i < 0 never, i >= 3, (i - 0) % 3 == 2
    assert [oracle.q4_k_m_type(4, i, "attn_v") for i in range(4)] == [12, 12, 14, 14]


def test_sdpa_with_causal_ones_mask_is_the_chatbot_chain():
    """tlo_sdpa (device_impl.rs:775-872) with a lower-triangular ones mask and one KV head per
    query head equals the chatbot's attention chain with the causal mask (pinned above, and
    against the literal op chain in test_oracle.py) bit for bit: the scale is 1/sqrt(64) =
    0.125 exactly, -1e9 and -inf both vanish in exp, and every sum runs in the same order."""
    rng = np.random.default_rng(31)
    sl, nh, hd = 7, 3, 64
    q = rng.standard_normal((sl, nh, hd)).astype(np.float32)
    kc = rng.standard_normal((nh, sl, hd)).astype(np.float32)
    vc = rng.standard_normal((nh, sl, hd)).astype(np.float32)
    chain = oracle.attention(q, kc, vc, 0.125, True).reshape(sl, nh, hd)
    mask = np.tril(np.ones((sl, sl), np.float32))
    got = oracle.sdpa(q.transpose(1, 0, 2), kc, vc, mask)
    assert np.array_equal(got.transpose(1, 0, 2).view(np.uint32), chain.view(np.uint32))


def _sdpa64(q, k, v, keep=None):
    s = q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2) / np.sqrt(q.shape[-1])
    if keep is not None:
        s = np.where(keep, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    return (p / p.sum(-1, keepdims=True)) @ v.astype(np.float64)


def test_sdpa_closed_forms_and_mask_rule():
    rng = np.random.default_rng(32)
    for shape_q, sk, dv in [((2, 3, 5, 16), 9, 24), ((4, 6, 32), 6, 32), ((5, 8), 11, 3)]:
        q = rng.standard_normal(shape_q).astype(np.float32)
        k = rng.standard_normal(shape_q[:-2] + (sk, shape_q[-1])).astype(np.float32)
        v = rng.standard_normal(shape_q[:-2] + (sk, dv)).astype(np.float32)
        out = oracle.sdpa(q, k, v)
        assert out.shape == shape_q[:-1] + (dv,)
        np.testing.assert_allclose(out, _sdpa64(q, k, v), rtol=1e-5, atol=1e-5)
        # mask == 0 drops a key (each row keeps at least one); other values change nothing
        sq = shape_q[-2]
        keep = rng.random((sq, sk)) > 0.4
        keep[:, 0] = True
        mask = np.where(keep, rng.choice([1.0, -np.inf, 5.0, np.nan], (sq, sk)), 0.0).astype(np.float32)
        np.testing.assert_allclose(oracle.sdpa(q, k, v, mask), _sdpa64(q, k, v, keep), rtol=1e-5, atol=1e-5)
        assert np.array_equal(oracle.sdpa(q, k, v, np.ones((sq, sk), np.float32)), out)
        # a fully masked row gives every key the same weight: the mean of V
        full = mask.copy()
        full[0] = 0.0
        got = oracle.sdpa(q, k, v, full)
        np.testing.assert_allclose(got[..., 0, :], v.astype(np.float64).mean(-2), rtol=1e-5, atol=1e-6)
        # a mask shorter than seq_q * seq_k masks only the entries it holds
        short = np.zeros(sk, np.float32)       # row 0 fully masked, the rest unmasked
        got = oracle.sdpa(q, k, v, short)
        np.testing.assert_allclose(got[..., 1:, :], out[..., 1:, :], rtol=0, atol=0)
    # one key: the output is that key's V row
    q = rng.standard_normal((2, 4, 8)).astype(np.float32)
    k = rng.standard_normal((2, 1, 8)).astype(np.float32)
    v = rng.standard_normal((2, 1, 5)).astype(np.float32)
    assert np.array_equal(oracle.sdpa(q, k, v), np.repeat(v, 4, axis=1))
