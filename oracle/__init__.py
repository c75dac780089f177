"""numpy bindings of the CPU oracle (libtl_oracle.so, built from tl_cpu_oracle.c and
tl_llama_oracle.c by oracle/Makefile).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU
baseline leg as the checker.  The product (tl_amd) never imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtl_oracle.so")

_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_i64p = C.POINTER(C.c_int64)
_i64, _f32, _f64, _int = C.c_int64, C.c_float, C.c_double, C.c_int

_PROTOS = {
    "tlo_f16_to_f32": (_f32, [C.c_uint16]),
    "tlo_dequantize_f16": (_int, [_u8p, _i64, _f32p]),
    "tlo_dequantize_q4_0": (_int, [_u8p, _i64, _i64, _f32p]),
    "tlo_dequantize_q8_0": (_int, [_u8p, _i64, _i64, _f32p]),
    "tlo_dequantize_q4_k": (_int, [_u8p, _i64, _i64, _f32p]),
    "tlo_dequantize_q6_k": (_int, [_u8p, _i64, _i64, _f32p]),
    "tlo_transpose_2d": (None, [_f32p, _i64, _i64, _f32p]),
    "tlo_transpose": (_int, [_f32p, _i64p, _int, _int, _int, _f32p]),
    "tlo_matmul": (_int, [_f32p, _i64p, _int, _f32p, _i64p, _int, _f32p]),
    "tlo_matmul_fast": (None, [_f32p, _f32p, _f32p, _i64, _i64, _i64]),
    "tlo_qtensor_matmul": (_int, [_f32p, _i64, _i64, _u8p, _i64, _int, _i64, _f32p, _int]),
    "tlo_rms_norm": (None, [_f32p, _i64, _i64, _f32p, _f32, _f32p]),
    "tlo_fused_rms_norm": (None, [_f32p, _i64, _i64, _f32p, _f32, _f32p]),
    "tlo_fused_add_rms_norm": (None, [_f32p, _f32p, _i64, _i64, _f32p, _f32, _f32p]),
    "tlo_rope_new_cos": (None, [_i64, _i64, _f32, _f32p]),
    "tlo_rope_new_sin": (None, [_i64, _i64, _f32, _f32p]),
    "tlo_apply_rope": (None, [_f32p, _i64, _i64, _f32p, _i64, _f32p, _i64, _f32p]),
    "tlo_silu": (None, [_f32p, _i64, _f32p]),
    "tlo_fused_silu_mul": (None, [_f32p, _f32p, _i64, _f32p]),
    "tlo_fused_rotary_emb": (None, [_f32p, _i64, _f32p, _i64, _f32p]),
    "tlo_fused_add_relu": (None, [_f32p, _f32p, _i64, _f32p]),
    "tlo_fused_bias_gelu": (None, [_f32p, _i64, _f32p, _i64, _f32p]),
    "tlo_binop": (_int, [_int, _f32p, _i64p, _int, _f32p, _i64p, _int, _f32p, _i64p]),
    "tlo_scale": (None, [_f32p, _i64, _f64, _f32p]),
    "tlo_softmax": (_int, [_f32p, _i64p, _int, _int, _f32p]),
    "tlo_causal_mask": (None, [_i64, _f32p]),
    "tlo_repeat_interleave": (_int, [_f32p, _i64p, _int, _i64, _int, _f32p]),
    "tlo_cat": (_int, [_f32p, _i64p, _f32p, _i64p, _int, _int, _f32p]),
    "tlo_narrow": (_int, [_f32p, _i64p, _int, _int, _i64, _i64, _f32p]),
    "tlo_embedding": (_int, [_f32p, _i64, _i64, _f32p, _i64, _f32p]),
    "tlo_argmax_last": (_i64, [_f32p, _i64]),
    "tlo_sample": (_i64, [_f32p, _i64, _f32, _f32, _f64]),
    "tlo_repetition_penalty": (None, [_f32p, _i64, _i64, _f32p, _i64, _f64, _f32p]),
    "tlo_sdpa": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _i64, _f32p]),
    "tlo_attention": (_int, [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64, _f32, _int, _f32p]),
    "tlo_llama_new": (C.c_void_p, [_int, _int, _int, _int, _int, _int, _f32, _f32, _int]),
    "tlo_llama_free": (None, [C.c_void_p]),
    "tlo_llama_set_linear": (_int, [C.c_void_p, _int, _int, _u8p, _i64, _int, _i64, _i64]),
    "tlo_llama_set_norm": (_int, [C.c_void_p, _int, _int, _f32p]),
    "tlo_llama_set_embedding": (_int, [C.c_void_p, _f32p]),
    "tlo_llama_reset": (None, [C.c_void_p]),
    "tlo_llama_forward": (_int, [C.c_void_p, _f32p, _i64, _f32p]),
}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return a.ctypes.data_as(_f32p)


def _shape(s):
    return (C.c_int64 * max(1, len(s)))(*[int(v) for v in s])


class OracleError(RuntimeError):
    pass


def _rc(rc, what):
    if rc != 0:
        raise OracleError(f"{what}: error {rc}")


def f16_to_f32(h):
    return lib().tlo_f16_to_f32(int(h))


def dequantize(ggml_type, data, numel):
    d = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
    out = np.empty(max(numel, 1), dtype=np.float32)
    if ggml_type == 2:
        rc = lib().tlo_dequantize_q4_0(d.ctypes.data_as(_u8p), d.size, numel, _p(out))
    elif ggml_type == 8:
        rc = lib().tlo_dequantize_q8_0(d.ctypes.data_as(_u8p), d.size, numel, _p(out))
    elif ggml_type == 12:
        rc = lib().tlo_dequantize_q4_k(d.ctypes.data_as(_u8p), d.size, numel, _p(out))
    elif ggml_type == 14:
        rc = lib().tlo_dequantize_q6_k(d.ctypes.data_as(_u8p), d.size, numel, _p(out))
    elif ggml_type == 1:
        rc = lib().tlo_dequantize_f16(d.ctypes.data_as(_u8p), d.size, _p(out))
    else:
        raise OracleError("unsupported type")
    _rc(rc, "dequantize")
    return out[:numel]


def matmul(a, b):
    a, b = _f(a), _f(b)
    m = a.shape[-2] if a.ndim >= 2 else 1
    n = b.shape[-1] if b.ndim >= 2 else 1
    shape = list(a.shape[:-2]) + [m] + ([n] if b.ndim >= 2 else [])
    out = np.empty(int(np.prod(shape)) or 1, dtype=np.float32)
    _rc(lib().tlo_matmul(_p(a), _shape(a.shape), a.ndim, _p(b), _shape(b.shape), b.ndim, _p(out)), "matmul")
    return out[:int(np.prod(shape))].reshape(shape)


def matmul_fast(a, b):
    a, b = _f(a), _f(b)
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), dtype=np.float32)
    lib().tlo_matmul_fast(_p(a), _p(b), _p(out), m, k, n)
    return out


def qtensor_matmul(x, wbytes, ggml_type, n, fast=True):
    x = _f(x)
    m, k = (1, x.shape[0]) if x.ndim == 1 else (int(np.prod(x.shape[:-1])), x.shape[-1])
    w = np.ascontiguousarray(np.frombuffer(bytes(wbytes), dtype=np.uint8))
    y = np.empty((m, n), dtype=np.float32)
    _rc(lib().tlo_qtensor_matmul(_p(x), m, k, w.ctypes.data_as(_u8p), w.size, ggml_type, n, _p(y), int(fast)),
        "qtensor_matmul")
    return y


def rms_norm(x, w, eps):
    x = _f(x)
    n = x.shape[-1]
    out = np.empty_like(x)
    wp = _p(_f(w)) if w is not None else None
    ww = _f(w) if w is not None else None
    lib().tlo_rms_norm(_p(x), x.size // n, n, _p(ww) if ww is not None else wp, eps, _p(out))
    return out


def fused_rms_norm(x, w, eps):
    x, w = _f(x), _f(w)
    n = x.shape[-1]
    out = np.empty_like(x)
    lib().tlo_fused_rms_norm(_p(x), x.size // n, n, _p(w), eps, _p(out))
    return out


def fused_add_rms_norm(x, r, w, eps):
    x, r, w = _f(x), _f(r), _f(w)
    n = x.shape[-1]
    out = np.empty_like(x)
    lib().tlo_fused_add_rms_norm(_p(x), _p(r), x.size // n, n, _p(w), eps, _p(out))
    return out


def rope_table(seq_len, dim, base, sin=False):
    out = np.empty((seq_len, dim), dtype=np.float32)
    (lib().tlo_rope_new_sin if sin else lib().tlo_rope_new_cos)(seq_len, dim, base, _p(out))
    return out


def apply_rope(x, cos_t, sin_t):
    x, c, s = _f(x), _f(cos_t), _f(sin_t)
    out = np.empty_like(x)
    lib().tlo_apply_rope(_p(x), x.size, x.shape[-1], _p(c), c.size, _p(s), s.size, _p(out))
    return out


def silu(x):
    x = _f(x)
    out = np.empty_like(x)
    lib().tlo_silu(_p(x), x.size, _p(out))
    return out


def fused_silu_mul(g, u):
    g, u = _f(g), _f(u)
    out = np.empty_like(g)
    lib().tlo_fused_silu_mul(_p(g), _p(u), g.size, _p(out))
    return out


def fused_rotary_emb(x, freqs, head_dim):
    """tl_cpu fused_rotary_emb (fused_ops.rs:87-108): half-split pairs, cos / sin of freqs."""
    x, freqs = _f(x), _f(freqs)
    out = np.empty_like(x)
    lib().tlo_fused_rotary_emb(_p(x), x.size, _p(freqs), int(head_dim), _p(out))
    return out


def fused_add_relu(a, b):
    a, b = _f(a), _f(b)
    out = np.empty_like(a)
    lib().tlo_fused_add_relu(_p(a), _p(b), a.size, _p(out))
    return out


def fused_bias_gelu(x, bias):
    x, bias = _f(x), _f(bias)
    out = np.empty_like(x)
    lib().tlo_fused_bias_gelu(_p(x), x.size, _p(bias), bias.size, _p(out))
    return out


def binop(op, a, b):
    a, b = _f(a), _f(b)
    nd = max(a.ndim, b.ndim)
    oshape = np.broadcast_shapes(a.shape, b.shape)
    out = np.empty(max(1, int(np.prod(oshape))), dtype=np.float32)
    os_ = (C.c_int64 * max(1, nd))()
    r = lib().tlo_binop({"add": 0, "mul": 1, "sub": 2, "div": 3}[op], _p(a), _shape(a.shape), a.ndim, _p(b),
                        _shape(b.shape), b.ndim, _p(out), os_)
    if r < 0:
        raise OracleError(f"binop: error {r}")
    return out[:int(np.prod(oshape))].reshape(oshape)


def scale(x, s):
    x = _f(x)
    out = np.empty_like(x)
    lib().tlo_scale(_p(x), x.size, s, _p(out))
    return out


def softmax(x, axis):
    x = _f(x)
    out = np.empty_like(x)
    _rc(lib().tlo_softmax(_p(x), _shape(x.shape), x.ndim, axis, _p(out)), "softmax")
    return out


def causal_mask(size):
    out = np.empty((size, size), dtype=np.float32)
    lib().tlo_causal_mask(size, _p(out))
    return out


def transpose(x, d0, d1):
    x = _f(x)
    shape = list(x.shape)
    shape[d0], shape[d1] = shape[d1], shape[d0]
    out = np.empty(shape, dtype=np.float32)
    _rc(lib().tlo_transpose(_p(x), _shape(x.shape), x.ndim, d0, d1, _p(out)), "transpose")
    return out


def repeat_interleave(x, repeats, axis):
    x = _f(x)
    shape = list(x.shape)
    shape[axis] *= repeats
    out = np.empty(shape, dtype=np.float32)
    _rc(lib().tlo_repeat_interleave(_p(x), _shape(x.shape), x.ndim, repeats, axis, _p(out)), "repeat_interleave")
    return out


def cat(a, b, axis):
    a, b = _f(a), _f(b)
    shape = list(a.shape)
    shape[axis] += b.shape[axis]
    out = np.empty(shape, dtype=np.float32)
    _rc(lib().tlo_cat(_p(a), _shape(a.shape), _p(b), _shape(b.shape), a.ndim, axis, _p(out)), "cat")
    return out


def narrow(x, axis, start, length):
    x = _f(x)
    shape = list(x.shape)
    shape[axis] = length
    out = np.empty(shape, dtype=np.float32)
    _rc(lib().tlo_narrow(_p(x), _shape(x.shape), x.ndim, axis, start, length, _p(out)), "narrow")
    return out


def embedding(table, ids):
    table, ids = _f(table), _f(ids)
    out = np.empty(tuple(ids.shape) + (table.shape[1],), dtype=np.float32)
    _rc(lib().tlo_embedding(_p(table), table.shape[0], table.shape[1], _p(ids), ids.size, _p(out)), "embedding")
    return out


def argmax_last(x):
    x = _f(x)
    return int(lib().tlo_argmax_last(_p(x), x.size))


def sample(x, temp, top_p, u):
    """sample_impl over all elements of x with the uniform draw u (-1 for an empty input)."""
    x = _f(x)
    return int(lib().tlo_sample(_p(x), x.size, temp, top_p, u))


def repetition_penalty(logits, tokens, penalty):
    lg, tk = _f(logits), _f(tokens)
    vocab = lg.shape[-1]
    out = np.empty_like(lg)
    lib().tlo_repetition_penalty(_p(lg), lg.size // vocab, vocab, _p(tk), tk.size, penalty, _p(out))
    return out


def attention(q, kc, vc, scale_, causal):
    """q [sl, nh, hd]; kc, vc [nkv, L, hd] -> [sl, nh*hd] (chatbot attention composition)."""
    q, kc, vc = _f(q), _f(kc), _f(vc)
    sl, nh, hd = q.shape
    nkv, L, _ = kc.shape
    out = np.empty((sl, nh * hd), dtype=np.float32)
    _rc(lib().tlo_attention(_p(q), _p(kc), _p(vc), sl, nh, nkv, hd, L, scale_, int(causal), _p(out)), "attention")
    return out


# Linear weights of one decoder block in slot order: Attention::from_map q, k, v, output and
# MLP::from_map gate, up, down (chatbot.tl:23-26, 43-47); slot 7 stands for the LM head
# "output.weight" (chatbot.tl:154).
LINEAR_SLOTS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")

GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 2, 8, 12, 14


def linear_shape(cfg, name):
    """Row-major [n, k] of a linear weight (gguf.rs:129-136 order) for the chatbot's model:
    q / output [D, D], k / v [Hkv hd, D] (the reshape to [1, sl, 4, 64], chatbot.tl:53-54),
    gate / up [F, D], down [D, F], LM head [vocab, D]."""
    D, F = cfg.d_model, cfg.ffn_dim
    kvd = cfg.n_kv_heads * (D // cfg.n_heads)
    return {"attn_q": (D, D), "attn_k": (kvd, D), "attn_v": (kvd, D), "attn_output": (D, D),
            "ffn_gate": (F, D), "ffn_up": (F, D), "ffn_down": (D, F), "output": (cfg.vocab, D)}[name]


def q4_k_m_type(n_layers, layer, name):
    """GGML type of a linear weight in a llama.cpp "Q4_K_M" file -- the third-party rule
    (llama.cpp llama_tensor_get_type, not part of the reference) that decides the type mixture of
    the chatbot's own checkpoint (chatbot.tl:119): output.weight (layer -1) Q6_K; attn_v and
    ffn_down Q6_K in the layers where use_more_bits(i, n) holds, i.e. i < n/8, i >= 7n/8 or
    (i - n/8) % 3 == 2 (integer division); every other linear Q4_K."""
    if layer < 0:
        return GGML_Q6_K
    more = layer < n_layers // 8 or layer >= 7 * n_layers // 8 or (layer - n_layers // 8) % 3 == 2
    if name in ("attn_v", "ffn_down") and more:
        return GGML_Q6_K
    return GGML_Q4_K


def weight_type(plan, cfg, layer, name):
    """GGML type of one linear weight under a type plan: an int for every linear, "Q4_K_M" for
    q4_k_m_type, or a callable (cfg, layer, name)."""
    if callable(plan):
        return int(plan(cfg, layer, name))
    if plan == "Q4_K_M":
        return q4_k_m_type(cfg.n_layers, layer, name)
    return int(plan)


def sdpa(q, k, v, mask=None):
    """IDevice::tensor_scaled_dot_product_attention on tl_cpu (device_impl.rs:775-872): q [.., sq, dk]
    (rank 2-4), k [.., sk, dk], v [.., sk, dv] with the same leading dims; mask == 0 -> -1e9."""
    q, k, v = _f(q), _f(k), _f(v)
    sq, dk = q.shape[-2], q.shape[-1]
    sk, dv = k.shape[-2], v.shape[-1]
    slices = int(np.prod(q.shape[:-2])) if q.ndim > 2 else 1
    out = np.empty(tuple(q.shape[:-2]) + (sq, dv), dtype=np.float32)
    m = _f(mask) if mask is not None else None
    lib().tlo_sdpa(_p(q), _p(k), _p(v), _p(m) if m is not None else None, m.size if m is not None else 0,
                   slices, sq, sk, dk, dv, _p(out))
    return out


class Llama:
    """The chatbot.tl decoder on the CPU oracle (bit-identical to the tl_cpu op chain)."""

    def __init__(self, cfg):
        self.cfg = cfg
        self.h = lib().tlo_llama_new(cfg.n_layers, cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.ffn_dim,
                                     cfg.vocab, cfg.eps, cfg.rope_theta, cfg.max_seq)
        if not self.h:
            raise OracleError("tlo_llama_new failed")

    def load(self, tensors, ggml_type=GGML_Q4_0):
        """tensors: (kind, layer, which, payload) with kind "embedding" / "norm" / "linear";
        a linear's payload is its GGUF block bytes, typed by the plan `ggml_type`."""
        cfg = self.cfg
        for kind, layer, which, payload in tensors:
            if kind == "embedding":
                p = _f(payload)
                _rc(lib().tlo_llama_set_embedding(self.h, _p(p)), "set_embedding")
            elif kind == "norm":
                p = _f(payload)
                _rc(lib().tlo_llama_set_norm(self.h, layer, which, _p(p)), "set_norm")
            else:
                name = LINEAR_SLOTS[which] if layer >= 0 else "output"
                n, k = linear_shape(cfg, name)
                p = np.ascontiguousarray(payload, dtype=np.uint8)
                t = weight_type(ggml_type, cfg, layer, name)
                _rc(lib().tlo_llama_set_linear(self.h, layer, which, p.ctypes.data_as(_u8p), p.size, t, n, k),
                    "set_linear")

    def reset(self):
        lib().tlo_llama_reset(self.h)

    def forward(self, ids):
        ids = _f(np.asarray(ids, dtype=np.float32))
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        _rc(lib().tlo_llama_forward(self.h, _p(ids), ids.size, _p(out)), "llama_forward")
        return out

    def greedy(self, prompt, n_tokens, penalty=1.0):
        """chatbot.tl:174-222 with sample(temp <= 0); returns the generated ids."""
        self.reset()
        toks = [int(t) for t in prompt]
        cur = list(toks)
        out = []
        for _ in range(n_tokens):
            logits = self.forward(cur)
            if penalty != 1.0:
                logits = repetition_penalty(logits[None, :], np.array(toks, dtype=np.float32), penalty)[0]
            nxt = argmax_last(logits)
            out.append(nxt)
            toks.append(nxt)
            cur = [nxt]
        return np.array(out, dtype=np.int32)

    def close(self):
        if self.h:
            lib().tlo_llama_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
