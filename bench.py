"""Benchmark of the tl_hip hot path on one MI355X.

Headline (BASELINE.json metric, configs[4]): greedy decode tokens/s at batch 1 of a
random-init TinyLlama-shape Q4_0 decoder (22 layers, d_model 2048, 32/4 heads, FFN 5632,
vocab 32000) after a 512-token prompt.  A step is one decoded token (the whole decoder + LM
head + argmax, replayed from hipGraphs that hold eight steps each); weights, KV cache and
activations are resident in HBM.

Roofline object: the dominant kernel of decode, the Q4_0 matvec, at the 4096 x 4096 shape of
algorithmic bytes per launch (9,437,184 B of blocks + 16 KiB x + 16 KiB y) over
the average launch duration, timed with HIP events on the launch stream while rotating over
36 distinct weight copies (341 MB > the 256 MB Infinity Cache), beside the one-launch read
floor of the same loads (tl_hip_read_floor).

CPU baseline: the oracle's restatement of the tl_cpu loops (matmul_impl order) on one pinned
host core: one decoder layer + the LM head at the same shapes, times 22 layers, plus the
configs[0]-[3] legs (cold / steady matvec, row ops, a sampled GEMM, the attention op chain).

Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import itertools
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MATVEC_N = MATVEC_K = 4096
MATVEC_BYTES = MATVEC_N * MATVEC_K // 32 * 18 + MATVEC_K * 4 + MATVEC_N * 4  # 9,469,952 (Q4_0)
HBM_PEAK_GBS = 8000.0
# HBM bytes per 4096 x 4096 matvec launch from the two counter runs of
# `bench.py --matvec-only` (FETCH_SIZE 4,711.01 KiB x 1.99895 + WRITE_SIZE 16.0 KiB x 1.0,
# the scale factors read off a 64 MiB device copy in the same runs): 1.0200 x the
# algorithmic bytes
MATVEC_TRAFFIC = 9_659_467


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def matvec_bytes(t, n=MATVEC_N, k=MATVEC_K):
    """Algorithmic bytes of one m = 1 matvec: the GGUF blocks + x + y (f32)."""
    per = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}[t]
    return n * k // per[0] * per[1] + k * 4 + n * 4


def bench_matvec(dev, t=2, launches=340, min_bytes=320 << 20, n=MATVEC_N, k=MATVEC_K, floor=False, blocks=1):
    """Average seconds of one n x k matvec (m = 1, default 4096 x 4096) of GGML type t,
    launched back to back over enough resident weight copies (>= 320 MB) that the 256 MB
    Infinity Cache cannot serve them.  floor=True times tl_hip_read_floor instead: the same
    launch shape and copies, reading the weight bytes and computing nothing.  blocks > 1:
    that many timed blocks of `launches` launches, each behind its own stall; returns the
    list of the blocks' per-launch averages."""
    import ctypes as C

    from tl_amd import QTensor
    from tl_amd.quant import random_q4_0_blocks, random_q4_k_blocks, random_q6_k_blocks, random_q8_0_blocks

    gen = {2: random_q4_0_blocks, 8: random_q8_0_blocks, 12: random_q4_k_blocks, 14: random_q6_k_blocks}[t]
    lib = dev.lib
    rng = np.random.default_rng(0x71510000)
    raw = gen(rng, n, k)
    copies = -(-min_bytes // raw.nbytes)
    ws = [QTensor(t, raw, (n, k)) for _ in range(copies)]
    hs = [w.upload(lib) for w in ws]
    x = dev.tensor_new(rng.standard_normal((1, k)).astype(np.float32))
    y = dev.tensor_zeros((1, n))
    stream = lib.tl_hip_stream()
    xp, yp = C.c_void_p(x.data_ptr), C.c_void_p(y.data_ptr)

    def launch(i):
        if floor:
            return lib.tl_hip_read_floor(hs[i % copies], stream)
        return lib.tl_hip_launch_quant_matvec(hs[i % copies], xp, yp, 1, stream)
    for i in range(2 * copies):  # warm-up
        if launch(i):
            raise RuntimeError(lib.tl_hip_last_error())
    dev.synchronize()
    e0, e1 = lib.tl_hip_event_create(), lib.tl_hip_event_create()
    per = []
    for _ in range(blocks):
        # the stall keeps the GPU busy while the host enqueues every timed launch, so the
        # events measure back-to-back GPU execution, not the host's launch rate
        lib.tl_hip_stall(20000)
        lib.tl_hip_event_record(e0)
        for i in range(launches):
            launch(i)
        lib.tl_hip_event_record(e1)
        ms = C.c_float()
        lib.tl_hip_event_elapsed_ms(e0, e1, C.byref(ms))
        per.append(ms.value / 1e3 / launches)
    lib.tl_hip_event_destroy(e0)
    lib.tl_hip_event_destroy(e1)
    for w in ws:
        w.release()
    return per if blocks > 1 else per[0]


def bench_quant_matvec(dev):
    """The 4096 x 4096 m = 1 matvec in every resident type (GB/s of algorithmic bytes)."""
    rows = []
    for t, name in ((2, "Q4_0"), (8, "Q8_0"), (12, "Q4_K"), (14, "Q6_K")):
        sec = bench_matvec(dev, t)
        gbs = matvec_bytes(t) / sec / 1e9
        rows.append({"type": name, "bytes": matvec_bytes(t), "us": round(sec * 1e6, 3), "gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)})
        log(f"[bench] matvec {name} 4096x4096: {sec * 1e6:.2f} us, {gbs:.0f} GB/s")
    return rows


def bench_matvec_shapes(dev):
    """configs[2] at M = 1: the Q4_0 and Q8_0 matvec at the three (N, K) shapes (GB/s)."""
    rows = []
    for t, name in ((2, "Q4_0"), (8, "Q8_0")):
        for n, k in GEMM_SHAPES:
            sec = bench_matvec(dev, t, launches=200, n=n, k=k)
            gbs = matvec_bytes(t, n, k) / sec / 1e9
            rows.append({"type": name, "n": n, "k": k, "bytes": matvec_bytes(t, n, k), "us": round(sec * 1e6, 3),
                         "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
            log(f"[bench] matvec {name} M=1 N={n} K={k}: {sec * 1e6:.2f} us, {gbs:.0f} GB/s")
    return rows


MFMA_F16_PEAK_TFLOPS = 2500.0
ROOFLINE_BLOCKS = 9  # timed blocks of the roofline matvec (their per-launch averages give p10 / median / p90)
GEMM_SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008)]  # configs[2] (N, K), M = 512
ATTN_CASES = [(512, 1), (2048, 1), (8192, 1), (512, 8), (2048, 8), (8192, 8)]  # configs[3] (L, B)


def _timed(dev, launch, reps):
    """Average seconds per call of launch(i) over reps back-to-back calls on the library
    stream (a stall kernel covers the host's enqueue time)."""
    import ctypes as C
    lib = dev.lib
    for i in range(3):
        launch(i)
    dev.synchronize()
    e0, e1 = lib.tl_hip_event_create(), lib.tl_hip_event_create()
    lib.tl_hip_stall(20000)
    lib.tl_hip_event_record(e0)
    for i in range(reps):
        launch(i)
    lib.tl_hip_event_record(e1)
    ms = C.c_float()
    lib.tl_hip_event_elapsed_ms(e0, e1, C.byref(ms))
    lib.tl_hip_event_destroy(e0)
    lib.tl_hip_event_destroy(e1)
    return ms.value / 1e3 / reps


def bench_sample(dev, reps=100):
    """Top-p sampling (tl_hip_tensor_sample_uniform, the chatbot's sample(temp, top_p) with
    the draw given) over vocab-sized logits [32000] ~ N(0, 3): us per call back to back."""
    rng = np.random.default_rng(0x5A41)
    t = dev.tensor_new((rng.standard_normal(32000) * 3).astype(np.float32))
    us = rng.random(reps)
    rows = []
    for temp, top_p in ((0.1, 0.9), (1.0, 0.9), (2.5, 0.95)):
        sec = _timed(dev, lambda i: dev.tensor_sample_uniform(t, temp, top_p, float(us[i % reps])), reps)
        rows.append({"n": 32000, "temp": temp, "top_p": top_p, "us": round(sec * 1e6, 2)})
        log(f"[bench] sample top-p n=32000 temp={temp} top_p={top_p}: {sec * 1e6:.1f} us")
    return rows


def bench_gemm(dev, ms=(512, 128, 16), reps=20, shapes=None):
    """Quantized prefill GEMM on the f16 MFMA path (tl_hip_launch_quant_gemm, mode 1: the
    f32 -> f16 operand conversion + the MFMA kernel) at the configs[2] shapes and M values
    (M = 1 is the matvec leg).  GB/s counts the quant weights + X + Y once."""
    import ctypes as C

    from tl_amd import GGML_Q4_0, GGML_Q8_0, QTensor
    from tl_amd.quant import random_q4_0_blocks, random_q8_0_blocks

    lib = dev.lib
    rows = []
    types = ((GGML_Q4_0, random_q4_0_blocks, "Q4_0"), (GGML_Q8_0, random_q8_0_blocks, "Q8_0"))
    for m, (t, gen, name), (n, k) in itertools.product(ms, types, shapes or GEMM_SHAPES):
        rng = np.random.default_rng(0x71520000 + n + k)
        raw = gen(rng, n, k)
        # below M = 512 the weight stream bounds the call: rotate copies past the Infinity Cache
        copies = 1 if m >= 512 else -(-(320 << 20) // raw.nbytes)
        qs = [QTensor(t, raw, (n, k)) for _ in range(copies)]
        hs = [q.upload(lib) for q in qs]
        x = dev.tensor_new(rng.standard_normal((m, k)).astype(np.float32))
        y = dev.tensor_zeros((m, n))
        stream = lib.tl_hip_stream()

        def launch(i):
            if lib.tl_hip_launch_quant_gemm(hs[i % copies], C.c_void_p(x.data_ptr), C.c_void_p(y.data_ptr), m, 1,
                                            stream):
                raise RuntimeError(lib.tl_hip_last_error())
        sec = _timed(dev, launch, max(reps, 2 * copies))
        tflops = 2.0 * m * n * k / sec / 1e12
        gbs = (matvec_bytes(t, n, k) - 4 * (n + k) + 4 * m * (n + k)) / sec / 1e9
        rows.append({"type": name, "m": m, "n": n, "k": k, "us": round(sec * 1e6, 2),
                     "tflops": round(tflops, 1), "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                     "gbs": round(gbs, 1)})
        log(f"[bench] prefill GEMM {name} M={m} N={n} K={k}: {sec * 1e6:.1f} us, {tflops:.0f} TFLOP/s "
            f"({100 * tflops / MFMA_F16_PEAK_TFLOPS:.1f}% of dense f16 MFMA peak), {gbs:.0f} GB/s")
        for q in qs:
            q.release()
    return rows


PREFILL_SHAPES = [(2560, 2048), (2048, 2048), (11264, 2048), (2048, 5632)]  # TinyLlama qkv, o, gate/up, down


def bench_vendor_gemm(dev, shapes, m=512, reps=30):
    """Reference point for the prefill GEMM: the vendor library's plain f16 GEMM
    (torch.nn.functional.linear -> hipBLASLt) on f16 weights already resident (4 x the Q4_0
    bytes, no dequantization) at the same M and shapes, timed back to back behind a stall
    kernel on torch's stream.  Not a product path: nothing in the library calls it."""
    import ctypes as C

    import torch

    lib = dev.lib
    # a stream of torch's own (default priority): torch's default stream is the null stream,
    # and a null handle would send the library's stall and events to the library stream
    ts = torch.cuda.Stream()
    lib.tl_hip_set_stream(C.c_void_p(ts.cuda_stream))
    rows = []
    try:
        for n, k in shapes:
            g = torch.Generator(device="cuda").manual_seed(n * 131 + k)
            x = torch.randn(m, k, device="cuda", dtype=torch.float16, generator=g)
            w = torch.randn(n, k, device="cuda", dtype=torch.float16, generator=g) * 0.02
            torch.cuda.synchronize()
            with torch.cuda.stream(ts):
                sec = _timed(dev, lambda i: torch.nn.functional.linear(x, w), reps)
            tflops = 2.0 * m * n * k / sec / 1e12
            rows.append({"m": m, "n": n, "k": k, "us": round(sec * 1e6, 2), "tflops": round(tflops, 1),
                         "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)})
            log(f"[bench] vendor f16 GEMM (hipBLASLt via torch) M={m} N={n} K={k}: {sec * 1e6:.1f} us, "
                f"{tflops:.0f} TFLOP/s ({100 * tflops / MFMA_F16_PEAK_TFLOPS:.1f}% of dense f16 MFMA peak)")
    finally:
        torch.cuda.synchronize()
        lib.tl_hip_set_stream(None)
    return rows


def _copy_floor(dev, half, reps, min_bytes):
    """Seconds per device-to-device copy of `half` bytes (read half, write half: the traffic of
    a row op of 2 half algorithmic bytes), sources and destinations rotated past the Infinity
    Cache like the row ops' inputs: the one-launch floor of a streaming kernel of that size."""
    import ctypes as C
    half = -(-half // 256) * 256
    n = -(-min_bytes // half)
    src = [dev.lib.tl_hip_malloc(half) for _ in range(n)]
    dst = [dev.lib.tl_hip_malloc(half) for _ in range(n)]

    def cp(i):
        dev.lib.tl_hip_memcpy_d2d(C.c_void_p(dst[i % n]), C.c_void_p(src[i % n]), half)
    sec = _timed(dev, cp, max(reps, n))
    dev.synchronize()
    for b in src + dst:
        dev.lib.tl_hip_free(C.c_void_p(b))
    return sec


def bench_row_ops(dev, reps=60, min_bytes=320 << 20):
    """configs[1] row ops on f32 activations, each input uploaded in enough copies (>= 320 MB)
    that the Infinity Cache cannot serve it: GB/s of the algorithmic bytes (every input read
    once, the output written once), beside a device copy that moves the same bytes."""
    rng = np.random.default_rng(0x71510001)
    x = rng.standard_normal((512, 4096)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    xr = rng.standard_normal((512, 32, 128)).astype(np.float32)
    g = rng.standard_normal((512, 11008)).astype(np.float32)
    u = rng.standard_normal((512, 11008)).astype(np.float32)
    lg = (3.0 * rng.standard_normal((512, 32000))).astype(np.float32)
    wt = dev.tensor_new(w)
    cos, sin = dev.tensor_rope_new_cos(128, 512, 10000.0), dev.tensor_rope_new_sin(128, 512, 10000.0)
    cases = [
        ("rms_norm", "[512, 4096] * w[4096], eps 1e-5", 16_793_600, (x,),
         lambda t: dev.tensor_rms_norm(t[0], wt, 1e-5)),
        ("apply_rope (per-token positions)", "[512, 32, 128], tables [512, 128]", 16_777_216 + 524_288, (xr,),
         lambda t: dev.tensor_apply_rope_pos(t[0], cos, sin, 0, 32)),
        ("fused_silu_mul", "gate, up [512, 11008]", 67_633_152, (g, u),
         lambda t: dev.fused_silu_mul(t[0], t[1])),
        ("softmax (last axis)", "[512, 32000]", 131_072_000, (lg,),
         lambda t: dev.tensor_softmax(t[0], -1)),
    ]
    rows = []
    for name, shape, nbytes, arrays, call in cases:
        copies = -(-min_bytes // sum(a.nbytes for a in arrays))
        ins = [tuple(dev.tensor_new(a) for a in arrays) for _ in range(copies)]

        def launch(i):
            call(ins[i % copies]).release()
        sec = _timed(dev, launch, max(reps, copies))
        gbs = nbytes / sec / 1e9
        for t in ins:
            for h in t:
                h.release()
        csec = _copy_floor(dev, nbytes // 2, reps, min_bytes)
        rows.append({"op": name, "shape": shape, "bytes": nbytes, "us": round(sec * 1e6, 2), "gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "copy_us": round(csec * 1e6, 2),
                     "of_copy": round(csec / sec, 3)})
        log(f"[bench] {name} {shape}: {sec * 1e6:.1f} us, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak); "
            f"a device copy of the same bytes {csec * 1e6:.1f} us")
    for t in (wt, cos, sin):
        t.release()
    return rows


def bench_attention(dev, reps=20, hq=32, hkv=8, d=128, min_bytes=300 << 20):
    """Decode attention over an f16 KV cache at the configs[3] cases, rotating KV copies so
    that at least 300 MB are touched (the 256 MB Infinity Cache cannot hold them)."""
    rows = []
    for L, B in ATTN_CASES:
        rng = np.random.default_rng(0x71530000 + L + B)
        kv_bytes = 2 * B * hkv * L * d * 2
        copies = max(1, min(64, -(-min_bytes // kv_bytes)))
        q = dev.tensor_new(rng.standard_normal((B, hq, d)).astype(np.float32))
        kvs = []
        for _ in range(copies):
            kh = rng.standard_normal((B, hkv, L, d)).astype(np.float16)
            kvs.append((dev.tensor_new_f16(kh), dev.tensor_new_f16(kh[..., ::-1].copy())))

        def launch(i):
            k, v = kvs[i % copies]
            dev.attention_decode(q, k, v, L, 1.0 / np.sqrt(d)).release()
        sec = _timed(dev, launch, max(reps, copies))
        algo = kv_bytes + B * hq * d * 4 * 2
        gbs = algo / sec / 1e9
        rows.append({"L": L, "B": B, "us": round(sec * 1e6, 2), "gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)})
        log(f"[bench] decode attention L={L} B={B}: {sec * 1e6:.1f} us, {gbs:.0f} GB/s")
        for k, v in kvs:
            k.release()
            v.release()
        q.release()
    return rows


def _host_cpu():
    """Host CPU model, the cores this process may use, and the core the CPU legs are pinned to."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cores = sorted(os.sched_getaffinity(0))
    return {"cpu_model": model, "nproc": len(cores), "os_cpu_count": os.cpu_count(), "pinned_core": cores[0]}


def _cpu_time(fn, reps=1):
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps


def cpu_baseline(cfg, L):
    """The reference's tl_cpu path restated by the oracle, on one host core (the process is
    pinned to it first; tl_cpu is single-threaded and scalar).  Legs:
      * decode token: per layer the seven linears as matmul_impl over the cached transposed f32
        weights (system.rs:193-222, tensor.rs:1284-1305), RMSNorm with real norm weights, RoPE,
        the chatbot's attention chain at cache length L (transpose / repeat_interleave /
        matmul_4d / scale / softmax / matmul_4d, chatbot.tl:63-87), SiLU, mul, residual adds;
        one layer timed and multiplied by n_layers, plus the LM head;
      * the configs[0] matvec (4096 x 4096, Q4_0 and Q8_0): cold = dequantize + transpose +
        matmul_impl (the first tl_qtensor_matmul of a weight, system.rs:193-221), steady = the
        cached transposed matmul only;
      * the configs[1] row ops at full size;
      * one configs[2] GEMM (M = 512, 4096 x 4096, Q4_0) on the first 16 rows of X, scaled x32;
      * the configs[3] attention at L = 512, B = 1 through the literal op chain.
    Returns (tok/s, the cpu_baseline object without its "value")."""
    import oracle
    from tl_amd.llama import SLOTS, synthetic_linear, synthetic_norm
    from tl_amd.quant import random_q4_0_blocks, random_q8_0_blocks

    host = _host_cpu()
    allowed = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {host["pinned_core"]})
    rng = np.random.default_rng(5)
    legs = {}
    # -- decode token (configs[4] shape)
    D, H, KV, hd = cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    wts = {}
    for w in SLOTS + ["output"]:
        n, k = cfg.linear_shape(w)
        raw = synthetic_linear(cfg, 1234, 0 if w != "output" else -1, w)
        wts[w] = np.ascontiguousarray(oracle.dequantize(2, raw, n * k).reshape(n, k).T)
    x = rng.standard_normal((1, D)).astype(np.float32)
    an, fn = synthetic_norm(cfg, 1234, 0, 0), synthetic_norm(cfg, 1234, 0, 1)
    cos_t = oracle.rope_table(L + 1, hd, cfg.rope_theta)
    sin_t = oracle.rope_table(L + 1, hd, cfg.rope_theta, sin=True)
    kc = rng.standard_normal((1, KV, L, hd)).astype(np.float32)
    vc = rng.standard_normal((1, KV, L, hd)).astype(np.float32)

    def attn_chain(q4, k4, v4, kcache, vcache, sp):
        # chatbot.tl:60-87 for sl = 1 at start position sp
        cs, ss = oracle.narrow(cos_t, 0, sp, 1), oracle.narrow(sin_t, 0, sp, 1)
        qr, kr = oracle.apply_rope(q4, cs, ss), oracle.apply_rope(k4, cs, ss)
        k_tot = oracle.cat(kcache, oracle.transpose(kr, 1, 2), 2)
        v_tot = oracle.cat(vcache, oracle.transpose(v4, 1, 2), 2)
        kw = oracle.repeat_interleave(k_tot, q4.shape[2] // k4.shape[2], 1)
        vw = oracle.repeat_interleave(v_tot, q4.shape[2] // k4.shape[2], 1)
        sm = oracle.scale(oracle.matmul(oracle.transpose(qr, 1, 2), oracle.transpose(kw, 2, 3)),
                          1.0 / np.sqrt(q4.shape[3]))
        return oracle.transpose(oracle.matmul(oracle.softmax(sm, 3), vw), 1, 2)

    def layer():
        h = oracle.rms_norm(x, an, cfg.eps)
        q = oracle.matmul(h, wts["attn_q"]).reshape(1, 1, H, hd)
        k = oracle.matmul(h, wts["attn_k"]).reshape(1, 1, KV, hd)
        v = oracle.matmul(h, wts["attn_v"]).reshape(1, 1, KV, hd)
        ao = attn_chain(q, k, v, kc, vc, L - 1).reshape(1, D)
        x2 = oracle.binop("add", x, oracle.matmul(ao, wts["attn_output"]))
        h2 = oracle.rms_norm(x2, fn, cfg.eps)
        g = oracle.silu(oracle.matmul(h2, wts["ffn_gate"]))
        u = oracle.matmul(h2, wts["ffn_up"])
        return oracle.binop("add", x2, oracle.matmul(oracle.binop("mul", g, u), wts["ffn_down"]))

    t_layer = _cpu_time(layer)
    x2 = layer()
    t_head = _cpu_time(lambda: oracle.matmul(oracle.rms_norm(x2, an, cfg.eps), wts["output"]))
    tok_s = 1.0 / (cfg.n_layers * t_layer + t_head)
    legs["decode_token"] = {"s": round(cfg.n_layers * t_layer + t_head, 3), "layer_s": round(t_layer, 3),
                            "lm_head_s": round(t_head, 3), "cache_len": L}
    del wts
    # -- 4096 x 4096 matvec, cold and steady
    n = k = 4096
    xv = rng.standard_normal((1, k)).astype(np.float32)
    for t, name, gen in ((2, "Q4_0", random_q4_0_blocks), (8, "Q8_0", random_q8_0_blocks)):
        raw = gen(np.random.default_rng(0x71510000), n, k)
        cold = _cpu_time(lambda: oracle.qtensor_matmul(xv, raw, t, n, fast=False))
        wt = np.ascontiguousarray(oracle.dequantize(t, raw, n * k).reshape(n, k).T)
        steady = _cpu_time(lambda: oracle.matmul(xv, wt), reps=3)
        legs[f"matvec_{name}_4096"] = {"cold_s": round(cold, 4), "steady_s": round(steady, 4),
                                       "steady_gbs_f32_weights": round(n * k * 4 / steady / 1e9, 2)}
        del wt
    # -- row ops at full size
    xr = rng.standard_normal((512, 4096)).astype(np.float32)
    w1 = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    xq = rng.standard_normal((512, 32, 128)).astype(np.float32)
    c1, s1 = oracle.rope_table(512, 128, 10000.0), oracle.rope_table(512, 128, 10000.0, sin=True)
    g1 = rng.standard_normal((512, 11008)).astype(np.float32)
    u1 = rng.standard_normal((512, 11008)).astype(np.float32)
    lg = (3.0 * rng.standard_normal((512, 32000))).astype(np.float32)
    legs["row_ops"] = {
        "rms_norm_512x4096_s": round(_cpu_time(lambda: oracle.rms_norm(xr, w1, 1e-5)), 4),
        "apply_rope_512x32x128_s": round(_cpu_time(lambda: oracle.apply_rope(xq, c1, s1)), 4),
        "silu_mul_512x11008_s": round(_cpu_time(lambda: oracle.binop("mul", oracle.silu(g1), u1)), 4),
        "softmax_512x32000_s": round(_cpu_time(lambda: oracle.softmax(lg, -1)), 4),
    }
    del g1, u1, lg
    # -- M = 512 GEMM, 4096 x 4096 Q4_0, rows 0..15 of X timed, x 32
    raw = random_q4_0_blocks(np.random.default_rng(0x71520000), n, k)
    wt = np.ascontiguousarray(oracle.dequantize(2, raw, n * k).reshape(n, k).T)
    xg = rng.standard_normal((16, k)).astype(np.float32)
    tg = _cpu_time(lambda: oracle.matmul(xg, wt)) * 32
    legs["gemm_Q4_0_m512_4096"] = {"s": round(tg, 3), "sample": "rows 0..15 of X timed, scaled x 32",
                                   "gflops": round(2 * 512 * n * k / tg / 1e9, 3)}
    del wt
    # -- decode attention L = 512, B = 1 (Hq 32, Hkv 8, D 128) through the op chain
    La = 512
    qa = rng.standard_normal((1, 1, 32, 128)).astype(np.float32)
    ka = rng.standard_normal((1, 1, 8, 128)).astype(np.float32)
    va = rng.standard_normal((1, 1, 8, 128)).astype(np.float32)
    kca = rng.standard_normal((1, 8, La - 1, 128)).astype(np.float16).astype(np.float32)
    vca = rng.standard_normal((1, 8, La - 1, 128)).astype(np.float16).astype(np.float32)
    cos_t = oracle.rope_table(La, 128, 10000.0)
    sin_t = oracle.rope_table(La, 128, 10000.0, sin=True)
    legs["attention_L512_B1"] = {"s": round(_cpu_time(lambda: attn_chain(qa, ka, va, kca, vca, La - 1), reps=3), 5)}
    os.sched_setaffinity(0, allowed)
    return tok_s, {"host": host, "legs": legs}


def bench_decode(dev, cfg, ggml_type, args, steps=None, variants=()):
    """Prefill of the prompt, then warm-up and timed greedy decode tokens (hipGraph replay
    unless --no-graph); returns (tok/s, decode seconds, prefill seconds, 32-token prefill
    seconds, variant rows).  The warm-up generate captures the decode step; the timed one
    must replay it without a new capture (checked with the library's capture counter).
    `variants` are further (kv, penalty[, temp, top_p]) settings timed the same way on the same
    weights; with temp > 0 every token is sampled (sample(temp, top_p), seeded draws), as the
    chatbot does with (0.1, 0.9)."""
    from tl_amd.llama import HipLlama, synthetic_prompt, synthetic_weights

    steps = steps or args.steps
    log(f"[bench] generating synthetic TinyLlama-shape {ggml_type if isinstance(ggml_type, str) else 'Q4_0'} "
        f"weights ...")
    t0 = time.time()
    model = HipLlama(cfg, kv_f16=(args.kv == "f16"))
    model.load(synthetic_weights(cfg, 1234, ggml_type=ggml_type), ggml_type=ggml_type)
    log(f"[bench] weights resident ({time.time() - t0:.1f} s)")
    prompt = synthetic_prompt(cfg, 1234, args.prompt)
    # one untimed prefill first: the activation buffers for the prompt length are allocated
    # and the kernels' code objects loaded on first use; the timed prefill is the second
    model.reset()
    model.forward(prompt, prefill_f16=True, want_logits=False)
    model.reset()
    dev.synchronize()
    t0 = time.perf_counter()
    model.forward(prompt, prefill_f16=True, want_logits=False)
    dev.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"[bench] prefill {args.prompt} tokens: {prefill_s * 1e3:.1f} ms")
    # a chat-length prompt (32 tokens: short-input GEMM tiles with split K), warm, then the
    # long prompt again so that decode continues from its cache
    short_s = 0.0
    for _ in range(2):
        model.reset()
        dev.synchronize()
        t0 = time.perf_counter()
        model.forward(prompt[:32], prefill_f16=True, want_logits=False)
        dev.synchronize()
        short_s = time.perf_counter() - t0
    log(f"[bench] prefill 32 tokens: {short_s * 1e3:.2f} ms")

    def timed_decode(penalty, temp=0.0, top_p=1.0):
        model.reset()
        model.forward(prompt, prefill_f16=True, want_logits=False)
        model.lib.tl_hip_sample_seed(1234)
        first = model.sample(temp, top_p, penalty, prompt)
        model.set_sampling(temp, top_p)
        hist = np.concatenate([prompt, [first]]).astype(np.int32)
        warm = model.generate(first, args.warmup, penalty, hist, use_graph=not args.no_graph) \
            if args.warmup else np.array([first], np.int32)
        nxt = int(warm[-1])
        hist = np.concatenate([hist, warm[:-1]]).astype(np.int32)
        builds = model.lib.tl_hip_llama_graph_builds(model.h)
        dev.synchronize()
        t0 = time.perf_counter()
        model.generate(nxt, steps, penalty, hist, use_graph=not args.no_graph)  # ends with a stream synchronize
        dev.synchronize()
        dt = time.perf_counter() - t0
        model.set_sampling(0.0)
        if args.warmup and not args.no_graph and model.lib.tl_hip_llama_graph_builds(model.h) != builds:
            raise RuntimeError("the timed decode captured a new graph")
        return dt

    decode_s = timed_decode(1.0)
    tok_s = steps / decode_s
    log(f"[bench] decode {steps} tokens: {decode_s * 1e3:.1f} ms -> {tok_s:.1f} tok/s")
    rows = []
    for kv, pen, *smp in variants:
        temp, top_p = smp if smp else (0.0, 1.0)
        model.configure(kv_f16=(kv == "f16"))
        dt = timed_decode(pen, temp, top_p)
        row = {"kv_cache": kv, "repetition_penalty": pen, "value": round(steps / dt, 2), "unit": "tok/s",
               "ms_per_step": round(dt * 1e3 / steps, 4)}
        if temp > 0:
            row["sample"] = {"temp": temp, "top_p": top_p}
        rows.append(row)
        log(f"[bench] decode {steps} tokens, {kv} KV cache, penalty {pen}"
            + (f", sample({temp}, {top_p})" if temp > 0 else "") + f": {dt * 1e3:.1f} ms -> {steps / dt:.1f} tok/s")
    model.close()
    return tok_s, decode_s, prefill_s, short_s, rows


def bench_prefill(dev, cfg, args, lengths=(32, 512), reps=4):
    """Warm f16 prefills of the synthetic TinyLlama-shape decoder (Q4_0, then the Q4_K_M
    mixture): the best of `reps` forwards per prompt length, in ms."""
    from tl_amd.llama import HipLlama, synthetic_prompt, synthetic_weights

    out = []
    for gt in (2, "Q4_K_M"):
        model = HipLlama(cfg, kv_f16=True)
        model.load(synthetic_weights(cfg, 1234, ggml_type=gt), ggml_type=gt)
        prompt = synthetic_prompt(cfg, 1234, max(lengths))
        row = {"weights": "Q4_0" if gt == 2 else gt}
        for n in lengths:
            best = float("inf")
            for _ in range(reps + 1):  # the first forward of a length allocates its buffers
                model.reset()
                dev.synchronize()
                t0 = time.perf_counter()
                model.forward(prompt[:n], prefill_f16=True, want_logits=False)
                dev.synchronize()
                best = min(best, time.perf_counter() - t0)
            row[f"prefill_{n}_ms"] = round(best * 1e3, 3)
        log(f"[bench] prefill {row}")
        out.append(row)
        model.close()
    return out


def copy_reference(dev, nbytes=64 << 20):
    """Reference dispatch for the FETCH_SIZE / WRITE_SIZE scale of counter runs: one device
    copy of a known size."""
    import ctypes as C
    src, dst = dev.lib.tl_hip_malloc(nbytes), dev.lib.tl_hip_malloc(nbytes)
    dev.lib.tl_hip_memcpy_d2d(C.c_void_p(dst), C.c_void_p(src), nbytes)
    dev.synchronize()
    dev.lib.tl_hip_free(C.c_void_p(src))
    dev.lib.tl_hip_free(C.c_void_p(dst))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode tokens before timing")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--kv", choices=["f16", "f32"], default="f16")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of hipGraph replay")
    ap.add_argument("--no-extra", action="store_true", help="skip the prefill GEMM and attention legs")
    ap.add_argument("--gemm-only", action="store_true", help="only the prefill GEMM leg (counter runs)")
    ap.add_argument("--gemm-m", type=int, default=0, help="with --gemm-only: this M only (default 512, 128, 16)")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only the M = 512 prefill GEMM at the configs[2] and TinyLlama shapes beside the vendor "
                         "library's plain f16 GEMM on f16 weights (a reference point, not a product path)")
    ap.add_argument("--kquant-only", action="store_true", help="only the per-type matvec and Q4_K_M decode legs")
    ap.add_argument("--attention-only", action="store_true", help="only the decode attention leg (counter runs)")
    ap.add_argument("--read-floor", action="store_true",
                    help="only the 4096x4096 matvec and its one-launch read floor (same shape and copies)")
    ap.add_argument("--matvec-only", action="store_true",
                    help="only the 4096x4096 matvec timing plus a 64 MiB device copy (counter runs)")
    ap.add_argument("--row-ops-only", action="store_true",
                    help="only the configs[1] row-op leg plus a 64 MiB device copy (counter runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the 32- and 512-token prefills of the Q4_0 and Q4_K_M decoders (kernel traces)")
    ap.add_argument("--sample-only", action="store_true", help="only the top-p sampling leg (kernel traces)")
    ap.add_argument("--two-launch-merges", action="store_true",
                    help="split kernels merge their partials in a second kernel, not in-kernel (A/B runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.vendor_gemm:
        # torch brings its own HIP runtime: it finds the GPU only when it initialises before
        # the library does
        import torch
        torch.cuda.init()

    from tl_amd import HipDevice
    from tl_amd.llama import LlamaConfig

    dev = HipDevice(0)
    if args.two_launch_merges:
        dev.lib.tl_hip_debug_one_launch_merge(0)
    cfg = LlamaConfig.tinyllama(max_seq=2048)
    if args.prompt + args.warmup + args.steps > cfg.max_seq:
        sys.exit("prompt + warmup + steps exceed the 2048-position cache")

    if args.vendor_gemm:
        shapes = GEMM_SHAPES + PREFILL_SHAPES
        print(json.dumps({"prefill_gemm": bench_gemm(dev, ms=(512,), shapes=shapes),
                          "vendor_f16_gemm": bench_vendor_gemm(dev, shapes)}), flush=True)
        return
    if args.gemm_only:
        print(json.dumps({"prefill_gemm": bench_gemm(dev, ms=(args.gemm_m,) if args.gemm_m else (512, 128, 16))}),
              flush=True)
        return
    if args.attention_only:
        print(json.dumps({"decode_attention": bench_attention(dev)}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps({"prefill": bench_prefill(dev, cfg, args)}), flush=True)
        return
    if args.sample_only:
        print(json.dumps({"sample_top_p": bench_sample(dev)}), flush=True)
        return
    if args.row_ops_only:
        rows = bench_row_ops(dev)
        copy_reference(dev)
        print(json.dumps({"row_ops": rows, "copy_bytes": 64 << 20}), flush=True)
        return
    if args.kquant_only:
        print(json.dumps({"quant_matvec": bench_quant_matvec(dev)}), flush=True)
        tok_s, decode_s, prefill_s, _, _ = bench_decode(dev, cfg, "Q4_K_M", args, steps=64)
        print(json.dumps({"q4_k_m_decode_tok_s": round(tok_s, 2), "prefill_ms": round(prefill_s * 1e3, 2)}),
              flush=True)
        return

    log("[bench] Q4_0 4096x4096 matvec roofline ...")
    blocks_s = bench_matvec(dev, blocks=ROOFLINE_BLOCKS)
    avg_s = float(np.mean(blocks_s))  # every block has the same launch count: the mean per launch
    spread = {"blocks": ROOFLINE_BLOCKS, "launches_per_block": 340,
              **{f"{name}_us": round(float(np.percentile(blocks_s, q)) * 1e6, 3)
                 for name, q in (("p10", 10), ("median", 50), ("p90", 90))}}
    achieved = MATVEC_BYTES / avg_s / 1e9
    log(f"[bench] matvec avg {avg_s * 1e6:.2f} us -> {achieved:.0f} GB/s; per-block p10 / median / p90 "
        f"{spread['p10_us']:.3f} / {spread['median_us']:.3f} / {spread['p90_us']:.3f} us")
    floor_s = bench_matvec(dev, floor=True)
    log(f"[bench] read floor (the matvec's loads only, same copies) {floor_s * 1e6:.2f} us -> "
        f"{MATVEC_BYTES / floor_s / 1e9:.0f} GB/s")
    if args.read_floor:
        print(json.dumps({"matvec_avg_us": round(avg_s * 1e6, 3), "floor_us": round(floor_s * 1e6, 3)}), flush=True)
        return
    if args.matvec_only:
        copy_reference(dev)
        print(json.dumps({"matvec_avg_us": round(avg_s * 1e6, 3), "matvec_gbs": round(achieved, 1),
                          "copy_bytes": 64 << 20}), flush=True)
        return

    gemm = attn = qmv = qmv2 = rowops = smp = None
    if not args.no_extra:
        qmv = bench_quant_matvec(dev)
        qmv2 = bench_matvec_shapes(dev)
        rowops = bench_row_ops(dev)
        smp = bench_sample(dev)
        gemm = bench_gemm(dev)
        attn = bench_attention(dev)

    other_kv = "f32" if args.kv == "f16" else "f16"
    tok_s, decode_s, prefill_s, short_s, variants = bench_decode(
        dev, cfg, 2, args, variants=[(args.kv, 1.1), (other_kv, 1.0), (args.kv, 1.1, 0.1, 0.9)])
    kq = None
    if not args.no_extra:
        kq_tok_s, kq_decode_s, kq_prefill_s, kq_short_s, _ = bench_decode(dev, cfg, "Q4_K_M", args, steps=64)
        kq = {"workload": "same decoder with llama.cpp's Q4_K_M type mixture (Q4_K; Q6_K for the LM head and "
                          "attn_v / ffn_down of 10 of 22 layers: 0, 1, 4, 7, 10, 13, 16, 19, 20, 21)", "value": round(kq_tok_s, 2), "unit": "tok/s",
              "steps": 64, "ms_per_step": round(kq_decode_s * 1e3 / 64, 4), "prefill_ms": round(kq_prefill_s * 1e3, 2),
              "prefill_32_ms": round(kq_short_s * 1e3, 3),
              "prefill_path": "fused f16 MFMA prefill; Q4_K dequantized in registers (per-unit scale pairs built "
                             "once per tensor), Q6_K dequantized to f16 operand order per call"}

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle, 1 pinned core) ...")
        L = args.prompt + args.warmup + args.steps // 2
        cpu_tok_s, extra = cpu_baseline(cfg, L)
        leg = extra["legs"]["decode_token"]
        cpu = {"value": round(cpu_tok_s, 4), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"one decode token at cache length {L}: 1 layer timed ({leg['layer_s']:.2f} s: 7 linears "
                         f"in tl_cpu matmul_impl order over cached transposed f32 weights, the chatbot's "
                         f"attention op chain, norms) x {cfg.n_layers} + LM head ({leg['lm_head_s']:.2f} s)",
               **extra}
        log(f"[bench] CPU {cpu_tok_s:.4f} tok/s on {extra['host']['cpu_model']} (core "
            f"{extra['host']['pinned_core']} of {extra['host']['nproc']}); legs {json.dumps(extra['legs'])}")

    out = {
        "metric": "Q4_0 decode tok/s (batch 1)",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(decode_s * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "TinyLlama-1.1B-shape decoder, Q4_0 linears (random N(0,0.02) before quantization), "
                        "22 layers, d_model 2048, 32 heads / 4 KV heads, FFN 5632, vocab 32000; "
                        f"{args.prompt}-token prompt then greedy decode at batch 1",
            "prompt_tokens": args.prompt,
            "kv_cache": args.kv,
            "repetition_penalty": 1.0,
            "prefill_ms": round(prefill_s * 1e3, 2),
            "prefill_32_ms": round(short_s * 1e3, 3),
        },
        "decode_variants": {"note": "the same model and prompt: the chatbot's repetition penalty 1.1 "
                                    "(chatbot.tl:188), the other KV-cache element type, and the chatbot's "
                                    "loop as it runs: penalty 1.1 then sample(0.1, 0.9) every token "
                                    "(chatbot.tl:189; seeded draws)", "runs": variants},
        "roofline": {
            "bound": "hbm",
            "kernel": "k_mv<Q4_0> 4096x4096 (m=1)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": MATVEC_TRAFFIC,
            "traffic_source": "not measured in this run: FETCH_SIZE + WRITE_SIZE counter runs of "
                              "`bench.py --matvec-only` (profiles/q4_0_matvec_4096x4096.md)",
            "avg_launch_us": round(avg_s * 1e6, 3),
            "launch_spread": spread,
            "floor_us": round(floor_s * 1e6, 3),
            "floor_note": "tl_hip_read_floor: the matvec's own loads (launch plan, access pattern, quant bytes + "
                          "scales) over the same weight copies, with no math, reduction or store",
        },
        "cpu_baseline": cpu,
        "prefill_gemm": {"path": "f16 MFMA (v_mfma_f32_16x16x32_f16), f32 accumulate", "unit": "TFLOP/s",
                         "peak": MFMA_F16_PEAK_TFLOPS, "shapes": gemm},
        "decode_attention": {"kv": "f16", "hq": 32, "hkv": 8, "head_dim": 128, "unit": "GB/s",
                             "peak": HBM_PEAK_GBS, "cases": attn},
        "quant_matvec": {"shape": "4096x4096, m=1", "unit": "GB/s", "peak": HBM_PEAK_GBS, "types": qmv,
                         "configs2_m1": qmv2},
        "row_ops": {"config": "configs[1]", "unit": "GB/s", "peak": HBM_PEAK_GBS, "ops": rowops},
        "sample_top_p": {"unit": "us per call", "cases": smp},
        "q4_k_m_decode": kq,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
