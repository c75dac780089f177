"""tl_hip_launch_quant_gemm_noalloc (the allocation-free GEMM entry) against the allocating
tl_hip_launch_quant_gemm on the same inputs, called through the C ABI: calls in a row, each
with a smaller input than the one before (64-row tiles with split-K partials in the scratch,
then the short-input kernel), the size and type limits of its fixed scratch, and the entry
under hipGraph capture, on the library stream (one-launch split-K sums) and on a caller
stream."""
import ctypes as C

import numpy as np
import pytest

import oracle
from tl_amd import GGML_Q4_0, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, QTensor, _lib
from tl_amd.quant import random_q4_0_blocks, random_q4_k_blocks, random_q6_k_blocks, random_q8_0_blocks

pytestmark = pytest.mark.gpu

_GEN = {GGML_Q4_0: random_q4_0_blocks, GGML_Q8_0: random_q8_0_blocks}


def _plan(lib):
    v = [C.c_int32() for _ in range(3)]
    assert lib.tl_hip_debug_last_gemm_plan(*[C.byref(x) for x in v]) == 0
    return tuple(x.value for x in v)


def _run(dev, lib, entry, hw, x, n):
    m = x.shape[0]
    xt = dev.tensor_new(x)
    yt = dev.tensor_new(np.full((m, n), np.nan, np.float32))
    noalloc = entry.__name__ == "tl_hip_launch_quant_gemm_noalloc"
    if noalloc:   # any allocation inside the call fails it (AllocationError)
        dev.synchronize()
        lib.tl_hip_debug_fail_alloc(0)
    try:
        rc = entry(hw, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), m, 1, None)
    finally:
        if noalloc:
            lib.tl_hip_debug_fail_alloc(-1)
    assert rc == 0, lib.tl_hip_last_error()
    return yt.to_numpy(), _plan(lib)


@pytest.mark.parametrize("t", [GGML_Q4_0, GGML_Q8_0])
def test_noalloc_gemm_equals_the_allocating_entry(dev, t):
    lib = _lib.load()
    rng = np.random.default_rng(0x71580000 + t)
    n, k = 4096, 4096
    raw = _GEN[t](rng, n, k)
    w = QTensor(t, raw, (n, k))
    hw = w.upload(lib)
    # each call smaller than the one before: 128-row tiles; 64-row tiles with K split (partial
    # tiles in the scratch); the short-input kernel (no scratch at all)
    for m in (512, 64, 16):
        x = rng.standard_normal((m, k)).astype(np.float32)
        want, want_plan = _run(dev, lib, lib.tl_hip_launch_quant_gemm, hw, x, n)
        got, got_plan = _run(dev, lib, lib.tl_hip_launch_quant_gemm_noalloc, hw, x, n)
        assert got_plan == want_plan
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"m={m}: results differ"
        ref = oracle.qtensor_matmul(x, raw, t, n)
        err = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
        assert err <= 1e-2, f"m={m}: max-rel-err {err:.2e} vs the oracle"
        if m == 64:
            assert got_plan[2] > 1  # split-K partials in the scratch


def test_noalloc_gemm_limits(dev):
    lib = _lib.load()
    rng = np.random.default_rng(0x71580100)
    k = 4096
    w = QTensor(GGML_Q4_0, random_q4_0_blocks(rng, 256, k), (256, k))
    hw = w.upload(lib)
    big = dev.tensor_new(np.zeros((4100, k), np.float32))   # 4100 x 4096 f16 > 32 MiB
    y = dev.tensor_new(np.zeros((4100, 256), np.float32))
    lib.tl_hip_clear_error()
    assert lib.tl_hip_launch_quant_gemm_noalloc(hw, C.c_void_p(big.data_ptr), C.c_void_p(y.data_ptr), 4100, 1,
                                                None) == 8
    assert b"scratch" in lib.tl_hip_last_error()
    # Q6_K needs an f16 copy of the weight for the MFMA path: rejected; the f32 path runs
    w6 = QTensor(GGML_Q6_K, random_q6_k_blocks(rng, 256, k), (256, k))
    h6 = w6.upload(lib)
    x = rng.standard_normal((8, k)).astype(np.float32)
    xt = dev.tensor_new(x)
    yt = dev.tensor_new(np.zeros((8, 256), np.float32))
    assert lib.tl_hip_launch_quant_gemm_noalloc(h6, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), 8, 1,
                                                None) == 8
    assert lib.tl_hip_launch_quant_gemm_noalloc(h6, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), 8, 0,
                                                None) == 0
    ref = oracle.qtensor_matmul(x, w6.data, GGML_Q6_K, 256)
    assert float(np.max(np.abs(yt.to_numpy() - ref)) / np.max(np.abs(ref))) <= 1e-4
    # Q4_K takes the MFMA path once its per-unit scales exist (built by an allocating f16 call)
    w4 = QTensor(GGML_Q4_K, random_q4_k_blocks(rng, 256, k), (256, k))
    h4 = w4.upload(lib)
    assert lib.tl_hip_launch_quant_gemm_noalloc(h4, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), 8, 1,
                                                None) == 8
    assert lib.tl_hip_launch_quant_gemm(h4, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), 8, 1, None) == 0
    want = yt.to_numpy()
    yt2 = dev.tensor_new(np.zeros((8, 256), np.float32))
    assert lib.tl_hip_launch_quant_gemm_noalloc(h4, C.c_void_p(xt.data_ptr), C.c_void_p(yt2.data_ptr), 8, 1,
                                                None) == 0
    assert np.array_equal(yt2.to_numpy(), want)


def test_one_launch_gemm_under_capture_on_the_library_stream(dev):
    """The allocation-free entry captured on the library's own stream, where K-split GEMMs add
    their slices in the same launch (the tile's last-arriving split) while no other stream has
    run library work: M = 16 (short-input kernel) and M = 48 (64-row tiles, after the X
    conversion).  Every replay -- with a NaN fill of y and eager work between replays -- gives
    the eager call's bits, and the graph holds one kernel node fewer when the one-launch form
    is in effect than when the sum is a kernel of its own."""
    lib = _lib.load()
    hip = C.CDLL("libamdhip64.so.7")
    rng = np.random.default_rng(0x71580300)
    n, k = 4096, 4096
    raw = random_q4_0_blocks(rng, n, k)
    w = QTensor(GGML_Q4_0, raw, (n, k))   # kept alive: the handle below belongs to it
    hw = w.upload(lib)
    stream = C.c_void_p(lib.tl_hip_stream())
    for m in (16, 48):
        x = rng.standard_normal((m, k)).astype(np.float32)
        want, plan = _run(dev, lib, lib.tl_hip_launch_quant_gemm, hw, x, n)
        # K split 8 / 4 ways: within both kernels' one-launch limits (8 and 16 splits)
        assert 1 < plan[2] <= 8, plan
        one = lib.tl_hip_debug_one_launch_merge(-1) == 1
        xt = dev.tensor_new(x)
        yt = dev.tensor_new(np.zeros((m, n), np.float32))
        args = (hw, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), m, 1, stream)
        dev.synchronize()
        graph, gexec = C.c_void_p(), C.c_void_p()
        lib.tl_hip_debug_fail_alloc(0)
        try:
            assert hip.hipStreamBeginCapture(stream, 1) == 0   # thread-local mode
            rc = lib.tl_hip_launch_quant_gemm_noalloc(*args)
            assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
        finally:
            lib.tl_hip_debug_fail_alloc(-1)
        assert rc == 0, lib.tl_hip_last_error()
        try:
            nodes = C.c_size_t(0)
            assert hip.hipGraphGetNodes(graph, None, C.byref(nodes)) == 0
            base = 1 if m <= 16 else 2   # the X conversion precedes the tiled GEMM
            assert nodes.value == base + (0 if one else 1), (m, one, nodes.value)
            assert hip.hipGraphInstantiate(C.byref(gexec), graph, None, None, C.c_size_t(0)) == 0
            nan = np.full((m, n), np.nan, np.float32)
            for rep in range(3):
                assert lib.tl_hip_memcpy_h2d(C.c_void_p(yt.data_ptr), nan.ctypes.data_as(C.c_void_p), nan.nbytes) == 0
                dev.synchronize()
                assert hip.hipGraphLaunch(gexec, stream) == 0
                assert hip.hipStreamSynchronize(stream) == 0
                got = yt.to_numpy()
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"m={m}: replay {rep} differs"
                again, _ = _run(dev, lib, lib.tl_hip_launch_quant_gemm, hw, x, n)
                assert np.array_equal(again.view(np.uint32), want.view(np.uint32))
        finally:
            if gexec.value:
                hip.hipGraphExecDestroy(gexec)
            hip.hipGraphDestroy(graph)


def test_noalloc_gemm_under_graph_capture(dev):
    """The allocation-free entry captured on a caller stream (hipStreamBeginCapture / EndCapture /
    Instantiate / Launch): every replay -- with eager library work and a fresh NaN fill of y
    between replays -- gives the allocating entry's bits, at M = 16 (split-K partials in the
    scratch) and M = 256.  Allocation is made to fail while the call is captured."""
    lib = _lib.load()
    hip = C.CDLL("libamdhip64.so.7")
    rng = np.random.default_rng(0x71580200)
    n, k = 2048, 4096
    raw = random_q4_0_blocks(rng, n, k)
    w = QTensor(GGML_Q4_0, raw, (n, k))   # kept alive: the handle below belongs to it
    hw = w.upload(lib)
    stream = C.c_void_p()
    assert hip.hipStreamCreateWithFlags(C.byref(stream), 1) == 0
    try:
        for m in (16, 256):
            x = rng.standard_normal((m, k)).astype(np.float32)
            want, _ = _run(dev, lib, lib.tl_hip_launch_quant_gemm, hw, x, n)
            xt = dev.tensor_new(x)
            yt = dev.tensor_new(np.zeros((m, n), np.float32))
            args = (hw, C.c_void_p(xt.data_ptr), C.c_void_p(yt.data_ptr), m, 1, stream)
            # one call on the stream before capturing it (the library's first use of a stream)
            assert lib.tl_hip_launch_quant_gemm_noalloc(*args) == 0, lib.tl_hip_last_error()
            assert hip.hipStreamSynchronize(stream) == 0
            graph, gexec = C.c_void_p(), C.c_void_p()
            lib.tl_hip_debug_fail_alloc(0)
            try:
                assert hip.hipStreamBeginCapture(stream, 1) == 0   # thread-local mode
                rc = lib.tl_hip_launch_quant_gemm_noalloc(*args)
                assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
            finally:
                lib.tl_hip_debug_fail_alloc(-1)
            assert rc == 0, lib.tl_hip_last_error()
            assert hip.hipGraphInstantiate(C.byref(gexec), graph, None, None, C.c_size_t(0)) == 0
            try:
                nan = np.full((m, n), np.nan, np.float32)
                for rep in range(3):
                    assert lib.tl_hip_memcpy_h2d(C.c_void_p(yt.data_ptr), nan.ctypes.data_as(C.c_void_p),
                                                 nan.nbytes) == 0
                    dev.synchronize()
                    assert hip.hipGraphLaunch(gexec, stream) == 0
                    assert hip.hipStreamSynchronize(stream) == 0
                    got = yt.to_numpy()
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"m={m}: replay {rep} differs"
                    # eager work on the library stream between replays
                    again, _ = _run(dev, lib, lib.tl_hip_launch_quant_gemm, hw, x, n)
                    assert np.array_equal(again.view(np.uint32), want.view(np.uint32))
            finally:
                hip.hipGraphExecDestroy(gexec)
                hip.hipGraphDestroy(graph)
    finally:
        hip.hipStreamSynchronize(stream)
        hip.hipStreamDestroy(stream)
