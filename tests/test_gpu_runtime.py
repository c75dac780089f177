"""GPU checks of the runtime around the kernels: allocation failure surfaces as NULL +
AllocationError (where the reference panics, tl_cuda tensor.rs:128-141), and the caching
allocator does not hand memory with pending work on one stream to another stream."""
import ctypes as C

import numpy as np
import pytest

import oracle
from tl_amd import GGML_Q4_0, QTensor, _lib
from tl_amd.quant import random_q4_0_blocks

pytestmark = pytest.mark.gpu


def _hip():
    for name in ("libamdhip64.so", "libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so"):
        try:
            return C.CDLL(name)
        except OSError:
            continue
    pytest.skip("libamdhip64 not found")


def test_impossible_allocation_is_an_allocation_error(dev):
    lib = _lib.load()
    for shape in ((1 << 40,), (1 << 31, 1 << 31)):   # 4 TiB of f32; 2^62 elements (size overflow)
        s = (C.c_int64 * len(shape))(*shape)
        lib.tl_hip_clear_error()
        assert not lib.tl_hip_tensor_zeros(s, len(shape), 0)
        assert lib.tl_hip_last_status() == 3, lib.tl_hip_last_error()
        assert b"AllocationError" in lib.tl_hip_last_error()
    # the library stays usable
    t = dev.tensor_new(np.arange(6, dtype=np.float32).reshape(2, 3))
    assert np.array_equal(t.to_numpy(), np.arange(6, dtype=np.float32).reshape(2, 3))


def test_injected_allocation_failure_returns_null(dev):
    lib = _lib.load()
    lib.tl_hip_debug_fail_alloc(0)
    try:
        s = (C.c_int64 * 1)(1000)
        assert not lib.tl_hip_tensor_zeros(s, 1, 0)
        assert lib.tl_hip_last_status() == 3
    finally:
        lib.tl_hip_debug_fail_alloc(-1)
    t = dev.tensor_new(np.ones(1000, np.float32))
    assert np.all(t.to_numpy() == 1.0)


def test_release_does_not_hand_pending_memory_to_another_stream(dev):
    """x is read by a matvec queued behind a 20 ms stall on the library stream and released
    right after the launch; a same-size tensor then written on a second stream must get other
    memory, or the matvec would read the new values."""
    hip = _hip()
    lib = _lib.load()
    other = C.c_void_p()
    assert hip.hipStreamCreate(C.byref(other)) == 0
    try:
        # first sight of a second stream: the allocator switches to event-tagged frees
        assert lib.tl_hip_set_stream(other) == 0
        assert lib.tl_hip_set_stream(None) == 0
        rng = np.random.default_rng(0x5107)
        n, k = 4096, 4096
        raw = random_q4_0_blocks(rng, n, k)
        w = QTensor(GGML_Q4_0, raw, (n, k))
        w.upload(lib)
        x = rng.standard_normal((1, k)).astype(np.float32)
        x_other = np.full((1, k), 1e6, np.float32)
        xt = dev.tensor_new(x)
        lib.tl_hip_synchronize()
        assert lib.tl_hip_stall(20000) == 0
        y = dev.tl_qtensor_matmul(xt, w)          # runs after the stall
        xt.release()                               # freed on the library stream, work pending
        assert lib.tl_hip_set_stream(other) == 0
        try:
            xo = dev.tensor_new(x_other)           # H2D on the other stream, finished at return
        finally:
            lib.tl_hip_set_stream(None)
        got = y.to_numpy()
        ref = oracle.qtensor_matmul(x, raw, GGML_Q4_0, n)
        err = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
        assert err <= 1e-4, f"matvec read memory rewritten by another stream (max-rel-err {err:.2e})"
        # and the same-stream case still reuses memory in stream order
        assert np.all(xo.to_numpy() == 1e6)
    finally:
        hip.hipStreamSynchronize(other)
        hip.hipStreamDestroy(other)


def test_launcher_on_a_caller_stream(dev):
    """tl_hip_launch_quant_gemm on a caller stream: its temporaries (f16 X copy, split-K
    partials) are freed on that stream; results equal the library-stream call."""
    hip = _hip()
    lib = _lib.load()
    other = C.c_void_p()
    assert hip.hipStreamCreate(C.byref(other)) == 0
    try:
        rng = np.random.default_rng(0x5108)
        n, k, m = 1024, 4096, 16
        raw = random_q4_0_blocks(rng, n, k)
        w = QTensor(GGML_Q4_0, raw, (n, k))
        hw = w.upload(lib)
        x = rng.standard_normal((m, k)).astype(np.float32)
        xt = dev.tensor_new(x)
        outs = []
        for stream in (None, other, other, None):
            yt = dev.tensor_new(np.zeros((m, n), np.float32))
            assert lib.tl_hip_launch_quant_gemm(hw, xt.data_ptr, yt.data_ptr, m, 1, stream) == 0
            if stream is not None:
                assert hip.hipStreamSynchronize(stream) == 0
            outs.append(yt.to_numpy())
        for o in outs[1:]:
            assert np.array_equal(o, outs[0])
        ref = oracle.qtensor_matmul(x, raw, GGML_Q4_0, n)
        assert float(np.max(np.abs(outs[0] - ref)) / np.max(np.abs(ref))) <= 1e-2
    finally:
        hip.hipStreamSynchronize(other)
        hip.hipStreamDestroy(other)


@pytest.mark.parametrize("t", [2, 8, 12, 14])
def test_read_floor_launches_for_every_type(dev, t):
    """tl_hip_read_floor (the roofline's one-launch read of a weight) runs for every resident
    type and leaves the library usable."""
    from tl_amd.quant import random_q4_0_blocks, random_q4_k_blocks, random_q6_k_blocks, random_q8_0_blocks
    lib = _lib.load()
    gen = {2: random_q4_0_blocks, 8: random_q8_0_blocks, 12: random_q4_k_blocks, 14: random_q6_k_blocks}[t]
    rng = np.random.default_rng(0x5109 + t)
    w = QTensor(t, gen(rng, 512, 2048), (512, 2048))
    hw = w.upload(lib)
    for _ in range(3):
        assert lib.tl_hip_read_floor(hw, None) == 0
    assert lib.tl_hip_synchronize() == 0
    assert lib.tl_hip_read_floor(None, None) == 4
