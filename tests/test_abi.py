"""C-ABI checks that need no GPU: the library loads, exports every symbol include/tl_hip.h
declares, and turns bad arguments into NULL + a BackendError-style message."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from tl_amd import _lib
from tl_amd.device import BackendError, QTensor, _raise

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "tl_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tl_hip_[a-z0-9_]+)\s*\(", src)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = declared()
    assert len(names) > 60
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/tl_hip.h but not exported"
    assert sorted(_lib.PROTOS) == names, "tl_amd/_lib.py prototypes out of sync with the header"


def test_no_cpu_symbols_from_the_oracle():
    # the product library must not carry the checker
    lib = _lib.load()
    assert not hasattr(lib, "tlo_qtensor_matmul")


def _err(lib):
    return lib.tl_hip_last_status(), lib.tl_hip_last_error().decode()


def test_qtensor_validation_errors_before_device_use():
    lib = _lib.load()
    shape = (C.c_int64 * 2)(4, 64)
    data = np.zeros(4 * 64 // 32 * 18, dtype=np.uint8)
    p = data.ctypes.data_as(_lib.u8p)
    # Data size mismatch (quantized.rs:195-200)
    assert not lib.tl_hip_qtensor_new(2, p, data.nbytes - 1, shape, 2)
    st, msg = _err(lib)
    assert st == 8 and "Data size mismatch for Q4_0" in msg
    # elements not a multiple of 32 (quantized.rs:190-192)
    bad = (C.c_int64 * 2)(3, 33)
    assert not lib.tl_hip_qtensor_new(2, p, data.nbytes, bad, 2)
    st, msg = _err(lib)
    assert st == 1 and "multiple of 32" in msg
    # types without a device residency (13 = Q5_K, 3 = Q4_1)
    for t in (13, 3, 0, 1):
        assert not lib.tl_hip_qtensor_new(t, p, data.nbytes, shape, 2)
        assert _err(lib)[0] == 7
    # K-quants: whole 256-weight blocks per row (quantized.rs:342-344) and 144 bytes each
    assert not lib.tl_hip_qtensor_new(12, p, data.nbytes, shape, 2)
    st, msg = _err(lib)
    assert st == 1 and "multiple of 256 for Q4_K" in msg
    sh256 = (C.c_int64 * 2)(1, 256)
    assert not lib.tl_hip_qtensor_new(14, p, 209, sh256, 2)
    st, msg = _err(lib)
    assert st == 8 and "Data size mismatch for Q6_K: expected 210" in msg
    # a 2-D QTensor is required (system.rs:228)
    assert not lib.tl_hip_qtensor_new(2, p, data.nbytes, shape, 1)
    assert _err(lib)[0] == 1
    # null data
    assert not lib.tl_hip_qtensor_new(2, None, data.nbytes, shape, 2)
    assert _err(lib)[0] == 4


def test_null_handles_are_errors_not_crashes():
    lib = _lib.load()
    assert not lib.tl_hip_qtensor_matmul(None, None)
    st, msg = _err(lib)
    assert st == 4 and "null argument" in msg
    assert lib.tl_hip_tensor_release(None) == 0
    assert lib.tl_hip_qtensor_release(None) == 0
    assert lib.tl_hip_tensor_to_host(None, None, 0) == 4
    assert lib.tl_hip_tensor_numel(None) == -1
    assert lib.tl_hip_llama_forward(None, None, 0, None, 0) == 4


@pytest.mark.skipif(_lib.load().tl_hip_device_count() > 0, reason="a GPU is present")
def test_without_a_device_calls_fail_with_device_error():
    lib = _lib.load()
    x = np.ones(4, np.float32)
    shape = (C.c_int64 * 1)(4)
    assert not lib.tl_hip_tensor_new(x.ctypes.data_as(_lib.f32p), shape, 1)
    st, msg = _err(lib)
    assert st == 2 and msg.startswith("DeviceError")
    with pytest.raises(BackendError) as e:
        _raise(lib)
    assert e.value.variant == "DeviceError"


def test_qtensor_host_object_keeps_bytes():
    q = QTensor(2, bytes(range(18)) * 2, (1, 64))
    assert q.data.nbytes == 36 and q.shape == (1, 64)
