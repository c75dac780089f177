"""The GGUF reader (tl_hip_gguf_*, host-only parsing) against the reference's own GGUF test
file (crates/tl_runtime/tests/gguf_test.rs:10-62), the writer of tl_amd.gguf and hand-built
corner cases.  CPU only: opening and inspecting a file makes no device call."""
import struct

import numpy as np
import pytest

from tl_amd import _lib
from tl_amd.gguf import GgufFile, write_gguf
from tl_amd.device import BackendError


def _reference_test_file(path):
    # byte for byte the file of gguf_test.rs:10-62: magic, version 3, 1 tensor, 0 KV,
    # "tensor1" [10] F32 at offset 0, padding from 63 to 64, ten f32 0.0 .. 9.0
    b = b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", 1) + struct.pack("<Q", 0)
    b += struct.pack("<Q", 7) + b"tensor1" + struct.pack("<I", 1) + struct.pack("<Q", 10)
    b += struct.pack("<I", 0) + struct.pack("<Q", 0)
    assert len(b) == 63
    b += bytes(1)
    b += np.arange(10, dtype=np.float32).tobytes()
    path.write_bytes(b)


def test_reference_gguf_test_file(tmp_path):
    p = tmp_path / "test_simple.gguf"
    _reference_test_file(p)
    g = GgufFile(p)
    assert g.names() == ["tensor1"]
    assert g.info("tensor1") == (0, (10,), 40)
    assert np.array_equal(np.frombuffer(g.data("tensor1"), np.float32), np.arange(10, dtype=np.float32))
    with pytest.raises(BackendError) as e:
        g.info("missing")
    assert e.value.variant == "ArgumentError" and "not found" in str(e.value)
    g.close()


def test_writer_roundtrip_shapes_types_metadata(tmp_path):
    rng = np.random.default_rng(1)
    tensors = [
        ("a.weight", 2, (3, 64), rng.integers(0, 256, 3 * 2 * 18, dtype=np.uint8)),   # Q4_0 [3, 64]
        ("b.weight", 12, (2, 256), rng.integers(0, 256, 2 * 144, dtype=np.uint8)),  # Q4_K
        ("c.weight", 14, (1, 512), rng.integers(0, 256, 2 * 210, dtype=np.uint8)),  # Q6_K, leading 1
        ("n.weight", 0, (7,), np.arange(7, dtype=np.float32).view(np.uint8)),
        ("h.weight", 1, (2, 3, 4), np.arange(24, dtype=np.float16).view(np.uint8)),
    ]
    meta = {"general.architecture": "llama", "llama.block_count": 22, "llama.rope.freq_base": 10000.0,
            "big": 2 ** 40}
    for align in (32, 64):
        p = tmp_path / f"w{align}.gguf"
        write_gguf(p, tensors, meta, alignment=align)
        g = GgufFile(p)
        assert g.names() == [t[0] for t in tensors]
        for name, t, shp, data in tensors:
            want = shp[1:] if shp[0] == 1 and len(shp) > 1 else shp  # gguf.rs:129-133 trims ne's trailing 1s
            assert g.info(name) == (t, want, data.size)
            assert g.data(name) == data.tobytes()
        assert g.meta("llama.block_count") == 22.0 and g.meta("general.architecture") == "llama"
        assert g.meta("llama.rope.freq_base") == 10000.0 and g.meta("big") == float(2 ** 40)
        if align != 32:
            assert g.meta("general.alignment") == align
        g.close()


def test_skips_unknown_types_and_out_of_bounds(tmp_path):
    # a Q5_K tensor (type 13, outside gguf.rs:157-168) is skipped; so is one whose data ends
    # past the end of the file (gguf.rs:177-182)
    p = tmp_path / "skip.gguf"
    write_gguf(p, [("q5k", 13, (1, 256), bytes(176)), ("ok", 0, (4,), np.ones(4, np.float32).view(np.uint8)),
                   ("cut", 0, (64,), np.ones(64, np.float32).view(np.uint8))])
    raw = p.read_bytes()
    p.write_bytes(raw[:-100])  # truncate inside the last tensor
    g = GgufFile(p)
    assert g.names() == ["ok"]
    g.close()


def test_big_endian_header(tmp_path):
    # "FUGG": header fields big-endian (gguf.rs:66-74); data bytes are taken as stored
    b = b"FUGG" + struct.pack(">I", 3) + struct.pack(">Q", 1) + struct.pack(">Q", 1)
    b += struct.pack(">Q", 17) + b"general.alignment" + struct.pack(">I", 4) + struct.pack(">I", 16)
    b += struct.pack(">Q", 1) + b"t" + struct.pack(">I", 2) + struct.pack(">QQ", 4, 2) + struct.pack(">I", 0)
    b += struct.pack(">Q", 0)
    b += bytes((16 - len(b) % 16) % 16) + np.arange(8, dtype=np.float32).tobytes()
    p = tmp_path / "be.gguf"
    p.write_bytes(b)
    g = GgufFile(p)
    assert g.info("t") == (0, (2, 4), 32)
    assert g.data("t") == np.arange(8, dtype=np.float32).tobytes()
    g.close()


def test_decode_errors(tmp_path):
    lib = _lib.load()
    cases = {
        "magic": b"GGML" + bytes(40),
        "version": b"GGUF" + struct.pack("<IQQ", 1, 0, 0),
        "truncated": b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + struct.pack("<Q", 100) + b"abc",
        "tiny": b"GG",
        "bad_kv_type": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 99),
    }
    for name, content in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(content)
        assert not lib.tl_hip_gguf_open(str(p).encode()), name
        assert lib.tl_hip_last_status() == 8, name
    assert not lib.tl_hip_gguf_open(str(tmp_path / "absent.gguf").encode())
    assert b"Failed to open" in lib.tl_hip_last_error()
