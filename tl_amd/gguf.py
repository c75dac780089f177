"""GGUF files: a v3 writer (numpy) and the reader binding.

``write_gguf`` lays a file out the way tl_gguf_load reads it (crates/tl_runtime/src/gguf.rs:
34-196) and the reference's own test writes one (crates/tl_runtime/tests/gguf_test.rs:10-62):
"GGUF", version u32 3, tensor count u64, metadata count u64, the metadata (key string, value
type u32, value), the tensor infos (name string, n_dims u32, ne u64[n_dims] -- the row-major
shape reversed --, ggml type u32, data offset u64), zero padding to ``general.alignment``
(32 unless given), then each tensor's bytes at its offset (offsets aligned too).  Strings are
a u64 length + UTF-8 bytes; integers little-endian.

``GgufFile`` wraps tl_hip_gguf_* (the C++ reader of libtl_hip.so); ``write_llama_gguf`` stores
a synthetic decoder under the tensor names chatbot.tl reads.
"""
import ctypes as C
import struct

import numpy as np

from . import _lib
from .device import BackendError, HipTensor, _raise

GGUF_U32, GGUF_I32, GGUF_F32, GGUF_STRING, GGUF_U64 = 4, 5, 6, 8, 10


def _gstr(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(v):
    if isinstance(v, str):
        return struct.pack("<I", GGUF_STRING) + _gstr(v)
    if isinstance(v, float):
        return struct.pack("<If", GGUF_F32, v)
    if isinstance(v, (int, np.integer)):
        v = int(v)
        if 0 <= v < 2 ** 32:
            return struct.pack("<II", GGUF_U32, v)
        return struct.pack("<IQ", GGUF_U64, v)
    raise TypeError(f"metadata value {v!r}")


def write_gguf(path, tensors, metadata=None, alignment=32):
    """tensors: iterable of (name, ggml_type, row-major shape, bytes-like)."""
    metadata = dict(metadata or {})
    if alignment != 32:
        metadata["general.alignment"] = int(alignment)
    tensors = [(n, int(t), tuple(int(d) for d in shp), np.frombuffer(bytes(b) if not isinstance(b, np.ndarray)
                                                                      else b.tobytes(), np.uint8))
               for n, t, shp, b in tensors]
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata)))
    for k, v in metadata.items():
        head += _gstr(k) + _value(v)
    off = 0
    offsets = []
    for name, t, shp, data in tensors:
        offsets.append(off)
        ne = list(reversed(shp))
        head += _gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", t, off)
        off += -(-data.size // alignment) * alignment
    head += bytes((alignment - len(head) % alignment) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        for (name, t, shp, data), o in zip(tensors, offsets):
            f.write(data.tobytes())
            f.write(bytes(-(-data.size // alignment) * alignment - data.size))


def llama_tensor_names(cfg):
    """(name, kind, layer, slot) of every decoder tensor, as chatbot.tl reads them."""
    from .llama import SLOTS
    out = [("token_embd.weight", "embedding", -1, 0)]
    for l in range(cfg.n_layers):
        for i, s in enumerate(SLOTS):
            out.append((f"blk.{l}.{s}.weight", "linear", l, i))
        out.append((f"blk.{l}.attn_norm.weight", "norm", l, 0))
        out.append((f"blk.{l}.ffn_norm.weight", "norm", l, 1))
    out.append(("output_norm.weight", "norm", -1, 0))
    out.append(("output.weight", "linear", -1, 0))
    return out


def write_llama_gguf(path, cfg, tensors, ggml_type, embed_type=0):
    """Writes the (kind, layer, which, payload) tensors of ``synthetic_weights`` as a GGUF file:
    linears in their ggml types (``linear_type``), norms F32, the embedding in ``embed_type``
    (0 = F32, or a quantized type, encoded here), with llama.* metadata.  Returns the stored
    embedding: the f32 table, or (ggml type, blocks) when quantized."""
    from .llama import SLOTS, _QUANTIZERS, linear_type
    out, emb = [], None
    names = {(k, l, w): n for n, k, l, w in llama_tensor_names(cfg)}
    for kind, layer, which, payload in tensors:
        name = names[(kind, layer, which)]
        if kind == "embedding":
            tab = np.ascontiguousarray(payload, np.float32)
            if embed_type == 0:
                out.append((name, 0, tab.shape, tab.view(np.uint8)))
                emb = tab
            else:
                blocks = _QUANTIZERS[embed_type](tab)
                out.append((name, embed_type, tab.shape, blocks))
                emb = (embed_type, blocks)
        elif kind == "norm":
            v = np.ascontiguousarray(payload, np.float32)
            out.append((name, 0, v.shape, v.view(np.uint8)))
        else:
            slot = SLOTS[which] if layer >= 0 else "output"
            out.append((name, linear_type(ggml_type, cfg, layer, slot), cfg.linear_shape(slot), payload))
    meta = {"general.architecture": "llama", "llama.block_count": cfg.n_layers,
            "llama.embedding_length": cfg.d_model, "llama.feed_forward_length": cfg.ffn_dim,
            "llama.attention.head_count": cfg.n_heads, "llama.attention.head_count_kv": cfg.n_kv_heads,
            "llama.attention.layer_norm_rms_epsilon": float(cfg.eps), "llama.rope.freq_base": float(cfg.rope_theta),
            "llama.context_length": cfg.max_seq}
    write_gguf(path, out, meta)
    return emb


class GgufFile:
    """A GGUF file opened by tl_hip_gguf_open (the tensor map of tl_gguf_load)."""

    def __init__(self, path):
        self.lib = _lib.load()
        h = self.lib.tl_hip_gguf_open(str(path).encode())
        if not h:
            _raise(self.lib)
        self.h = h

    def names(self):
        return [self.lib.tl_hip_gguf_tensor_name(self.h, i).decode() for i in
                range(self.lib.tl_hip_gguf_tensor_count(self.h))]

    def info(self, name):
        t, r, nb = C.c_int(), C.c_int(), C.c_uint64()
        shp = (C.c_int64 * 8)()
        if self.lib.tl_hip_gguf_tensor_info(self.h, name.encode(), C.byref(t), shp, C.byref(r), C.byref(nb)):
            _raise(self.lib)
        return t.value, tuple(shp[:r.value]), nb.value

    def data(self, name):
        nb = C.c_uint64()
        p = self.lib.tl_hip_gguf_tensor_data(self.h, name.encode(), C.byref(nb))
        if not p:
            _raise(self.lib)
        return bytes(C.string_at(p, nb.value))

    def meta(self, key):
        v = C.c_double()
        if self.lib.tl_hip_gguf_meta_f64(self.h, key.encode(), C.byref(v)) == 0:
            return v.value
        self.lib.tl_hip_clear_error()
        s = self.lib.tl_hip_gguf_meta_str(self.h, key.encode())
        if s is None:
            _raise(self.lib)
        return s.decode()

    def get(self, name):
        """tl_tensor_map_get: an f32 device tensor (needs a GPU)."""
        p = self.lib.tl_hip_gguf_get(self.h, name.encode())
        if not p:
            _raise(self.lib)
        return HipTensor(p, self.lib)

    def close(self):
        if self.h:
            self.lib.tl_hip_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = ["write_gguf", "write_llama_gguf", "llama_tensor_names", "GgufFile", "BackendError"]
