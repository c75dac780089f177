"""Host-side mirror of the reference's operator interface over the tl_hip C ABI.

``HipDevice`` carries the IDevice method names of the quantized-inference path
(crates/tl_backend/src/device.rs), ``HipTensor`` is the GpuTensor handle, ``QTensor`` the
quantized weight (crates/tl_runtime/src/quantized.rs:29-40) and ``tl_qtensor_matmul`` the
drop-in entry of the path (crates/tl_runtime/src/system.rs:180-382).  Errors surface as
``BackendError`` carrying the BackendError variant and message (error.rs:7-17), where the
reference returns NULL and stores the message in LAST_ERROR (device_ffi.rs:22-80).
"""
import ctypes as C

import numpy as np

from . import _lib

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 8, 12, 14
F32, F16 = 0, 1

_VARIANTS = {
    1: "ShapeMismatch", 2: "DeviceError", 3: "AllocationError", 4: "NullPointerError",
    5: "InternalError", 6: "IndexOutOfBounds", 7: "TypeMismatch", 8: "ArgumentError",
}


class BackendError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(message)
        self.status = status
        self.variant = _VARIANTS.get(status, "Unknown")


def _raise(lib):
    msg = lib.tl_hip_last_error().decode(errors="replace")
    raise BackendError(lib.tl_hip_last_status(), msg)


def _shape_arr(shape):
    return (C.c_int64 * max(1, len(shape)))(*[int(s) for s in shape])


class HipTensor:
    """Owned device tensor handle (reference count 1 on creation, released on drop)."""

    __slots__ = ("_h", "_lib")

    def __init__(self, handle, lib):
        self._h = handle
        self._lib = lib

    @property
    def handle(self):
        return self._h

    @property
    def shape(self):
        r = self._lib.tl_hip_tensor_rank(self._h)
        out = (C.c_int64 * max(1, r))()
        self._lib.tl_hip_tensor_shape(self._h, out)
        return tuple(out[i] for i in range(r))

    @property
    def numel(self):
        return int(self._lib.tl_hip_tensor_numel(self._h))

    @property
    def data_ptr(self):
        return self._lib.tl_hip_tensor_data(self._h)

    def to_numpy(self):
        """tensor_to_vec_f32 (device.rs:83), reshaped (f16 tensors are widened)."""
        n = self.numel
        out = np.empty(max(n, 1), dtype=np.float32)
        rc = self._lib.tl_hip_tensor_to_host(self._h, out.ctypes.data_as(_lib.f32p), n)
        if rc:
            _raise(self._lib)
        return out[:n].reshape(self.shape)

    def release(self):
        if self._h:
            self._lib.tl_hip_tensor_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class QTensor:
    """QTensor (quantized.rs:29-40): raw GGUF block bytes + row-major shape [n, k] + ggml type.

    ``upload`` builds the device residency (the gpu_raw_cache role, system.rs:316-331)."""

    def __init__(self, ggml_type, data, shape):
        self.ggml_type = int(ggml_type)
        self.data = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8)) \
            if not isinstance(data, np.ndarray) else np.ascontiguousarray(data, dtype=np.uint8)
        self.shape = tuple(int(s) for s in shape)
        self._h = None
        self._lib = None

    def upload(self, lib):
        if self._h is None:
            h = lib.tl_hip_qtensor_new(self.ggml_type, self.data.ctypes.data_as(_lib.u8p),
                                       self.data.nbytes, _shape_arr(self.shape), len(self.shape))
            if not h:
                _raise(lib)
            self._h, self._lib = h, lib
        return self._h

    def release(self):
        if self._h:
            self._lib.tl_hip_qtensor_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class HipDevice:
    """IDevice for TL_DEVICE=hip, restricted to the quantized LLM-inference path."""

    def __init__(self, device=0):
        self.lib = _lib.load()
        if self.lib.tl_hip_init(device):
            _raise(self.lib)

    # -- helpers
    def _wrap(self, h):
        if not h:
            _raise(self.lib)
        return HipTensor(h, self.lib)

    def _check(self, rc):
        if rc:
            _raise(self.lib)

    def synchronize(self):
        self._check(self.lib.tl_hip_synchronize())

    # -- creation (device.rs:21-53)
    def tensor_new(self, array):
        a = np.ascontiguousarray(array, dtype=np.float32)
        return self._wrap(self.lib.tl_hip_tensor_new(a.ctypes.data_as(_lib.f32p), _shape_arr(a.shape), a.ndim))

    def tensor_new_f16(self, array):
        a = np.ascontiguousarray(array, dtype=np.float16)
        return self._wrap(self.lib.tl_hip_tensor_new_f16(a.view(np.uint16).ctypes.data_as(_lib.u16p),
                                                         _shape_arr(a.shape), a.ndim))

    def tensor_zeros(self, shape, dtype=F32):
        return self._wrap(self.lib.tl_hip_tensor_zeros(_shape_arr(shape), len(shape), dtype))

    def tensor_new_causal_mask(self, size):
        return self._wrap(self.lib.tl_hip_tensor_new_causal_mask(size))

    def tensor_reshape(self, t, shape):
        return self._wrap(self.lib.tl_hip_tensor_reshape(t.handle, _shape_arr(shape), len(shape)))

    # -- quantized path (quantized.rs:117-165; system.rs:180-382)
    def qtensor_dequantize(self, q):
        return self._wrap(self.lib.tl_hip_qtensor_dequantize(q.upload(self.lib)))

    def tl_qtensor_matmul(self, x, q):
        return self._wrap(self.lib.tl_hip_qtensor_matmul(x.handle, q.upload(self.lib)))

    def tl_qtensor_matmul_f16(self, x, q):
        return self._wrap(self.lib.tl_hip_qtensor_matmul_f16(x.handle, q.upload(self.lib)))

    # -- operators (device.rs)
    def tensor_matmul(self, a, b):
        return self._wrap(self.lib.tl_hip_tensor_matmul(a.handle, b.handle))

    def tensor_transpose_2d(self, a):
        return self._wrap(self.lib.tl_hip_tensor_transpose_2d(a.handle))

    def tensor_transpose(self, a, d0, d1):
        return self._wrap(self.lib.tl_hip_tensor_transpose(a.handle, d0, d1))

    def tensor_rms_norm(self, x, w, eps):
        return self._wrap(self.lib.tl_hip_tensor_rms_norm(x.handle, w.handle if w is not None else None, eps))

    def tensor_rope_new_cos(self, dim, seq_len, base):
        return self._wrap(self.lib.tl_hip_tensor_rope_new_cos(dim, seq_len, base))

    def tensor_rope_new_sin(self, dim, seq_len, base):
        return self._wrap(self.lib.tl_hip_tensor_rope_new_sin(dim, seq_len, base))

    def tensor_apply_rope(self, x, cos, sin):
        return self._wrap(self.lib.tl_hip_tensor_apply_rope(x.handle, cos.handle, sin.handle))

    def tensor_apply_rope_pos(self, x, cos, sin, pos0, vectors_per_token):
        return self._wrap(self.lib.tl_hip_tensor_apply_rope_pos(x.handle, cos.handle, sin.handle, pos0,
                                                                vectors_per_token))

    def tensor_silu(self, x):
        return self._wrap(self.lib.tl_hip_tensor_silu(x.handle))

    def tensor_add(self, a, b):
        return self._wrap(self.lib.tl_hip_tensor_add(a.handle, b.handle))

    def tensor_mul(self, a, b):
        return self._wrap(self.lib.tl_hip_tensor_mul(a.handle, b.handle))

    def tensor_sub(self, a, b):
        return self._wrap(self.lib.tl_hip_tensor_sub(a.handle, b.handle))

    def tensor_div(self, a, b):
        return self._wrap(self.lib.tl_hip_tensor_div(a.handle, b.handle))

    def tensor_scale(self, x, s):
        return self._wrap(self.lib.tl_hip_tensor_scale(x.handle, s))

    def tensor_softmax(self, x, dim):
        return self._wrap(self.lib.tl_hip_tensor_softmax(x.handle, dim))

    def tensor_narrow(self, x, dim, start, length):
        return self._wrap(self.lib.tl_hip_tensor_narrow(x.handle, dim, start, length))

    def tensor_cat(self, a, b, dim):
        return self._wrap(self.lib.tl_hip_tensor_cat(a.handle, b.handle, dim))

    def tensor_repeat_interleave(self, x, repeats, dim):
        return self._wrap(self.lib.tl_hip_tensor_repeat_interleave(x.handle, repeats, dim))

    def tensor_embedding(self, weight, indices):
        return self._wrap(self.lib.tl_hip_tensor_embedding(weight.handle, indices.handle))

    def tensor_sample(self, logits, temp, top_p):
        return self._wrap(self.lib.tl_hip_tensor_sample(logits.handle, temp, top_p))

    def tensor_sample_uniform(self, logits, temp, top_p, u):
        return self._wrap(self.lib.tl_hip_tensor_sample_uniform(logits.handle, temp, top_p, u))

    def sample_seed(self, seed):
        self.lib.tl_hip_sample_seed(seed)

    def tensor_argmax_all(self, x):
        r = self.lib.tl_hip_tensor_argmax_all(x.handle)
        if r < 0:
            _raise(self.lib)
        return int(r)

    def tensor_repetition_penalty(self, logits, tokens, penalty):
        return self._wrap(self.lib.tl_hip_tensor_repetition_penalty(logits.handle, tokens.handle, penalty))

    # -- GpuFusedOps (fused_ops.rs:15-57)
    def fused_silu_mul(self, gate, up):
        return self._wrap(self.lib.tl_hip_fused_silu_mul(gate.handle, up.handle))

    def fused_rms_norm(self, x, w, eps):
        return self._wrap(self.lib.tl_hip_fused_rms_norm(x.handle, w.handle, eps))

    def fused_add_rms_norm(self, x, residual, w, eps):
        return self._wrap(self.lib.tl_hip_fused_add_rms_norm(x.handle, residual.handle, w.handle, eps))

    def fused_rotary_emb(self, x, freqs, head_dim):
        return self._wrap(self.lib.tl_hip_fused_rotary_emb(x.handle, freqs.handle, head_dim))

    def fused_add_relu(self, a, b):
        return self._wrap(self.lib.tl_hip_fused_add_relu(a.handle, b.handle))

    def fused_bias_gelu(self, x, bias):
        return self._wrap(self.lib.tl_hip_fused_bias_gelu(x.handle, bias.handle))

    def tensor_scaled_dot_product_attention(self, q, k, v, mask=None):
        """IDevice::tensor_scaled_dot_product_attention (device.rs:180-186): softmax(q k^T /
        sqrt(d_k), mask == 0 -> -1e9) v over [batch, heads,] seq, dim tensors."""
        return self._wrap(self.lib.tl_hip_tensor_scaled_dot_product_attention(
            q.handle, k.handle, v.handle, mask.handle if mask is not None else None))

    # -- decode attention over a KV cache
    def attention_decode(self, q, k, v, length, scale):
        return self._wrap(self.lib.tl_hip_attention_decode(q.handle, k.handle, v.handle, length, scale))

    def attention_prefill(self, q, k, v, pos0, scale):
        """Causal prefill attention (chatbot.tl:76-87 for sl > 1): q [n, Hq, D] f32 at positions
        pos0 .. pos0 + n - 1, k / v [Hkv, Lmax, D] f16 caches -> [n, Hq, D] f32."""
        return self._wrap(self.lib.tl_hip_attention_prefill(q.handle, k.handle, v.handle, pos0, scale))
