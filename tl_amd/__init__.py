"""tl_amd -- tl_hip, the MI355X (gfx950) backend for TL's quantized LLM-inference path.

The product is the shared library libtl_hip.so (hand-written HIP kernels behind the C ABI of
include/tl_hip.h).  This package binds it (``_lib``), mirrors the reference's operator
interface on top of it (``device``), encodes GGUF blocks on the host (``quant``) and drives
the Llama decoder composition (``llama``).
"""
from .device import (BackendError, HipDevice, HipTensor, QTensor, GGML_Q4_0, GGML_Q8_0,  # noqa: F401
                     GGML_Q4_K, GGML_Q6_K)

__all__ = ["BackendError", "HipDevice", "HipTensor", "QTensor", "GGML_Q4_0", "GGML_Q8_0", "GGML_Q4_K",
           "GGML_Q6_K"]
