"""ctypes binding of libtl_hip.so (declarations in include/tl_hip.h).

Loading fails loudly when the library has not been built: there is no fallback path.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtl_hip.so")

P = C.c_void_p
i32, i64, f32, f64, sz = C.c_int, C.c_int64, C.c_float, C.c_double, C.c_size_t
u8p = C.POINTER(C.c_uint8)
i64p = C.POINTER(C.c_int64)
i32p = C.POINTER(C.c_int32)
f32p = C.POINTER(C.c_float)
u16p = C.POINTER(C.c_uint16)

# name: (restype, argtypes)
PROTOS = {
    "tl_hip_last_error": (C.c_char_p, []),
    "tl_hip_last_status": (i32, []),
    "tl_hip_clear_error": (None, []),
    "tl_hip_init": (i32, [i32]),
    "tl_hip_device_count": (i32, []),
    "tl_hip_stream": (P, []),
    "tl_hip_set_stream": (i32, [P]),
    "tl_hip_synchronize": (i32, []),
    "tl_hip_malloc": (P, [sz]),
    "tl_hip_free": (i32, [P]),
    "tl_hip_memcpy_h2d": (i32, [P, P, sz]),
    "tl_hip_memcpy_d2h": (i32, [P, P, sz]),
    "tl_hip_memcpy_d2d": (i32, [P, P, sz]),
    "tl_hip_event_create": (P, []),
    "tl_hip_event_record": (i32, [P]),
    "tl_hip_event_elapsed_ms": (i32, [P, P, f32p]),
    "tl_hip_event_destroy": (i32, [P]),
    "tl_hip_stall": (i32, [C.c_uint32]),
    "tl_hip_debug_fail_alloc": (i32, [i64]),
    "tl_hip_tensor_new": (P, [f32p, i64p, i32]),
    "tl_hip_tensor_new_f16": (P, [u16p, i64p, i32]),
    "tl_hip_tensor_zeros": (P, [i64p, i32, i32]),
    "tl_hip_tensor_release": (i32, [P]),
    "tl_hip_tensor_acquire": (P, [P]),
    "tl_hip_tensor_to_host": (i32, [P, f32p, i64]),
    "tl_hip_tensor_rank": (i32, [P]),
    "tl_hip_tensor_shape": (i32, [P, i64p]),
    "tl_hip_tensor_numel": (i64, [P]),
    "tl_hip_tensor_dtype": (i32, [P]),
    "tl_hip_tensor_data": (P, [P]),
    "tl_hip_tensor_reshape": (P, [P, i64p, i32]),
    "tl_hip_qtensor_new": (P, [i32, u8p, sz, i64p, i32]),
    "tl_hip_qtensor_release": (i32, [P]),
    "tl_hip_qtensor_dequantize": (P, [P]),
    "tl_hip_qtensor_matmul": (P, [P, P]),
    "tl_hip_qtensor_matmul_f16": (P, [P, P]),
    "tl_hip_gguf_open": (P, [C.c_char_p]),
    "tl_hip_gguf_close": (i32, [P]),
    "tl_hip_gguf_tensor_count": (i64, [P]),
    "tl_hip_gguf_tensor_name": (C.c_char_p, [P, i64]),
    "tl_hip_gguf_tensor_info": (i32, [P, C.c_char_p, C.POINTER(i32), i64p, C.POINTER(i32),
                                      C.POINTER(C.c_uint64)]),
    "tl_hip_gguf_tensor_data": (P, [P, C.c_char_p, C.POINTER(C.c_uint64)]),
    "tl_hip_gguf_meta_f64": (i32, [P, C.c_char_p, C.POINTER(f64)]),
    "tl_hip_gguf_meta_str": (C.c_char_p, [P, C.c_char_p]),
    "tl_hip_gguf_get_quantized": (P, [P, C.c_char_p]),
    "tl_hip_gguf_get": (P, [P, C.c_char_p]),
    "tl_hip_llama_load_gguf": (i32, [P, P]),
    "tl_hip_launch_quant_matvec": (i32, [P, P, P, i64, P]),
    "tl_hip_launch_quant_gemm": (i32, [P, P, P, i64, i32, P]),
    "tl_hip_launch_quant_gemm_noalloc": (i32, [P, P, P, i64, i32, P]),
    "tl_hip_read_floor": (i32, [P, P]),
    "tl_hip_debug_last_gemm_plan": (i32, [i32p, i32p, i32p]),
    "tl_hip_tensor_matmul": (P, [P, P]),
    "tl_hip_tensor_transpose_2d": (P, [P]),
    "tl_hip_tensor_transpose": (P, [P, i64, i64]),
    "tl_hip_tensor_rms_norm": (P, [P, P, f32]),
    "tl_hip_tensor_rope_new_cos": (P, [i64, i64, f32]),
    "tl_hip_tensor_rope_new_sin": (P, [i64, i64, f32]),
    "tl_hip_tensor_apply_rope": (P, [P, P, P]),
    "tl_hip_tensor_apply_rope_pos": (P, [P, P, P, i64, i64]),
    "tl_hip_tensor_silu": (P, [P]),
    "tl_hip_tensor_add": (P, [P, P]),
    "tl_hip_tensor_mul": (P, [P, P]),
    "tl_hip_tensor_sub": (P, [P, P]),
    "tl_hip_tensor_div": (P, [P, P]),
    "tl_hip_tensor_scale": (P, [P, f32]),
    "tl_hip_tensor_softmax": (P, [P, i64]),
    "tl_hip_tensor_new_causal_mask": (P, [i64]),
    "tl_hip_tensor_narrow": (P, [P, i64, i64, i64]),
    "tl_hip_tensor_cat": (P, [P, P, i64]),
    "tl_hip_tensor_repeat_interleave": (P, [P, i64, i64]),
    "tl_hip_tensor_embedding": (P, [P, P]),
    "tl_hip_tensor_sample": (P, [P, f32, f32]),
    "tl_hip_tensor_sample_uniform": (P, [P, f32, f32, f64]),
    "tl_hip_sample_seed": (None, [C.c_uint64]),
    "tl_hip_tensor_argmax_all": (i64, [P]),
    "tl_hip_tensor_repetition_penalty": (P, [P, P, f64]),
    "tl_hip_fused_silu_mul": (P, [P, P]),
    "tl_hip_fused_rotary_emb": (P, [P, P, i64]),
    "tl_hip_fused_add_relu": (P, [P, P]),
    "tl_hip_fused_bias_gelu": (P, [P, P]),
    "tl_hip_fused_rms_norm": (P, [P, P, f32]),
    "tl_hip_fused_add_rms_norm": (P, [P, P, P, f32]),
    "tl_hip_tensor_scaled_dot_product_attention": (P, [P, P, P, P]),
    "tl_hip_attention_decode": (P, [P, P, P, i64, f32]),
    "tl_hip_debug_one_launch_merge": (i32, [i32]),
    "tl_hip_debug_prefill_rope_epilogue": (i32, [i32]),
    "tl_hip_attention_prefill": (P, [P, P, P, i64, f32]),
    "tl_hip_llama_new": (P, [i32, i32, i32, i32, i32, i32, f32, f32, i32]),
    "tl_hip_llama_free": (i32, [P]),
    "tl_hip_llama_set_linear": (i32, [P, i32, i32, i32, u8p, sz]),
    "tl_hip_llama_set_norm": (i32, [P, i32, i32, f32p]),
    "tl_hip_llama_set_embedding": (i32, [P, f32p]),
    "tl_hip_llama_configure": (i32, [P, i32, i32]),
    "tl_hip_llama_reset": (i32, [P]),
    "tl_hip_llama_position": (i64, [P]),
    "tl_hip_llama_graph_builds": (i64, [P]),
    "tl_hip_llama_forward": (i32, [P, i32p, i32, f32p, i32]),
    "tl_hip_llama_sample_greedy": (C.c_int32, [P, f64, i32p, i32]),
    "tl_hip_llama_sample": (C.c_int32, [P, f32, f32, f64, i32p, i32]),
    "tl_hip_llama_set_sampling": (i32, [P, f32, f32]),
    "tl_hip_llama_generate": (i32, [P, C.c_int32, i32, i32p, f64, i32p, i32, i32]),
}

_lib = None


def load():
    """Returns the loaded library with prototypes applied (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m tl_amd.build` "
            "(tl_hip has no CPU fallback)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
