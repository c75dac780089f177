//! Rust declarations of the tl_hip C ABI (`include/tl_hip.h`), for a `tl_hip` crate in the
//! reference tree (`crates/tl_hip/src/ffi.rs`).  One `extern "C"` item per declaration of the
//! header, same order, names, arity and C types (`tests/test_ffi_decl.py` checks this file
//! against the header, in the manner of the reference's `scripts/check_ffi_signatures.py`).
//! The handle types are opaque: a `*mut tl_hip_tensor` is an owned reference (release with
//! `tl_hip_tensor_release`), `*const tl_hip_tensor` a borrowed one.
//!
//! Not compiled here (this image has no cargo); `device_impl.rs` beside it shows the `IDevice`
//! methods built on these declarations.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_void};

#[repr(C)]
pub struct tl_hip_tensor {
    _opaque: [u8; 0],
}
#[repr(C)]
pub struct tl_hip_qtensor {
    _opaque: [u8; 0],
}
#[repr(C)]
pub struct tl_hip_llama {
    _opaque: [u8; 0],
}
#[repr(C)]
pub struct tl_hip_gguf {
    _opaque: [u8; 0],
}

pub const TL_HIP_OK: i32 = 0;
pub const TL_HIP_ERR_SHAPE: i32 = 1;
pub const TL_HIP_ERR_DEVICE: i32 = 2;
pub const TL_HIP_ERR_ALLOC: i32 = 3;
pub const TL_HIP_ERR_NULL: i32 = 4;
pub const TL_HIP_ERR_INTERNAL: i32 = 5;
pub const TL_HIP_ERR_INDEX: i32 = 6;
pub const TL_HIP_ERR_TYPE: i32 = 7;
pub const TL_HIP_ERR_ARG: i32 = 8;
pub const TL_HIP_F32: i32 = 0;
pub const TL_HIP_F16: i32 = 1;
pub const TL_HIP_GGML_Q4_0: i32 = 2;
pub const TL_HIP_GGML_Q8_0: i32 = 8;
pub const TL_HIP_GGML_Q4_K: i32 = 12;
pub const TL_HIP_GGML_Q6_K: i32 = 14;
pub const TL_HIP_MAX_RANK: usize = 8;

#[link(name = "tl_hip")]
extern "C" {
    pub fn tl_hip_last_error() -> *const c_char;
    pub fn tl_hip_last_status() -> i32;
    pub fn tl_hip_clear_error();
    pub fn tl_hip_init(device: i32) -> i32;
    pub fn tl_hip_device_count() -> i32;
    pub fn tl_hip_stream() -> *mut c_void;
    pub fn tl_hip_set_stream(hip_stream: *mut c_void) -> i32;
    pub fn tl_hip_synchronize() -> i32;
    pub fn tl_hip_malloc(bytes: usize) -> *mut c_void;
    pub fn tl_hip_free(p: *mut c_void) -> i32;
    pub fn tl_hip_memcpy_h2d(dst: *mut c_void, src: *const c_void, bytes: usize) -> i32;
    pub fn tl_hip_memcpy_d2h(dst: *mut c_void, src: *const c_void, bytes: usize) -> i32;
    pub fn tl_hip_memcpy_d2d(dst: *mut c_void, src: *const c_void, bytes: usize) -> i32;
    pub fn tl_hip_event_create() -> *mut c_void;
    pub fn tl_hip_event_record(ev: *mut c_void) -> i32;
    pub fn tl_hip_event_elapsed_ms(start: *mut c_void, stop: *mut c_void, ms: *mut f32) -> i32;
    pub fn tl_hip_event_destroy(ev: *mut c_void) -> i32;
    pub fn tl_hip_stall(us: u32) -> i32;
    pub fn tl_hip_debug_fail_alloc(after: i64) -> i32;
    pub fn tl_hip_tensor_new(host: *const f32, shape: *const i64, rank: i32) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_new_f16(
        host: *const u16,
        shape: *const i64,
        rank: i32,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_zeros(shape: *const i64, rank: i32, dtype: i32) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_release(t: *mut tl_hip_tensor) -> i32;
    pub fn tl_hip_tensor_acquire(t: *mut tl_hip_tensor) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_to_host(t: *const tl_hip_tensor, out: *mut f32, numel: i64) -> i32;
    pub fn tl_hip_tensor_rank(t: *const tl_hip_tensor) -> i32;
    pub fn tl_hip_tensor_shape(t: *const tl_hip_tensor, shape_out: *mut i64) -> i32;
    pub fn tl_hip_tensor_numel(t: *const tl_hip_tensor) -> i64;
    pub fn tl_hip_tensor_dtype(t: *const tl_hip_tensor) -> i32;
    pub fn tl_hip_tensor_data(t: *const tl_hip_tensor) -> *mut c_void;
    pub fn tl_hip_tensor_reshape(
        t: *const tl_hip_tensor,
        shape: *const i64,
        rank: i32,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_qtensor_new(
        ggml_type: i32,
        data: *const u8,
        nbytes: usize,
        shape: *const i64,
        rank: i32,
    ) -> *mut tl_hip_qtensor;
    pub fn tl_hip_qtensor_release(q: *mut tl_hip_qtensor) -> i32;
    pub fn tl_hip_qtensor_dequantize(q: *const tl_hip_qtensor) -> *mut tl_hip_tensor;
    pub fn tl_hip_qtensor_matmul(
        x: *const tl_hip_tensor,
        q: *const tl_hip_qtensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_qtensor_matmul_f16(
        x: *const tl_hip_tensor,
        q: *const tl_hip_qtensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_gguf_open(path: *const c_char) -> *mut tl_hip_gguf;
    pub fn tl_hip_gguf_close(g: *mut tl_hip_gguf) -> i32;
    pub fn tl_hip_gguf_tensor_count(g: *const tl_hip_gguf) -> i64;
    pub fn tl_hip_gguf_tensor_name(g: *const tl_hip_gguf, i: i64) -> *const c_char;
    pub fn tl_hip_gguf_tensor_info(
        g: *const tl_hip_gguf,
        name: *const c_char,
        ggml_type: *mut i32,
        shape: *mut i64,
        rank: *mut i32,
        nbytes: *mut u64,
    ) -> i32;
    pub fn tl_hip_gguf_tensor_data(
        g: *const tl_hip_gguf,
        name: *const c_char,
        nbytes: *mut u64,
    ) -> *const u8;
    pub fn tl_hip_gguf_meta_f64(g: *const tl_hip_gguf, key: *const c_char, out: *mut f64) -> i32;
    pub fn tl_hip_gguf_meta_str(g: *const tl_hip_gguf, key: *const c_char) -> *const c_char;
    pub fn tl_hip_gguf_get_quantized(
        g: *mut tl_hip_gguf,
        name: *const c_char,
    ) -> *mut tl_hip_qtensor;
    pub fn tl_hip_gguf_get(g: *mut tl_hip_gguf, name: *const c_char) -> *mut tl_hip_tensor;
    pub fn tl_hip_launch_quant_matvec(
        w: *const tl_hip_qtensor,
        x: *const f32,
        y: *mut f32,
        m: i64,
        stream: *mut c_void,
    ) -> i32;
    pub fn tl_hip_launch_quant_gemm(
        w: *const tl_hip_qtensor,
        x: *const f32,
        y: *mut f32,
        m: i64,
        use_f16_mfma: i32,
        stream: *mut c_void,
    ) -> i32;
    pub fn tl_hip_read_floor(w: *const tl_hip_qtensor, stream: *mut c_void) -> i32;
    pub fn tl_hip_launch_quant_gemm_noalloc(
        w: *const tl_hip_qtensor,
        x: *const f32,
        y: *mut f32,
        m: i64,
        use_f16_mfma: i32,
        stream: *mut c_void,
    ) -> i32;
    pub fn tl_hip_debug_last_gemm_plan(
        tile_m: *mut i32,
        tile_n: *mut i32,
        k_splits: *mut i32,
    ) -> i32;
    pub fn tl_hip_tensor_matmul(
        a: *const tl_hip_tensor,
        b: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_transpose_2d(a: *const tl_hip_tensor) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_transpose(
        a: *const tl_hip_tensor,
        dim0: i64,
        dim1: i64,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_rms_norm(
        x: *const tl_hip_tensor,
        w: *const tl_hip_tensor,
        eps: f32,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_rope_new_cos(dim: i64, seq_len: i64, base: f32) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_rope_new_sin(dim: i64, seq_len: i64, base: f32) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_apply_rope(
        x: *const tl_hip_tensor,
        cos_t: *const tl_hip_tensor,
        sin_t: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_apply_rope_pos(
        x: *const tl_hip_tensor,
        cos_t: *const tl_hip_tensor,
        sin_t: *const tl_hip_tensor,
        pos0: i64,
        vectors_per_token: i64,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_silu(x: *const tl_hip_tensor) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_add(
        a: *const tl_hip_tensor,
        b: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_mul(
        a: *const tl_hip_tensor,
        b: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_sub(
        a: *const tl_hip_tensor,
        b: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_div(
        a: *const tl_hip_tensor,
        b: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_scale(x: *const tl_hip_tensor, s: f32) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_softmax(x: *const tl_hip_tensor, dim: i64) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_new_causal_mask(size: i64) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_narrow(
        x: *const tl_hip_tensor,
        dim: i64,
        start: i64,
        len: i64,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_cat(
        a: *const tl_hip_tensor,
        b: *const tl_hip_tensor,
        dim: i64,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_repeat_interleave(
        x: *const tl_hip_tensor,
        repeats: i64,
        dim: i64,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_embedding(
        weight: *const tl_hip_tensor,
        ids: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_sample(
        logits: *const tl_hip_tensor,
        temp: f32,
        top_p: f32,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_sample_uniform(
        logits: *const tl_hip_tensor,
        temp: f32,
        top_p: f32,
        u: f64,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_sample_seed(seed: u64);
    pub fn tl_hip_tensor_argmax_all(x: *const tl_hip_tensor) -> i64;
    pub fn tl_hip_tensor_repetition_penalty(
        logits: *const tl_hip_tensor,
        tokens: *const tl_hip_tensor,
        penalty: f64,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_fused_silu_mul(
        gate: *const tl_hip_tensor,
        up: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_fused_rms_norm(
        x: *const tl_hip_tensor,
        w: *const tl_hip_tensor,
        eps: f32,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_fused_add_rms_norm(
        x: *const tl_hip_tensor,
        residual: *const tl_hip_tensor,
        w: *const tl_hip_tensor,
        eps: f32,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_fused_rotary_emb(
        x: *const tl_hip_tensor,
        freqs: *const tl_hip_tensor,
        head_dim: i64,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_fused_add_relu(
        a: *const tl_hip_tensor,
        b: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_fused_bias_gelu(
        x: *const tl_hip_tensor,
        bias: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_tensor_scaled_dot_product_attention(
        q: *const tl_hip_tensor,
        k: *const tl_hip_tensor,
        v: *const tl_hip_tensor,
        mask: *const tl_hip_tensor,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_attention_decode(
        q: *const tl_hip_tensor,
        k: *const tl_hip_tensor,
        v: *const tl_hip_tensor,
        L: i64,
        scale: f32,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_debug_one_launch_merge(on: i32) -> i32;
    pub fn tl_hip_debug_prefill_rope_epilogue(on: i32) -> i32;
    pub fn tl_hip_attention_prefill(
        q: *const tl_hip_tensor,
        k: *const tl_hip_tensor,
        v: *const tl_hip_tensor,
        pos0: i64,
        scale: f32,
    ) -> *mut tl_hip_tensor;
    pub fn tl_hip_llama_new(
        n_layers: i32,
        d_model: i32,
        n_heads: i32,
        n_kv_heads: i32,
        ffn_dim: i32,
        vocab: i32,
        eps: f32,
        rope_theta: f32,
        max_seq: i32,
    ) -> *mut tl_hip_llama;
    pub fn tl_hip_llama_free(m: *mut tl_hip_llama) -> i32;
    pub fn tl_hip_llama_set_linear(
        m: *mut tl_hip_llama,
        layer: i32,
        which: i32,
        ggml_type: i32,
        data: *const u8,
        nbytes: usize,
    ) -> i32;
    pub fn tl_hip_llama_set_norm(
        m: *mut tl_hip_llama,
        layer: i32,
        which: i32,
        w: *const f32,
    ) -> i32;
    pub fn tl_hip_llama_set_embedding(m: *mut tl_hip_llama, table: *const f32) -> i32;
    pub fn tl_hip_llama_load_gguf(m: *mut tl_hip_llama, g: *mut tl_hip_gguf) -> i32;
    pub fn tl_hip_llama_configure(m: *mut tl_hip_llama, kv_f16: i32, rope_per_token: i32) -> i32;
    pub fn tl_hip_llama_reset(m: *mut tl_hip_llama) -> i32;
    pub fn tl_hip_llama_position(m: *const tl_hip_llama) -> i64;
    pub fn tl_hip_llama_graph_builds(m: *const tl_hip_llama) -> i64;
    pub fn tl_hip_llama_forward(
        m: *mut tl_hip_llama,
        ids: *const i32,
        n: i32,
        logits_out: *mut f32,
        prefill_f16: i32,
    ) -> i32;
    pub fn tl_hip_llama_sample_greedy(
        m: *mut tl_hip_llama,
        repetition_penalty: f64,
        history: *const i32,
        n_history: i32,
    ) -> i32;
    pub fn tl_hip_llama_sample(
        m: *mut tl_hip_llama,
        temp: f32,
        top_p: f32,
        repetition_penalty: f64,
        history: *const i32,
        n_history: i32,
    ) -> i32;
    pub fn tl_hip_llama_set_sampling(m: *mut tl_hip_llama, temp: f32, top_p: f32) -> i32;
    pub fn tl_hip_llama_generate(
        m: *mut tl_hip_llama,
        first: i32,
        n_steps: i32,
        out_ids: *mut i32,
        repetition_penalty: f64,
        history: *const i32,
        n_history: i32,
        use_graph: i32,
    ) -> i32;
}
