//! `IDevice` (crates/tl_backend/src/device.rs:19-524) for tl_hip: the methods of the quantized
//! inference path, each one call into the C ABI declared in `tl_hip_ffi.rs`.  Goes to
//! `crates/tl_hip/src/device_impl.rs` in the reference tree; not compiled here (no cargo).
//!
//! Conventions carried over from the reference backends:
//!   * a NULL result becomes the `BackendError` variant named by the thread-local status, with
//!     the thread-local message (error.rs:7-17; the LAST_ERROR convention of
//!     device_ffi.rs:22-80);
//!   * every tensor-returning call hands back a new handle with reference count 1, inputs are
//!     borrowed (ffi_helpers.rs:43-66);
//!   * where an `IDevice` method's argument order or width differs from the C entry (usize
//!     shapes, `req_grad` flags, embedding options), the adapter converts here, so the C ABI
//!     keeps one convention (i64 shapes, rank after shape).
//! Methods outside the path (autograd, CNN, IO, ...) return
//! `BackendError::InternalError("not provided by tl_hip")`.

use std::ffi::{c_void, CStr};

use tl_backend::error::{BackendError, BackendResult};

use crate::ffi;

pub struct HipDevice;

fn err_from_status() -> BackendError {
    let msg = unsafe { CStr::from_ptr(ffi::tl_hip_last_error()) }.to_string_lossy().into_owned();
    match unsafe { ffi::tl_hip_last_status() } {
        ffi::TL_HIP_ERR_SHAPE => BackendError::ShapeMismatch(msg),
        ffi::TL_HIP_ERR_DEVICE => BackendError::DeviceError(msg),
        ffi::TL_HIP_ERR_ALLOC => BackendError::AllocationError(msg),
        ffi::TL_HIP_ERR_NULL => BackendError::NullPointerError(msg),
        ffi::TL_HIP_ERR_INDEX => BackendError::IndexOutOfBounds(msg),
        ffi::TL_HIP_ERR_TYPE => BackendError::TypeMismatch(msg),
        ffi::TL_HIP_ERR_ARG => BackendError::ArgumentError(msg),
        _ => BackendError::InternalError(msg),
    }
}

fn check(p: *mut ffi::tl_hip_tensor) -> BackendResult<*mut c_void> {
    if p.is_null() {
        Err(err_from_status())
    } else {
        Ok(p as *mut c_void)
    }
}

fn status(rc: i32) -> BackendResult<()> {
    if rc == ffi::TL_HIP_OK {
        Ok(())
    } else {
        Err(err_from_status())
    }
}

#[inline]
fn h(t: *mut c_void) -> *const ffi::tl_hip_tensor {
    t as *const ffi::tl_hip_tensor
}

/// `*const usize` shapes of IDevice -> the i64 shape array of the C ABI.
fn shape_i64(rank: usize, shape: *const usize) -> BackendResult<Vec<i64>> {
    if rank > ffi::TL_HIP_MAX_RANK || (rank > 0 && shape.is_null()) {
        return Err(BackendError::ArgumentError(format!("rank {} or shape pointer invalid", rank)));
    }
    Ok((0..rank).map(|i| unsafe { *shape.add(i) } as i64).collect())
}

fn not_provided<T>(what: &str) -> BackendResult<T> {
    Err(BackendError::InternalError(format!("{} is not provided by tl_hip", what)))
}

impl HipDevice {
    // ========== creation (device.rs:21-53) ==========
    /// device.rs:21-26 tensor_new(data, rank, shape): the C entry takes (data, shape, rank).
    pub fn tensor_new(&self, data: *const f32, rank: usize, shape: *const usize) -> BackendResult<*mut c_void> {
        let s = shape_i64(rank, shape)?;
        check(unsafe { ffi::tl_hip_tensor_new(data, s.as_ptr(), rank as i32) })
    }

    /// device.rs:34-39 tensor_zeros(rank, shape, req_grad): tl_hip has no autograd, so a
    /// gradient-tracking request is an error rather than silently ignored.
    pub fn tensor_zeros(&self, rank: usize, shape: *const usize, req_grad: bool) -> BackendResult<*mut c_void> {
        if req_grad {
            return not_provided("autograd (req_grad = true)");
        }
        let s = shape_i64(rank, shape)?;
        check(unsafe { ffi::tl_hip_tensor_zeros(s.as_ptr(), rank as i32, ffi::TL_HIP_F32) })
    }

    /// device.rs:53 tensor_new_causal_mask(size)
    pub fn tensor_new_causal_mask(&self, size: usize) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_new_causal_mask(size as i64) })
    }

    // ========== to host (device.rs:83) ==========
    /// The vector is handed over as (pointer, length) of a leaked `Vec<f32>`, as tl_cpu does
    /// (tl_cpu device_impl.rs:151-158).
    pub fn tensor_to_vec_f32(&self, t: *mut c_void) -> BackendResult<(*mut f32, usize)> {
        let n = unsafe { ffi::tl_hip_tensor_numel(h(t)) };
        if n < 0 {
            return Err(err_from_status());
        }
        let mut v = vec![0.0f32; n as usize];
        status(unsafe { ffi::tl_hip_tensor_to_host(h(t), v.as_mut_ptr(), n) })?;
        let out = (v.as_mut_ptr(), v.len());
        std::mem::forget(v);
        Ok(out)
    }

    // ========== lifetime (device.rs:213-214) ==========
    pub fn tensor_release(&self, t: *mut c_void) -> BackendResult<()> {
        status(unsafe { ffi::tl_hip_tensor_release(t as *mut ffi::tl_hip_tensor) })
    }
    pub fn tensor_acquire(&self, t: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_acquire(t as *mut ffi::tl_hip_tensor) })
    }

    // ========== element-wise and products (device.rs:253-285, 310) ==========
    pub fn tensor_add(&self, a: *mut c_void, b: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_add(h(a), h(b)) })
    }
    pub fn tensor_sub(&self, a: *mut c_void, b: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_sub(h(a), h(b)) })
    }
    pub fn tensor_mul(&self, a: *mut c_void, b: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_mul(h(a), h(b)) })
    }
    pub fn tensor_div(&self, a: *mut c_void, b: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_div(h(a), h(b)) })
    }
    pub fn tensor_matmul(&self, a: *mut c_void, b: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_matmul(h(a), h(b)) })
    }
    pub fn tensor_scale(&self, t: *mut c_void, s: f32) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_scale(h(t), s) })
    }
    pub fn tensor_silu(&self, t: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_silu(h(t)) })
    }
    pub fn tensor_softmax(&self, t: *mut c_void, dim: i64) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_softmax(h(t), dim) })
    }
    /// device.rs:349 tensor_sample(t, temp, top_p): greedy for temp <= 0, else top-p
    /// sampling with the library's per-thread uniform draw (tl_hip_sample_seed fixes it).
    pub fn tensor_sample(&self, t: *mut c_void, temp: f32, top_p: f32) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_sample(h(t), temp, top_p) })
    }
    /// device.rs:194-199.  `tokens` holds the token ids as f32 (tl_hip tensors are f32 / f16);
    /// a runtime that keeps ids as i64 converts them with tensor_new first.
    pub fn tensor_repetition_penalty(
        &self,
        logits: *mut c_void,
        tokens: *mut c_void,
        penalty: f64,
    ) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_repetition_penalty(h(logits), h(tokens), penalty) })
    }
    /// device.rs:180-186
    pub fn tensor_scaled_dot_product_attention(
        &self,
        q: *mut c_void,
        k: *mut c_void,
        v: *mut c_void,
        mask: *mut c_void,
    ) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_scaled_dot_product_attention(h(q), h(k), h(v), h(mask)) })
    }

    // ========== shape ops (device.rs:367-425, 513-522) ==========
    /// device.rs:367-371 tensor_reshape_new(t, new_shape): the shape arrives as a tensor of
    /// f32 dims (tl_cpu ffi.rs:1408-1422 casts each to usize).
    pub fn tensor_reshape_new(&self, t: *mut c_void, new_shape: *mut c_void) -> BackendResult<*mut c_void> {
        let (p, n) = self.tensor_to_vec_f32(new_shape)?;
        let dims = unsafe { Vec::from_raw_parts(p, n, n) };
        let s: Vec<i64> = dims.iter().map(|&d| d as usize as i64).collect();
        check(unsafe { ffi::tl_hip_tensor_reshape(h(t), s.as_ptr(), s.len() as i32) })
    }
    pub fn tensor_transpose(&self, t: *mut c_void, dim0: usize, dim1: usize) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_transpose(h(t), dim0 as i64, dim1 as i64) })
    }
    pub fn tensor_transpose_2d(&self, t: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_transpose_2d(h(t)) })
    }
    pub fn tensor_narrow(&self, t: *mut c_void, dim: usize, start: usize, len: usize) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_narrow(h(t), dim as i64, start as i64, len as i64) })
    }
    pub fn tensor_cat(&self, a: *mut c_void, b: *mut c_void, dim: i64) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_cat(h(a), h(b), dim) })
    }
    /// device.rs:406 tensor_cat_4d: the same concatenation (any rank).
    pub fn tensor_cat_4d(&self, a: *mut c_void, b: *mut c_void, dim: i64) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_cat(h(a), h(b), dim) })
    }
    pub fn tensor_repeat_interleave(&self, t: *mut c_void, repeats: usize, dim: usize) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_repeat_interleave(h(t), repeats as i64, dim as i64) })
    }
    /// device.rs:418-425: tl_cpu ignores padding_idx / scale_grad / sparse (ffi.rs:1892-1898),
    /// and so does this adapter.
    pub fn tensor_embedding(
        &self,
        weight: *mut c_void,
        indices: *mut c_void,
        _padding_idx: i64,
        _scale_grad: bool,
        _sparse: bool,
    ) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_embedding(h(weight), h(indices)) })
    }
    /// device.rs:521-522: batched product and broadcast add over 4-D operands.
    pub fn tensor_matmul_4d(&self, a: *mut c_void, b: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_matmul(h(a), h(b)) })
    }
    pub fn tensor_add_4d(&self, a: *mut c_void, b: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_add(h(a), h(b)) })
    }

    // ========== LLM (device.rs:428-451) ==========
    pub fn tensor_rms_norm(&self, x: *mut c_void, w: *mut c_void, eps: f32) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_rms_norm(h(x), h(w), eps) })
    }
    pub fn tensor_rope_new_cos(&self, dim: usize, seq_len: usize, base: f32) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_rope_new_cos(dim as i64, seq_len as i64, base) })
    }
    pub fn tensor_rope_new_sin(&self, dim: usize, seq_len: usize, base: f32) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_rope_new_sin(dim as i64, seq_len as i64, base) })
    }
    pub fn tensor_apply_rope(&self, t: *mut c_void, cos: *mut c_void, sin: *mut c_void) -> BackendResult<*mut c_void> {
        check(unsafe { ffi::tl_hip_tensor_apply_rope(h(t), h(cos), h(sin)) })
    }
}

// In the crate these bodies sit in `impl IDevice for HipDevice { ... }`; every other IDevice
// method body is `not_provided("<method>")`.

/// The quantized linear of tl_runtime (system.rs:180-382, `tl_qtensor_matmul`) for
/// TL_DEVICE=hip: the raw GGUF blocks go to the device once (the `gpu_raw_cache` slot of the
/// QTensor, system.rs:316-331) and every call is one fused dequant + product.
pub fn qtensor_matmul_hip(
    x: *mut c_void,
    ggml_type: i32,
    raw: &[u8],
    shape: [usize; 2],
    cache: &mut *mut ffi::tl_hip_qtensor,
) -> BackendResult<*mut c_void> {
    if cache.is_null() {
        let s = [shape[0] as i64, shape[1] as i64];
        let q = unsafe { ffi::tl_hip_qtensor_new(ggml_type, raw.as_ptr(), raw.len(), s.as_ptr(), 2) };
        if q.is_null() {
            return Err(err_from_status());
        }
        *cache = q;
    }
    check(unsafe { ffi::tl_hip_qtensor_matmul(h(x), *cache) })
}
