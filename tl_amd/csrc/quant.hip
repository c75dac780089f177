// Quantized weights: GGUF Q4_0 / Q8_0 upload + repack, dequantisation, and the fused
// entry points of the quantized linear (matvec kernels: matvec.hip, GEMM: gemm.hip).
//
// Residency format (built once at upload, the role of QTensor::gpu_raw_cache,
// crates/tl_runtime/src/system.rs:316-331):  the 18-byte (Q4_0) / 34-byte (Q8_0) GGUF blocks
// are split into a 16-byte-aligned quant array qs[n][nb][16|32] and a scale array
// d[n][nb] (f16).  Bytes are unchanged (18 / 34 per 32 weights); every quant block is one
// (Q4_0) or two (Q8_0) 16-byte vector loads and the blocks of a row are contiguous, so a
// wavefront whose lanes walk consecutive blocks of a row reads 1 KiB (Q4_0) of contiguous
// memory per load instruction.
#include "internal.h"

#include <cstring>

namespace tlhip {

// ---------------------------------------------------------------- repack -----------
// One thread per GGUF block.  Q4_0: bytes 0-1 = d (LE f16), 2-17 = nibbles
// (quantized.rs:182-225).  Q8_0: bytes 0-1 = d, 2-33 = int8 (quantized.rs:227-260).
template <int QB>  // quant bytes per block: 16 (Q4_0) or 32 (Q8_0)
__global__ void k_repack(const uint8_t* __restrict__ raw, uint8_t* __restrict__ qs,
                         __half* __restrict__ d, int64_t nblocks) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* p = raw + b * (2 + QB);
    uint16_t h = (uint16_t)(p[0] | (p[1] << 8));
    d[b] = __ushort_as_half(h);
    uint32_t w[QB / 4];
#pragma unroll
    for (int i = 0; i < QB / 4; i++)
        w[i] = (uint32_t)p[2 + 4 * i] | ((uint32_t)p[3 + 4 * i] << 8) |
               ((uint32_t)p[4 + 4 * i] << 16) | ((uint32_t)p[5 + 4 * i] << 24);
    uint4* o = reinterpret_cast<uint4*>(qs + b * QB);
#pragma unroll
    for (int i = 0; i < QB / 16; i++) o[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
}

// ------------------------------------------------------------- dequantise ----------
// QTensor::dequantize_q4_0 / q8_0 (quantized.rs:182-260): one thread per 4 output
// elements.  d * (q - 8) and d * q are exact in f32 (11-bit x <=8-bit significands), so
// the result is bit-identical to the CPU path.
__global__ void k_dequant_q4_0(const uint8_t* __restrict__ qs, const __half* __restrict__ d,
                               float* __restrict__ out, int64_t nblocks) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (block, dword)
    int64_t b = t >> 2;
    int c = t & 3;
    if (b >= nblocks) return;
    uint32_t w = reinterpret_cast<const uint32_t*>(qs + b * 16)[c];
    float s = __half2float(d[b]);
    float* o = out + b * 32;
    float4 lo, hi;
    lo.x = s * (float)((int)(w & 0xF) - 8);
    lo.y = s * (float)((int)((w >> 8) & 0xF) - 8);
    lo.z = s * (float)((int)((w >> 16) & 0xF) - 8);
    lo.w = s * (float)((int)((w >> 24) & 0xF) - 8);
    hi.x = s * (float)((int)((w >> 4) & 0xF) - 8);
    hi.y = s * (float)((int)((w >> 12) & 0xF) - 8);
    hi.z = s * (float)((int)((w >> 20) & 0xF) - 8);
    hi.w = s * (float)((int)((w >> 28) & 0xF) - 8);
    reinterpret_cast<float4*>(o)[c] = lo;       // elements 4c .. 4c+3
    reinterpret_cast<float4*>(o + 16)[c] = hi;  // elements 16+4c .. 16+4c+3
}

__global__ void k_dequant_q8_0(const uint8_t* __restrict__ qs, const __half* __restrict__ d,
                               float* __restrict__ out, int64_t nblocks) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (block, dword)
    int64_t b = t >> 3;
    int c = t & 7;
    if (b >= nblocks) return;
    uint32_t w = reinterpret_cast<const uint32_t*>(qs + b * 32)[c];
    float s = __half2float(d[b]);
    float4 v;
    v.x = s * (float)(int8_t)(w & 0xFF);
    v.y = s * (float)(int8_t)((w >> 8) & 0xFF);
    v.z = s * (float)(int8_t)((w >> 16) & 0xFF);
    v.w = s * (float)(int8_t)(w >> 24);
    reinterpret_cast<float4*>(out + b * 32)[c] = v;
}

}  // namespace tlhip

using namespace tlhip;

static bool q_validate(int ggml_type, size_t nbytes, const int64_t* shape, int rank,
                       int64_t* n, int64_t* k) {
    if (!shape) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: shape");
        return false;
    }
    if (ggml_type != TL_HIP_GGML_Q4_0 && ggml_type != TL_HIP_GGML_Q8_0) {
        set_error(TL_HIP_ERR_TYPE,
                  "TypeMismatch: ggml type %d has no device residency (Q4_0=2, Q8_0=8)",
                  ggml_type);
        return false;
    }
    if (rank != 2) {
        // tl_qtensor_matmul asserts a 2-D QTensor (system.rs:228)
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: QTensor must be 2D, got %dD", rank);
        return false;
    }
    int64_t numel = shape[0] * shape[1];
    if (shape[0] <= 0 || shape[1] <= 0) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: empty quantized tensor");
        return false;
    }
    const char* tn = ggml_type == TL_HIP_GGML_Q4_0 ? "Q4_0" : "Q8_0";
    if (numel % 32 != 0 || shape[1] % 32 != 0) {
        // quantized.rs:190-192 (rows must also hold whole blocks for a row-wise product)
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Number of elements must be multiple of 32 for %s", tn);
        return false;
    }
    int64_t nblocks = numel / 32;
    size_t bs = ggml_type == TL_HIP_GGML_Q4_0 ? 18 : 34;
    if (nbytes != (size_t)nblocks * bs) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: Data size mismatch for %s: expected %lld, got %zu",
                  tn, (long long)(nblocks * (int64_t)bs), nbytes);  // quantized.rs:195-200
        return false;
    }
    *n = shape[0];
    *k = shape[1];
    return true;
}

extern "C" {

tl_hip_qtensor* tl_hip_qtensor_new(int ggml_type, const uint8_t* data, size_t nbytes,
                                   const int64_t* shape, int rank) {
    int64_t n, k;
    if (!data) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: data");
        return nullptr;
    }
    if (!q_validate(ggml_type, nbytes, shape, rank, &n, &k)) return nullptr;
    if (!state()) return nullptr;
    hipStream_t s = cur_stream();
    const int QB = ggml_type == TL_HIP_GGML_Q4_0 ? 16 : 32;
    int64_t nblocks = n * k / 32;
    QWeight* w = new QWeight();
    w->ggml_type = ggml_type;
    w->n = n;
    w->k = k;
    w->nb = k / 32;
    w->rank = 2;
    w->shape[0] = n;
    w->shape[1] = k;
    w->qs = (uint8_t*)dev_alloc(nblocks * QB);
    w->d = (__half*)dev_alloc(nblocks * 2 + 4);  // + 4: the prefill GEMM reads scales as aligned words
    uint8_t* raw = (uint8_t*)dev_alloc(nbytes);
    if (!w->qs || !w->d || !raw) {
        dev_free(w->qs);
        dev_free(w->d);
        dev_free(raw);
        delete w;
        return nullptr;
    }
    hipError_t e = hipMemcpyAsync(raw, data, nbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        if (QB == 16)
            k_repack<16><<<cdiv(nblocks, 256), 256, 0, s>>>(raw, w->qs, w->d, nblocks);
        else
            k_repack<32><<<cdiv(nblocks, 256), 256, 0, s>>>(raw, w->qs, w->d, nblocks);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // the host buffer may go away
    dev_free(raw);
    if (e != hipSuccess) {
        hip_fail(e, "qtensor upload");
        dev_free(w->qs);
        dev_free(w->d);
        delete w;
        return nullptr;
    }
    return reinterpret_cast<tl_hip_qtensor*>(w);
}

int tl_hip_qtensor_release(tl_hip_qtensor* h) {
    if (!h) return TL_HIP_OK;
    QWeight* w = Q(h);
    if (w->refs.fetch_sub(1) == 1) {
        dev_free(w->qs);
        dev_free(w->d);
        delete w;
    }
    return TL_HIP_OK;
}

tl_hip_tensor* tl_hip_qtensor_dequantize(const tl_hip_qtensor* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: qtensor");
        return nullptr;
    }
    const QWeight* w = reinterpret_cast<const QWeight*>(h);
    Tensor* t = tensor_alloc(w->shape, 2);
    if (!t) return nullptr;
    hipStream_t s = cur_stream();
    int64_t nblocks = w->n * w->nb;
    if (w->ggml_type == TL_HIP_GGML_Q4_0)
        k_dequant_q4_0<<<cdiv(nblocks * 4, 256), 256, 0, s>>>(w->qs, w->d, t->f32(), nblocks);
    else
        k_dequant_q8_0<<<cdiv(nblocks * 8, 256), 256, 0, s>>>(w->qs, w->d, t->f32(), nblocks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        hip_fail(e, "dequant launch");
        tensor_drop(t);
        return nullptr;
    }
    return H(t);
}

static tl_hip_tensor* qmatmul(const tl_hip_tensor* xh, const tl_hip_qtensor* qh, int f16) {
    if (!xh || !qh) {
        // system.rs:184-187
        set_error(TL_HIP_ERR_NULL, "NullPointerError: tl_qtensor_matmul received null argument");
        return nullptr;
    }
    const Tensor* x = reinterpret_cast<const Tensor*>(xh);
    const QWeight* w = reinterpret_cast<const QWeight*>(qh);
    if (x->dtype != TL_HIP_F32) {
        set_error(TL_HIP_ERR_TYPE, "TypeMismatch: x must be f32");
        return nullptr;
    }
    if (x->rank < 1 || x->shape[x->rank - 1] != w->k) {
        set_error(TL_HIP_ERR_SHAPE,
                  "ShapeMismatch: Matmul shape mismatch: x last dim %lld vs weight [%lld, %lld]",
                  (long long)(x->rank ? x->shape[x->rank - 1] : 0), (long long)w->n,
                  (long long)w->k);
        return nullptr;
    }
    int64_t m = x->numel / w->k;
    int64_t oshape[TL_HIP_MAX_RANK];
    int orank = x->rank < 2 ? 2 : x->rank;
    if (x->rank < 2) {
        oshape[0] = 1;  // a 1-D x is one row (matmul_impl treats [k] as m = 1)
    } else {
        for (int i = 0; i < x->rank - 1; i++) oshape[i] = x->shape[i];
    }
    oshape[orank - 1] = w->n;
    Tensor* y = tensor_alloc(oshape, orank);
    if (!y) return nullptr;
    int rc = TL_HIP_OK;
    if (m > 0) {
        if (m <= 4)
            rc = launch_quant_matvec(w, x->f32(), y->f32(), m, cur_stream(), nullptr);
        else
            rc = launch_quant_gemm(w, x->f32(), y->f32(), m, cur_stream(), f16);
    }
    if (rc != TL_HIP_OK) {
        tensor_drop(y);
        return nullptr;
    }
    return H(y);
}

tl_hip_tensor* tl_hip_qtensor_matmul(const tl_hip_tensor* x, const tl_hip_qtensor* q) {
    return qmatmul(x, q, 0);
}

tl_hip_tensor* tl_hip_qtensor_matmul_f16(const tl_hip_tensor* x, const tl_hip_qtensor* q) {
    return qmatmul(x, q, 1);
}

int tl_hip_launch_quant_matvec(const tl_hip_qtensor* h, const float* x, float* y, int64_t m,
                               void* stream) {
    if (!h || !x || !y) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: weight, x or y");
        return TL_HIP_ERR_NULL;
    }
    if (!state()) return tl_hip_last_status();
    return launch_quant_matvec(reinterpret_cast<const QWeight*>(h), x, y, m,
                               stream ? (hipStream_t)stream : cur_stream(), nullptr);
}

int tl_hip_launch_quant_gemm(const tl_hip_qtensor* h, const float* x, float* y, int64_t m,
                             int use_f16_mfma, void* stream) {
    if (!h || !x || !y) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: weight, x or y");
        return TL_HIP_ERR_NULL;
    }
    if (!state()) return tl_hip_last_status();
    return launch_quant_gemm(reinterpret_cast<const QWeight*>(h), x, y, m,
                             stream ? (hipStream_t)stream : cur_stream(), use_f16_mfma);
}

}  // extern "C"
