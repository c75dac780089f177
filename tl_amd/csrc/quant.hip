// Quantized weights: GGUF Q4_0 / Q8_0 / Q4_K / Q6_K upload + repack, dequantisation, and the
// fused entry points of the quantized linear (matvec kernels: matvec.hip, GEMM: gemm.hip).
//
// Residency format (built once at upload, the role of QTensor::gpu_raw_cache,
// crates/tl_runtime/src/system.rs:316-331): the GGUF blocks are split into struct-of-arrays
// form over 32-weight units (layout in internal.h, struct QWeight).  Bytes are unchanged
// (18 / 34 per 32 weights, 144 / 210 per 256); every unit's quant bytes are one (two for
// Q8_0) 16-byte vector load, and the units of a row are contiguous, so a wavefront whose
// lanes walk consecutive units of a row reads 1 KiB of contiguous memory per load
// instruction.  The K-quant nibbles are re-ordered so a unit's 32 weights sit in one
// 16-byte chunk in Q4_0 order (low nibble of byte j = weight j, high = weight j + 16).
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

// K-quant repack: one thread per 32-weight unit.  Q4_K (quantized.rs:337-400): unit u of a
// super-block is sub-block u; its weights are the low (u even) or high (u odd) nibbles of
// quant bytes 32 (u / 2) .. +31.  Unit thread 0 writes the header: d and dmin as stored, the
// eight (scale, min) pairs unpacked by the get_scale_min_k4 rule (quantized.rs:405-415) and
// re-laid as q4k_hdr_sm reads them.
__global__ void k_repack_q4_k(const uint8_t* __restrict__ raw, uint8_t* __restrict__ qs,
                              uint8_t* __restrict__ hdr, int64_t nunits) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nunits) return;
    const int64_t sb = t >> 3;
    const int u = (int)(t & 7);
    const uint8_t* p = raw + sb * 144;
    const uint8_t* g = p + 16 + 32 * (u >> 1);
    uint8_t o[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint8_t a = g[j], b = g[16 + j];
        o[j] = (u & 1) ? (uint8_t)((a >> 4) | (b & 0xF0)) : (uint8_t)((a & 0x0F) | (b << 4));
    }
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        w[i] = o[4 * i] | (o[4 * i + 1] << 8) | (o[4 * i + 2] << 16) | ((uint32_t)o[4 * i + 3] << 24);
    reinterpret_cast<uint4*>(qs)[t] = make_uint4(w[0], w[1], w[2], w[3]);
    if (u == 0) {
        const uint8_t* q = p + 4;  // the 12 packed scale bytes
        uint64_t sc = 0, mn = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t s = j < 4 ? q[j] & 63u : (q[j + 4] & 0xFu) | ((uint32_t)(q[j - 4] >> 6) << 4);
            const uint32_t m = j < 4 ? q[j + 4] & 63u : (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
            sc |= (uint64_t)s << (6 * j);
            mn |= (uint64_t)m << (6 * j);
        }
        const uint32_t x = p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);  // f16 d | f16 dmin
        reinterpret_cast<uint4*>(hdr)[sb] =
            make_uint4(x, (uint32_t)sc, (uint32_t)(sc >> 32) | (uint32_t)(mn << 16), (uint32_t)(mn >> 16));
    }
}

// Q6_K (quantized.rs:268-329): unit u covers weights 32u .. 32u+31 of the super-block, i.e.
// in the reference's terms half h = u / 4, a = u % 4, l = 0..31 with the 6-bit value
// (a odd ? ql[l + 32] : ql[l]) >> (a >= 2 ? 4 : 0) & 15 | (qh[l] >> 2a & 3) << 4 and the
// scales (32u + j) / 16 = 2u, 2u + 1.
__global__ void k_repack_q6_k(const uint8_t* __restrict__ raw, uint8_t* __restrict__ qs,
                              uint8_t* __restrict__ qh, int8_t* __restrict__ sc,
                              __half* __restrict__ d, int64_t nunits) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nunits) return;
    const int64_t sb = t >> 3;
    const int u = (int)(t & 7), h = u >> 2, a = u & 3;
    const uint8_t* p = raw + sb * 210;
    const uint8_t* ql = p + 64 * h + ((a & 1) ? 32 : 0);
    const uint8_t* qhp = p + 128 + 32 * h;
    const int sh = (a & 2) ? 4 : 0;
    uint8_t q[32];
#pragma unroll
    for (int l = 0; l < 32; l++) q[l] = (uint8_t)(((ql[l] >> sh) & 0xF) | (((qhp[l] >> (2 * a)) & 3) << 4));
    uint32_t w[4], hw[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        w[i] = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) w[i] |= (uint32_t)((q[4 * i + b] & 0xF) | ((q[16 + 4 * i + b] & 0xF) << 4)) << (8 * b);
    }
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
                hw[half] |= (uint32_t)((q[16 * half + b + 4 * tt] >> 4) & 3) << (8 * b + 2 * tt);
    reinterpret_cast<uint4*>(qs)[t] = make_uint4(w[0], w[1], w[2], w[3]);
    reinterpret_cast<uint2*>(qh)[t] = make_uint2(hw[0], hw[1]);
    sc[2 * t] = (int8_t)p[192 + 2 * u];
    sc[2 * t + 1] = (int8_t)p[192 + 2 * u + 1];
    if (u == 0) d[sb] = __ushort_as_half((uint16_t)(p[208] | (p[209] << 8)));
}

// Q4_K (scale, min) of sub-block j from the header's 12 packed bytes (words 1..3 of the
// header), QTensor::get_scale_min_k4 (quantized.rs:405-415).

// Dequantisation from the residency format, one thread per unit.  Q4_K: (d * sc) * q -
// dmin * m (quantized.rs:380-390; both products exact, one rounding in the subtraction).
__global__ void k_dequant_q4_k(const uint8_t* __restrict__ qs, const uint8_t* __restrict__ hdr,
                               float* __restrict__ out, int64_t nunits) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nunits) return;
    const uint4 hd = reinterpret_cast<const uint4*>(hdr)[t >> 3];
    const uint4 w = reinterpret_cast<const uint4*>(qs)[t];
    uint32_t sc, mn;
    q4k_hdr_sm(hd, (int)(t & 7), &sc, &mn);
    const float d = __half2float(__ushort_as_half((uint16_t)(hd.x & 0xFFFF)));
    const float dmin = __half2float(__ushort_as_half((uint16_t)(hd.x >> 16)));
    const float d1 = d * (float)sc, m1 = dmin * (float)mn;
    const uint32_t q[4] = {w.x, w.y, w.z, w.w};
    float lo[16], hi[16];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t byte = (q[c] >> (8 * b)) & 0xFF;
            lo[4 * c + b] = d1 * (float)(byte & 0xF) - m1;
            hi[4 * c + b] = d1 * (float)(byte >> 4) - m1;
        }
    float4* o = reinterpret_cast<float4*>(out + t * 32);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        o[c] = make_float4(lo[4 * c], lo[4 * c + 1], lo[4 * c + 2], lo[4 * c + 3]);
        o[4 + c] = make_float4(hi[4 * c], hi[4 * c + 1], hi[4 * c + 2], hi[4 * c + 3]);
    }
}

// Q6_K: (d * sc) * (q - 32), evaluated in that order (quantized.rs:315-318; exact in f32).
__global__ void k_dequant_q6_k(const uint8_t* __restrict__ qs, const uint8_t* __restrict__ qh,
                               const int8_t* __restrict__ sc, const __half* __restrict__ dsc,
                               float* __restrict__ out, int64_t nunits) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nunits) return;
    const uint4 w = reinterpret_cast<const uint4*>(qs)[t];
    const uint2 h = reinterpret_cast<const uint2*>(qh)[t];
    const float d = __half2float(dsc[t >> 3]);
    const float e0 = d * (float)sc[2 * t], e1 = d * (float)sc[2 * t + 1];
    const uint32_t q[4] = {w.x, w.y, w.z, w.w};
    float lo[16], hi[16];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t byte = (q[c] >> (8 * b)) & 0xFF;
            const uint32_t h0 = (h.x >> (8 * b + 2 * c)) & 3, h1 = (h.y >> (8 * b + 2 * c)) & 3;
            lo[4 * c + b] = e0 * (float)((int)((byte & 0xF) | (h0 << 4)) - 32);
            hi[4 * c + b] = e1 * (float)((int)((byte >> 4) | (h1 << 4)) - 32);
        }
    float4* o = reinterpret_cast<float4*>(out + t * 32);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        o[c] = make_float4(lo[4 * c], lo[4 * c + 1], lo[4 * c + 2], lo[4 * c + 3]);
        o[4 + c] = make_float4(hi[4 * c], hi[4 * c + 1], hi[4 * c + 2], hi[4 * c + 3]);
    }
}

}  // namespace tlhip

using namespace tlhip;

static bool q_validate(int ggml_type, size_t nbytes, const int64_t* shape, int rank,
                       int64_t* n, int64_t* k) {
    if (!shape) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: shape");
        return false;
    }
    const int be = ggml_block_elems(ggml_type);
    if (!be) {
        set_error(TL_HIP_ERR_TYPE,
                  "TypeMismatch: ggml type %d has no device residency (Q4_0=2, Q8_0=8, Q4_K=12, Q6_K=14)",
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
    const char* tn = ggml_type_name(ggml_type);
    if (numel % be != 0 || shape[1] % be != 0) {
        // quantized.rs:190-192 / 273-275 / 342-344 (rows must also hold whole blocks for a
        // row-wise product)
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Number of elements must be multiple of %d for %s", be, tn);
        return false;
    }
    int64_t nblocks = numel / be;
    size_t bs = (size_t)ggml_block_bytes(ggml_type);
    if (nbytes != (size_t)nblocks * bs) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: Data size mismatch for %s: expected %lld, got %zu",
                  tn, (long long)(nblocks * (int64_t)bs), nbytes);  // quantized.rs:195-200, 278-283, 347-352
        return false;
    }
    *n = shape[0];
    *k = shape[1];
    return true;
}

static void q_free(QWeight* w) {
    dev_free(w->qs);
    dev_free(w->d);
    dev_free(w->hdr);
    dev_free(w->qh);
    dev_free(w->sc);
    dev_free(w->us);
    delete w;
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
    const int64_t nunits = n * k / 32;
    QWeight* w = new QWeight();
    w->ggml_type = ggml_type;
    w->n = n;
    w->k = k;
    w->nb = k / 32;
    w->rank = 2;
    w->shape[0] = n;
    w->shape[1] = k;
    bool ok = true;
    switch (ggml_type) {
        case TL_HIP_GGML_Q4_0:
        case TL_HIP_GGML_Q8_0:
            w->qs = (uint8_t*)dev_alloc(nunits * (ggml_type == TL_HIP_GGML_Q4_0 ? 16 : 32));
            w->d = (__half*)dev_alloc(nunits * 2 + 4);  // + 4: the prefill GEMM reads scales as aligned words
            ok = w->qs && w->d;
            break;
        case TL_HIP_GGML_Q4_K:
            w->qs = (uint8_t*)dev_alloc(nunits * 16);
            w->hdr = (uint8_t*)dev_alloc(nunits / 8 * 16);
            ok = w->qs && w->hdr;
            break;
        default:  // Q6_K
            w->qs = (uint8_t*)dev_alloc(nunits * 16);
            w->qh = (uint8_t*)dev_alloc(nunits * 8);
            w->sc = (int8_t*)dev_alloc(nunits * 2);
            w->d = (__half*)dev_alloc(nunits / 8 * 2 + 4);
            ok = w->qs && w->qh && w->sc && w->d;
            break;
    }
    uint8_t* raw = ok ? (uint8_t*)dev_alloc(nbytes) : nullptr;
    if (!raw) {
        q_free(w);
        return nullptr;
    }
    hipError_t e = hipMemcpyAsync(raw, data, nbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        switch (ggml_type) {
            case TL_HIP_GGML_Q4_0: k_repack<16><<<cdiv(nunits, 256), 256, 0, s>>>(raw, w->qs, w->d, nunits); break;
            case TL_HIP_GGML_Q8_0: k_repack<32><<<cdiv(nunits, 256), 256, 0, s>>>(raw, w->qs, w->d, nunits); break;
            case TL_HIP_GGML_Q4_K: k_repack_q4_k<<<cdiv(nunits, 256), 256, 0, s>>>(raw, w->qs, w->hdr, nunits); break;
            default: k_repack_q6_k<<<cdiv(nunits, 256), 256, 0, s>>>(raw, w->qs, w->qh, w->sc, w->d, nunits); break;
        }
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // the host buffer may go away
    dev_free(raw);
    if (e != hipSuccess) {
        hip_fail(e, "qtensor upload");
        q_free(w);
        return nullptr;
    }
    return reinterpret_cast<tl_hip_qtensor*>(w);
}

int tl_hip_qtensor_release(tl_hip_qtensor* h) {
    if (!h) return TL_HIP_OK;
    QWeight* w = Q(h);
    if (w->refs.fetch_sub(1) == 1) q_free(w);
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
    switch (w->ggml_type) {
        case TL_HIP_GGML_Q4_0:
            k_dequant_q4_0<<<cdiv(nblocks * 4, 256), 256, 0, s>>>(w->qs, w->d, t->f32(), nblocks);
            break;
        case TL_HIP_GGML_Q8_0:
            k_dequant_q8_0<<<cdiv(nblocks * 8, 256), 256, 0, s>>>(w->qs, w->d, t->f32(), nblocks);
            break;
        case TL_HIP_GGML_Q4_K:
            k_dequant_q4_k<<<cdiv(nblocks, 256), 256, 0, s>>>(w->qs, w->hdr, t->f32(), nblocks);
            break;
        default:
            k_dequant_q6_k<<<cdiv(nblocks, 256), 256, 0, s>>>(w->qs, w->qh, w->sc, w->d, t->f32(), nblocks);
            break;
    }
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
        // the matvec for up to 4 rows when its LDS staging holds the rows, else the GEMM
        // (which takes any k, as tl_qtensor_matmul does)
        if (matvec_fits(w, m))
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
    note_stream((hipStream_t)stream);
    return launch_quant_matvec(reinterpret_cast<const QWeight*>(h), x, y, m,
                               stream ? (hipStream_t)stream : cur_stream(), nullptr);
}

int tl_hip_read_floor(const tl_hip_qtensor* h, void* stream) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: weight");
        return TL_HIP_ERR_NULL;
    }
    if (!state()) return tl_hip_last_status();
    note_stream((hipStream_t)stream);
    return launch_read_floor(reinterpret_cast<const QWeight*>(h), stream ? (hipStream_t)stream : cur_stream());
}

int tl_hip_launch_quant_gemm(const tl_hip_qtensor* h, const float* x, float* y, int64_t m,
                             int use_f16_mfma, void* stream) {
    if (!h || !x || !y) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: weight, x or y");
        return TL_HIP_ERR_NULL;
    }
    if (!state()) return tl_hip_last_status();
    note_stream((hipStream_t)stream);
    return launch_quant_gemm(reinterpret_cast<const QWeight*>(h), x, y, m,
                             stream ? (hipStream_t)stream : cur_stream(), use_f16_mfma);
}

}  // extern "C"
