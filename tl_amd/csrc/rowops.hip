// Memory-bound row and element operators of the decode/prefill path, single pass where
// the reference makes several: RMSNorm (+weight), RoPE tables and application, SiLU /
// SwiGLU, row softmax, broadcast binary ops, scale, and the data-movement glue of the
// chatbot's attention (narrow / cat / repeat_interleave / transpose), embedding gather,
// greedy argmax and repetition penalty.  f32 math throughout.
#include "internal.h"

#include <cmath>
#include <cstring>
#include <random>
#include <vector>

namespace tlhip {

// block-wide sum; every thread receives the result.  `red` holds >= blockDim/64 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_allsum(v);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}
__device__ __forceinline__ float block_max(float v, float* red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_allmax(v);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = -INFINITY;
    for (int i = 0; i < nw; i++) s = fmaxf(s, red[i]);
    return s;
}

// float4 loads / stores with the non-temporal policy (streams read or written once)
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt(const float4* p) {
    const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void st_nt(float4* p, const float4& v) {
    __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4*>(p));
}

// ------------------------------------------------------------------ RMSNorm ---------
// One workgroup of T threads per row; the row is held in registers (V float4 per thread) so
// x is read once.  mode 0: (x / sqrt(ms + eps)) * w     (tl_cpu ffi.rs:2444-2486 + mul_impl)
//      mode 1: x * (1 / sqrt(ms + eps)) * w   (fused_rms_norm, fused_ops.rs:37-57)
// With a residual r the row is x + r first (fused_add_rms_norm, fused_ops.rs:59-85).
// The row, the residual and the weight are all requested before the reduction (the weight
// used to follow it: a second memory round trip per row), the row streams are non-temporal.
// (One wavefront per row, no barrier, measured slower: 8.9 against 5.8 us at [512, 4096] --
// two wavefronts per CU then issue all the loads.)
template <int V, int T = 256>
__global__ __launch_bounds__(T) void k_rmsnorm(const float* __restrict__ x,
                                                 const float* __restrict__ r,
                                                 const float* __restrict__ w,
                                                 float* __restrict__ out, int64_t n, float eps,
                                                 int mode) {
    asm volatile("" : : "s"(x), "s"(r), "s"(w), "s"(out), "s"(n), "s"(eps), "s"(mode));  // one round of loads
    __shared__ float red[T / 64];
    const int64_t row = blockIdx.x;
    const float4* xr = reinterpret_cast<const float4*>(x + row * n);
    const float4* rr = r ? reinterpret_cast<const float4*>(r + row * n) : nullptr;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    const int64_t n4 = n >> 2;
    float4 v[V], ww[V];
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int64_t j = threadIdx.x + (int64_t)i * T;
        v[i] = j < n4 ? ld_nt(xr + j) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int64_t j = threadIdx.x + (int64_t)i * T;
        ww[i] = w4 && j < n4 ? w4[j] : make_float4(1.f, 1.f, 1.f, 1.f);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int64_t j = threadIdx.x + (int64_t)i * T;
        if (rr && j < n4) {
            const float4 q = ld_nt(rr + j);
            v[i].x = v[i].x + q.x;
            v[i].y = v[i].y + q.y;
            v[i].z = v[i].z + q.z;
            v[i].w = v[i].w + q.w;
        }
        ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    }
    // block sum with one barrier (red is written once per launch)
    ss = wave_allsum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    if constexpr (T == 256) ss = red[0] + red[1] + red[2] + red[3];
    else {
        ss = 0.f;
#pragma unroll
        for (int w = 0; w < T / 64; w++) ss += red[w];
    }
    const float ms = ss / (float)n;
    const float rms = sqrtf(ms + eps);
    const float rcp = 1.0f / rms;
    float4* o = reinterpret_cast<float4*>(out + row * n);
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int64_t j = threadIdx.x + (int64_t)i * T;
        if (j >= n4) continue;
        const float4 a = v[i], b = ww[i];
        float4 res;
        if (mode == 0) {
            res.x = a.x / rms; res.y = a.y / rms; res.z = a.z / rms; res.w = a.w / rms;
            if (w4) { res.x = res.x * b.x; res.y = res.y * b.y; res.z = res.z * b.z; res.w = res.w * b.w; }
        } else {
            res.x = a.x * rcp * b.x; res.y = a.y * rcp * b.y;
            res.z = a.z * rcp * b.z; res.w = a.w * rcp * b.w;
        }
        st_nt(o + j, res);
    }
}

// generic RMSNorm for rows not divisible by 4 or longer than 8192: two reads of the row
__global__ __launch_bounds__(256) void k_rmsnorm_generic(const float* __restrict__ x,
                                                         const float* __restrict__ r,
                                                         const float* __restrict__ w,
                                                         float* __restrict__ out, int64_t n,
                                                         float eps, int mode) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const float* xr = x + row * n;
    const float* rr = r ? r + row * n : nullptr;
    float ss = 0.f;
    for (int64_t j = threadIdx.x; j < n; j += 256) {
        float a = rr ? xr[j] + rr[j] : xr[j];
        ss += a * a;
    }
    ss = block_sum(ss, red);
    const float rms = sqrtf(ss / (float)n + eps), rcp = 1.0f / rms;
    for (int64_t j = threadIdx.x; j < n; j += 256) {
        float a = rr ? xr[j] + rr[j] : xr[j];
        float res;
        if (mode == 0) {
            res = a / rms;
            if (w) res = res * w[j];
        } else {
            res = a * rcp * (w ? w[j] : 1.f);
        }
        out[row * n + j] = res;
    }
}

// RMSNorm mode 0 whose output goes straight to the f16 operand order of the GEMM that reads
// it: the sum of squares in the order of k_rmsnorm's 256-thread form (thread j's float4 j,
// j + 256, ...; k_rmsnorm takes that form for rows up to 2048 elements, so there the f32 value
// is k_rmsnorm's, rounded once to f16), then one 8-half word per (block, t) unit.  (The norm
// weight requested with the row, before the reduction, measured no faster: L2 hits.)
// SUM: the row is first completed from a deferred split-K GEMM -- x = x + part_0 + ... +
// part_{nsp-1} in slice order, the additions of k_splitk_sum -- written back to x (the new
// residual) and kept in LDS for the normalisation: one launch instead of the sum's and this.
template <int V, bool SUM = false>
__global__ __launch_bounds__(256) void k_rmsnorm_f16q(float* __restrict__ x, const float* __restrict__ w,
                                                      _Float16* __restrict__ out16, int64_t n, float eps,
                                                      int order, const float* __restrict__ part, int nsp,
                                                      int64_t mn) {
    asm volatile("" : : "s"(x), "s"(w), "s"(out16), "s"(n), "s"(eps), "s"(order));  // arguments in one round
    __shared__ float red[4];
    __shared__ float4 rowbuf[SUM ? V * 256 : 1];
    const int64_t row = blockIdx.x;
    float* xr = x + row * n;
    float4* x4 = reinterpret_cast<float4*>(xr);
    const int64_t n4 = n >> 2;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int64_t j = threadIdx.x + (int64_t)i * 256;
        float4 v = j < n4 ? x4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (SUM) {
            if (j < n4) {
                const float4* p4 = reinterpret_cast<const float4*>(part + row * n) + j;
                for (int p = 0; p < nsp; p++) {
                    const float4 t = p4[p * (mn >> 2)];
                    v.x += t.x;
                    v.y += t.y;
                    v.z += t.z;
                    v.w += t.w;
                }
                x4[j] = v;
                rowbuf[j] = v;
            }
        }
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = block_sum(ss, red);  // its barriers also publish rowbuf
    const float rms = sqrtf(ss / (float)n + eps);
    const int64_t units = (n >> 5) * 4;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    for (int64_t u = threadIdx.x; u < units; u += 256) {
        // word t of block b: float4s (8b + t, 8b + 4 + t) in Q4 order, (8b + 2t, 8b + 2t + 1) in Q8
        const int64_t b = u >> 2;
        const int t = (int)(u & 3);
        const int64_t i0 = order == F16Q_Q8 ? 8 * b + 2 * t : 8 * b + t, i1 = order == F16Q_Q8 ? i0 + 1 : i0 + 4;
        const float4 e = SUM ? rowbuf[i0] : x4[i0], f = SUM ? rowbuf[i1] : x4[i1], we = w4[i0], wf = w4[i1];
        const float v[8] = {(e.x / rms) * we.x, (e.y / rms) * we.y, (e.z / rms) * we.z, (e.w / rms) * we.w,
                            (f.x / rms) * wf.x, (f.y / rms) * wf.y, (f.z / rms) * wf.z, (f.w / rms) * wf.w};
        half8 h;
        if (order == F16Q_Q8) {  // slots: e0 e2 e1 e3 f0 f2 f1 f3
            h = half8{(_Float16)v[0], (_Float16)v[2], (_Float16)v[1], (_Float16)v[3],
                      (_Float16)v[4], (_Float16)v[6], (_Float16)v[5], (_Float16)v[7]};
        } else {
            h = half8{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3],
                      (_Float16)v[4], (_Float16)v[5], (_Float16)v[6], (_Float16)v[7]};
        }
        reinterpret_cast<half8*>(out16)[row * units + u] = h;
    }
}

int launch_rmsnorm_f16q(float* x, const float* w, _Float16* out16, int64_t rows, int64_t n, float eps, int order,
                        hipStream_t s, const float* part, int nsp) {
    if (rows <= 0) return TL_HIP_OK;
    const int64_t per = cdiv(n / 4, 256);
    if (n % 32 != 0 || per > 8 || (uintptr_t)x % 16 != 0 || !w || (uintptr_t)w % 16 != 0 ||
        (part && ((uintptr_t)part % 16 != 0 || nsp < 1))) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: f16 operand-order RMSNorm takes rows of 32k <= 8192 floats");
        return TL_HIP_ERR_ARG;
    }
    const int64_t mn = rows * n;
#define TLH_RN(VV)                                                                                      \
    if (part) k_rmsnorm_f16q<VV, true><<<rows, 256, 0, s>>>(x, w, out16, n, eps, order, part, nsp, mn); \
    else k_rmsnorm_f16q<VV><<<rows, 256, 0, s>>>(x, w, out16, n, eps, order, nullptr, 0, mn)
    if (per <= 1) TLH_RN(1);
    else if (per <= 2) TLH_RN(2);
    else if (per <= 4) TLH_RN(4);
    else TLH_RN(8);
#undef TLH_RN
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "rmsnorm launch");
}

int launch_rmsnorm(const float* x, const float* r, const float* w, float* out, int64_t rows,
                   int64_t n, float eps, int mode, hipStream_t s) {
    if (rows <= 0 || n <= 0) return TL_HIP_OK;
    const bool vec = (n % 4 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)out % 16 == 0) &&
                     (!r || (uintptr_t)r % 16 == 0) && (!w || (uintptr_t)w % 16 == 0);
    const int64_t per = cdiv(n / 4, 256);
    if (vec && per <= 1)
        k_rmsnorm<1><<<rows, 256, 0, s>>>(x, r, w, out, n, eps, mode);
    else if (vec && per <= 2)
        k_rmsnorm<2><<<rows, 256, 0, s>>>(x, r, w, out, n, eps, mode);
    else if (vec && per <= 4)  // 2049-4096 elements: 512 threads x 2 float4 (4.9 -> 4.7 us at [512, 4096])
        k_rmsnorm<2, 512><<<rows, 512, 0, s>>>(x, r, w, out, n, eps, mode);
    else if (vec && per <= 8)
        k_rmsnorm<8><<<rows, 256, 0, s>>>(x, r, w, out, n, eps, mode);
    else
        k_rmsnorm_generic<<<rows, 256, 0, s>>>(x, r, w, out, n, eps, mode);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "rmsnorm launch");
}

// -------------------------------------------------------------------- RoPE ----------
// Tables of tl_cpu_tensor_rope_new_cos/_sin (ffi.rs:2589-2629): [seq_len, dim], entries
// 2i and 2i+1 hold cos/sin(pos * 1/base^(2i/dim)).
__global__ void k_rope_table(float* __restrict__ out, int64_t seq_len, int64_t dim, float base,
                             int is_sin) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t half = dim / 2;
    if (t >= seq_len * half) return;
    int64_t pos = t / half, i = t % half;
    // f32 operation sequence of ffi.rs:2598-2601; pow / cos / sin are evaluated in double and
    // rounded once, i.e. correctly rounded f32 results (what the host libm returns for all
    // but rare halfway cases) -- the angle pos * freq amplifies any ulp difference in freq
    float e = 2.0f * (float)i / (float)dim;
    float r = (float)pow((double)base, (double)e);
    float freq = 1.0f / r;
    float a = (float)pos * freq;
    float v = is_sin ? (float)sin((double)a) : (float)cos((double)a);
    out[pos * dim + 2 * i] = v;
    out[pos * dim + 2 * i + 1] = v;
}

// apply_rope (ffi.rs:2631-2686): interleaved pairs (i, i+1) of each head_dim vector.
// Table row: row0 for every vector (tl_cpu semantics, vpt == 0), or row0 + v / vpt.
// Entries past the table's end read as cos 1, sin 0.
__global__ void k_apply_rope(const float* __restrict__ x, const float* __restrict__ ct,
                             const float* __restrict__ st, float* __restrict__ out,
                             int64_t npairs, int64_t hd, int64_t cos_len, int64_t sin_len,
                             int64_t row0, int64_t vpt) {
    int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npairs) return;
    int64_t hp = hd / 2;
    int64_t v = p / hp, i = 2 * (p % hp);
    int64_t row = vpt > 0 ? row0 + v / vpt : row0;
    int64_t ti = row * hd + i;
    float c = ti < cos_len ? ct[ti] : 1.0f;
    float s = ti < sin_len ? st[ti] : 0.0f;
    float2 a = reinterpret_cast<const float2*>(x)[p];
    float2 r;
    r.x = a.x * c - a.y * s;
    r.y = a.x * s + a.y * c;
    reinterpret_cast<float2*>(out)[p] = r;
}

// apply_rope with whole float4s: one workgroup per token (grid.y; every vector of a token
// uses table row row0 + token, or row0 for all with tl_cpu's rule), T threads x F float4
// (F T = 1024) of the token's vpt * hd floats (grid.x slabs of 1024 float4).  hd / 4 is a
// power of two dividing T, so a thread's F float4 sit at the same offset i0 of their head
// vectors and one float4 each of the cos and sin rows serves all of them (pairs (i0, i0+1), (i0+2, i0+3)
// take entries i0 and i0 + 2, as k_apply_rope).  No 64-bit division; x read and out written
// non-temporal.
template <int F = 4, int T = 256>
__global__ __launch_bounds__(T) void k_apply_rope4(const float* __restrict__ x, const float* __restrict__ ct,
                                                     const float* __restrict__ st, float* __restrict__ out,
                                                     int64_t units, int hd4, int64_t row0, int per_token,
                                                     int64_t cos_len, int64_t sin_len) {
    asm volatile("" : : "s"(x), "s"(ct), "s"(st), "s"(out), "s"(units), "s"(hd4), "s"(row0), "s"(per_token),
                 "s"(cos_len), "s"(sin_len));
    const int64_t tok = blockIdx.y;
    const int64_t u0 = (int64_t)blockIdx.x * (F * T) + threadIdx.x;  // float4 index within the token
    const int i0 = 4 * (threadIdx.x & (hd4 - 1));                  // offset within the head vector
    const int64_t ti = (per_token ? row0 + tok : row0) * (int64_t)hd4 * 4 + i0;
    float c0, c2, s0, s2;
    if (ti + 4 <= cos_len && ti + 4 <= sin_len) {
        const float4 c = *reinterpret_cast<const float4*>(ct + ti), sn = *reinterpret_cast<const float4*>(st + ti);
        c0 = c.x, c2 = c.z, s0 = sn.x, s2 = sn.z;
    } else {  // beyond a short table: identity, as k_apply_rope
        c0 = ti < cos_len ? ct[ti] : 1.0f;
        c2 = ti + 2 < cos_len ? ct[ti + 2] : 1.0f;
        s0 = ti < sin_len ? st[ti] : 0.0f;
        s2 = ti + 2 < sin_len ? st[ti + 2] : 0.0f;
    }
    const float4* xt = reinterpret_cast<const float4*>(x) + tok * units;
    float4* ot = reinterpret_cast<float4*>(out) + tok * units;
    float4 a[F];
#pragma unroll
    for (int k = 0; k < F; k++) {
        const int64_t u = u0 + T * k;
        a[k] = u < units ? ld_nt(xt + u) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int k = 0; k < F; k++) {
        const int64_t u = u0 + T * k;
        if (u >= units) break;
        float4 r;
        r.x = a[k].x * c0 - a[k].y * s0;
        r.y = a[k].x * s0 + a[k].y * c0;
        r.z = a[k].z * c2 - a[k].w * s2;
        r.w = a[k].z * s2 + a[k].w * c2;
        st_nt(ot + u, r);
    }
}

// --------------------------------------------------------------- elementwise --------
// op: 0 add, 1 mul, 2 sub, 3 div  (tensor.rs:549-621)
__device__ __forceinline__ float binop(int op, float a, float b) {
    switch (op) {
        case 0: return a + b;
        case 1: return a * b;
        case 2: return a - b;
        default: return a / b;
    }
}

struct BStrides {
    int64_t out_stride[TL_HIP_MAX_RANK];
    int64_t a_stride[TL_HIP_MAX_RANK];
    int64_t b_stride[TL_HIP_MAX_RANK];
    int nd;
};

__global__ void k_binop_same(const float* __restrict__ a, const float* __restrict__ b,
                             float* __restrict__ o, int64_t n, int op) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = binop(op, a[i], b[i]);
}

__global__ void k_binop_bcast(const float* __restrict__ a, const float* __restrict__ b,
                              float* __restrict__ o, int64_t n, int op, BStrides st) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t rem = i, ai = 0, bi = 0;
    for (int d = 0; d < st.nd; d++) {
        int64_t c = rem / st.out_stride[d];
        rem -= c * st.out_stride[d];
        ai += c * st.a_stride[d];
        bi += c * st.b_stride[d];
    }
    o[i] = binop(op, a[ai], b[bi]);
}

__global__ void k_scale(const float* __restrict__ x, float* __restrict__ o, int64_t n, float s) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = x[i] * s;
}

// silu (ffi.rs:2097-2113): x * (1 / (1 + exp(-x)))
__global__ void k_silu(const float* __restrict__ x, float* __restrict__ o, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = x[i];
        o[i] = v * (1.0f / (1.0f + expf(-v)));
    }
}

// SwiGLU.  mode 0: silu(g) * u with the silu of ffi.rs:2102 then mul (chatbot.tl:33-38);
// mode 1: (g / (1 + exp(-g))) * u (fused_silu_mul, tl_cpu fused_ops.rs:15-35).
__global__ void k_swiglu(const float* __restrict__ g, const float* __restrict__ u,
                         float* __restrict__ o, int64_t n, int mode) {
    int64_t i4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i4 * 4 + 3 < n) {
        float4 a = reinterpret_cast<const float4*>(g)[i4];
        float4 b = reinterpret_cast<const float4*>(u)[i4];
        float4 r;
        if (mode == 0) {
            r.x = (a.x * (1.0f / (1.0f + expf(-a.x)))) * b.x;
            r.y = (a.y * (1.0f / (1.0f + expf(-a.y)))) * b.y;
            r.z = (a.z * (1.0f / (1.0f + expf(-a.z)))) * b.z;
            r.w = (a.w * (1.0f / (1.0f + expf(-a.w)))) * b.w;
        } else {
            r.x = (a.x / (1.0f + expf(-a.x))) * b.x;
            r.y = (a.y / (1.0f + expf(-a.y))) * b.y;
            r.z = (a.z / (1.0f + expf(-a.z))) * b.z;
            r.w = (a.w / (1.0f + expf(-a.w))) * b.w;
        }
        reinterpret_cast<float4*>(o)[i4] = r;
    } else {
        for (int64_t i = i4 * 4; i < n; i++) {
            float a = g[i];
            o[i] = mode == 0 ? (a * (1.0f / (1.0f + expf(-a)))) * u[i] : (a / (1.0f + expf(-a))) * u[i];
        }
    }
}

int launch_swiglu(const float* g, const float* u, float* o, int64_t n, int mode, hipStream_t s) {
    if (n <= 0) return TL_HIP_OK;
    if (((uintptr_t)g | (uintptr_t)u | (uintptr_t)o) % 16 != 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: swiglu operands must be 16-byte aligned");
        return TL_HIP_ERR_ARG;
    }
    k_swiglu<<<cdiv(cdiv(n, 4), 256), 256, 0, s>>>(g, u, o, n, mode);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "swiglu launch");
}

// ------------------------------------------------------------------ softmax ---------
// Row softmax over the last dim (tensor.rs:1065-1092): max, e = exp(x - max), sum, e / sum.
// One workgroup of 512 threads per row with the row in registers (V float4 per thread),
// so x is read once and written once.
template <int V>
__global__ __launch_bounds__(512) void k_softmax_row(const float* __restrict__ x,
                                                     float* __restrict__ out, int64_t n) {
    __shared__ float red[8];
    const int64_t row = blockIdx.x;
    const float4* xr = reinterpret_cast<const float4*>(x + row * n);
    const int64_t n4 = n >> 2;
    float4 v[V];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < V; i++) {
        int64_t j = threadIdx.x + (int64_t)i * 512;
        v[i] = j < n4 ? xr[j] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        mx = fmaxf(mx, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    }
    mx = block_max(mx, red);
    // exp(x - max) as the hardware exp2 of (x - max) log2 e and one reciprocal per row: about
    // 2e-6 relative error against expf and the divide, and four VALU instructions per element
    // instead of ~25, which kept the kernel VALU-bound after its single read (27.8 us at
    // [512, 32000] before, ~60 % of HBM peak)
    constexpr float L2E = 1.44269504088896341f;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        int64_t j = threadIdx.x + (int64_t)i * 512;
        if (j < n4) {
            v[i].x = __builtin_amdgcn_exp2f((v[i].x - mx) * L2E);
            v[i].y = __builtin_amdgcn_exp2f((v[i].y - mx) * L2E);
            v[i].z = __builtin_amdgcn_exp2f((v[i].z - mx) * L2E);
            v[i].w = __builtin_amdgcn_exp2f((v[i].w - mx) * L2E);
            sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        }
    }
    sum = block_sum(sum, red);
    const float inv = 1.0f / sum;
    float4* o = reinterpret_cast<float4*>(out + row * n);
#pragma unroll
    for (int i = 0; i < V; i++) {
        int64_t j = threadIdx.x + (int64_t)i * 512;
        if (j < n4) {
            float4 r;
            r.x = v[i].x * inv;
            r.y = v[i].y * inv;
            r.z = v[i].z * inv;
            r.w = v[i].w * inv;
            o[j] = r;
        }
    }
}

// strided softmax for any axis / size: one thread per (outer, inner) column, three passes
__global__ void k_softmax_strided(const float* __restrict__ x, float* __restrict__ out,
                                  int64_t outer, int64_t as, int64_t inner) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= outer * inner) return;
    int64_t i = t / inner, kk = t % inner;
    const float* xp = x + i * as * inner + kk;
    float* op = out + i * as * inner + kk;
    float mx = -INFINITY;
    for (int64_t j = 0; j < as; j++) {
        float v = xp[j * inner];
        if (v > mx) mx = v;
    }
    float sum = 0.f;
    for (int64_t j = 0; j < as; j++) {
        float e = expf(xp[j * inner] - mx);
        op[j * inner] = e;
        sum += e;
    }
    for (int64_t j = 0; j < as; j++) op[j * inner] = op[j * inner] / sum;
}

int launch_softmax(const float* x, float* out, int64_t outer, int64_t as, int64_t inner,
                   hipStream_t s) {
    if (outer * as * inner == 0) return TL_HIP_OK;
    const bool vec = inner == 1 && as % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0;
    const int64_t per = cdiv(as / 4, 512);
    if (vec && per <= 2)
        k_softmax_row<2><<<outer, 512, 0, s>>>(x, out, as);
    else if (vec && per <= 4)
        k_softmax_row<4><<<outer, 512, 0, s>>>(x, out, as);
    else if (vec && per <= 8)
        k_softmax_row<8><<<outer, 512, 0, s>>>(x, out, as);
    else if (vec && per <= 16)
        k_softmax_row<16><<<outer, 512, 0, s>>>(x, out, as);
    else
        k_softmax_strided<<<cdiv(outer * inner, 256), 256, 0, s>>>(x, out, outer, as, inner);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "softmax launch");
}

// ------------------------------------------------------------ data movement ---------
// out[i, j, r, k] = x[i, j, k] for r < repeats (repeat_interleave, tensor.rs:1178-1200)
__global__ void k_repeat_interleave(const float* __restrict__ x, float* __restrict__ o,
                                    int64_t total, int64_t as, int64_t inner, int64_t rep) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    int64_t kk = t % inner;
    int64_t rest = t / inner;
    int64_t jr = rest % (as * rep);
    int64_t i = rest / (as * rep);
    o[t] = x[(i * as + jr / rep) * inner + kk];
}

// generic slab copy: out[i, off + j, k] = x[i, j, k] -- narrow (tensor.rs:989-1015) and
// cat (tensor.rs:1021-1063) are built from it.
__global__ void k_slab_copy(const float* __restrict__ x, float* __restrict__ o, int64_t outer,
                            int64_t in_as, int64_t in_start, int64_t len, int64_t out_as,
                            int64_t out_start, int64_t inner) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= outer * len * inner) return;
    int64_t kk = t % inner;
    int64_t j = (t / inner) % len;
    int64_t i = t / (inner * len);
    o[(i * out_as + out_start + j) * inner + kk] = x[(i * in_as + in_start + j) * inner + kk];
}

struct TStrides {
    int64_t out_stride[TL_HIP_MAX_RANK];  // strides of the output index space
    int64_t in_stride[TL_HIP_MAX_RANK];   // input stride for each output dim
    int nd;
};

__global__ void k_permute(const float* __restrict__ x, float* __restrict__ o, int64_t n,
                          TStrides st) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    int64_t rem = t, src = 0;
    for (int d = 0; d < st.nd; d++) {
        int64_t c = rem / st.out_stride[d];
        rem -= c * st.out_stride[d];
        src += c * st.in_stride[d];
    }
    o[t] = x[src];
}

// 2-D transpose through a 32 x 33 LDS tile (coalesced reads and writes)
__global__ void k_transpose2d(const float* __restrict__ a, float* __restrict__ o, int64_t rows,
                              int64_t cols) {
    __shared__ float tile[32][33];
    int64_t bx = (int64_t)blockIdx.x * 32, by = (int64_t)blockIdx.y * 32;
    int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 32 x 8
    for (int j = ty; j < 32; j += 8) {
        int64_t r = by + j, c = bx + tx;
        if (r < rows && c < cols) tile[j][tx] = a[r * cols + c];
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        int64_t r = bx + j, c = by + tx;  // output [cols, rows]
        if (r < cols && c < rows) o[r * rows + c] = tile[tx][j];
    }
}

__global__ void k_causal_mask(float* __restrict__ o, int64_t size) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= size * size) return;
    int64_t i = t / size, j = t % size;
    o[t] = j > i ? -INFINITY : 0.0f;
}

__global__ void k_embedding(const float* __restrict__ table, const int32_t* __restrict__ ids,
                            float* __restrict__ o, int64_t n, int64_t dim) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * dim) return;
    int64_t i = t / dim, j = t % dim;
    o[t] = table[(int64_t)ids[i] * dim + j];
}

// ------------------------------------------------------------------- argmax ---------
// Greedy choice (tensor.rs:1633-1637, 841-846): the left fold keeps the running best only
// when it compares strictly greater, so the last of equal maxima wins.  For NaN-free input
// that is the associative (max value, last index) reduction done here; if any NaN is
// present the fold is not associative and thread 0 replays it sequentially.
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int64_t n,
                                                 int32_t* __restrict__ out_idx) {
    __shared__ float sv[16];
    __shared__ int si[16];
    __shared__ int has_nan;
    if (threadIdx.x == 0) has_nan = 0;
    __syncthreads();
    float bv = -INFINITY;
    int bi = -1;  // n <= INT32_MAX (checked by the launcher)
    int nan_seen = 0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        float v = x[i];
        if (v != v) nan_seen = 1;
        if (bi < 0 || !(bv > v)) {  // later index wins ties (i increases per thread)
            bv = v;
            bi = (int)i;
        }
    }
    if (nan_seen) has_nan = 1;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    // keep the pair a fold would keep: larger value, ties -> larger index
    int nan_any = 0;
    argmax_allreduce(bv, bi, nan_any);
    if (lane == 0) {
        sv[w] = bv;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float fv = sv[0];
        int64_t fi = si[0];
        for (int i = 1; i < (int)(blockDim.x >> 6); i++) {
            if (si[i] >= 0 && (fi < 0 || sv[i] > fv || (sv[i] == fv && si[i] > fi))) {
                fv = sv[i];
                fi = si[i];
            }
        }
        if (has_nan) {
            fi = 0;
            for (int64_t i = 1; i < n; i++)
                if (!(x[fi] > x[i])) fi = i;
        }
        *out_idx = (int32_t)(fi < 0 ? 0 : fi);
    }
}

int launch_argmax(const float* x, int64_t n, int32_t* out_idx, hipStream_t s) {
    if (n > INT32_MAX) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: argmax returns an int32 index: n <= 2^31 - 1");
        return TL_HIP_ERR_ARG;
    }
    k_argmax<<<1, 1024, 0, s>>>(x, n, out_idx);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "argmax launch");
}

// repetition penalty (device_impl.rs:967-1001): entries flagged in `seen` get v / p when
// v > 0, else v * p, in every row.
__global__ void k_rep_penalty(const float* __restrict__ x, const uint8_t* __restrict__ seen,
                              float* __restrict__ o, int64_t rows, int64_t vocab, float p) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * vocab) return;
    float v = x[t];
    if (seen[t % vocab]) v = v > 0.0f ? v / p : v * p;
    o[t] = v;
}

int launch_rep_penalty(const float* x, const uint8_t* seen, float* o, int64_t rows,
                       int64_t vocab, float p, hipStream_t s) {
    k_rep_penalty<<<cdiv(rows * vocab, 256), 256, 0, s>>>(x, seen, o, rows, vocab, p);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "repetition penalty launch");
}

// ------------------------------------------------------------- top-p sampling ---------
// The stochastic branch of sample_impl (tensor.rs:1641-1679) for a given uniform draw u:
//   p_i = x_i / temp, m = max p, prob_i = expf(p_i - m) / sum_j expf(p_j - m);
//   order = the indices by descending prob, equal probs in index order (a stable sort);
//   the cutoff is the first place in that order where the running sum of probs exceeds top_p
//   (else the last place), cutoff_prob the running sum there;
//   r = (f32) u * cutoff_prob, and the first place up to the cutoff where the running sum
//   reaches r is chosen (order[0] when there is none).
// A NaN among the p, or a max that is not finite, makes every prob NaN in the reference:
// nothing compares, the order stays the index order and index 0 is chosen.
// The order is never built.  "The first place where the running sum crosses T" is found by
// a radix descent over the prob bits (non-negative floats order as their bit patterns):
// three 10-bit digits from the top, each a histogram of (count, sum) over the elements that
// share the digits found so far; the bin where everything above it plus the bin crosses T
// holds the place, and a bin holding one element is the place itself (the descent stops
// there).  After the last digit the prob value v there is known exactly and every larger
// prob is summed; the place is the j-th element of value v in index order, j the rank at
// which the sum crosses.  Sums are fixed point (prob * 2^47, integers, independent of
// the order they are added in), so the choice is deterministic; they are the exact sums the
// reference's f32 running sums round, and the two choices agree wherever T is not within that
// rounding of a running sum.  Elements of prob 0 never move a running sum across T and are
// skipped.
constexpr int SMP_T = 1024;                      // one workgroup
constexpr int SMP_E = 16;                        // elements per thread and round, loads issued together
constexpr int64_t SMP_ROUND = (int64_t)SMP_T * SMP_E;
constexpr double SMP_SCALE = 140737488355328.0;  // 2^47: a bin's sum stays below 2^48
constexpr unsigned long long SMP_LOW48 = (1ull << 48) - 1ull;

__device__ __forceinline__ unsigned long long smp_fx(uint32_t key) {
    return (unsigned long long)((double)__uint_as_float(key) * SMP_SCALE);  // prob <= 1
}

struct SmpCross {
    uint32_t key;              // prob bits of the place (the bits under `mask`)
    uint32_t rank;             // 1-based rank among the elements of that prob, in index order
    unsigned long long sum;    // running sum before the place's bin / at the place (fixed point)
    int found;
    uint32_t mask;             // bits of key that are known: all, or the leading digits of the
                               // place's bin when that bin holds the place alone
    unsigned long long bin;    // the bin's sum (fixed point)
};

constexpr int SMP_RE = 32;  // elements per thread kept in registers: n <= SMP_T * SMP_RE (vocab sizes)
// Radix digits of the descents: keys of probs <= 1 are below 2^30 (0x3F800000 at most), three
// levels of 10 bits, 1024 bins each
constexpr int SMP_DB = 10, SMP_NB = 1 << SMP_DB, SMP_LEVELS = 3;

struct SmpShared {
    uint32_t cnt[SMP_NB];
    unsigned long long sum[SMP_NB];
    // the top level's histogram as the cut's descent built it: the choice's descent has no
    // digits yet at that level either, so it reuses it (top_kept)
    uint32_t cnt0[SMP_NB];
    unsigned long long sum0[SMP_NB];
    int top_kept;
    uint32_t wtot[SMP_T / 64];
    uint32_t rc[SMP_RE * (SMP_T / 64)];  // (row, wavefront) match counts of smp_nth_reg
    SmpCross res;
    int64_t pick;
    float red[SMP_T / 64];
};

// f(i, x[i]) for every element, thread tid taking i = round base + e * SMP_T + tid: the
// SMP_E loads of a round are in flight together.
template <typename F>
__device__ __forceinline__ void smp_each(const float* __restrict__ x, int64_t n, F f) {
    for (int64_t base = 0; base < n; base += SMP_ROUND) {
        float v[SMP_E];
#pragma unroll
        for (int e = 0; e < SMP_E; e++) {
            const int64_t i = base + (int64_t)e * SMP_T + threadIdx.x;
            v[e] = i < n ? x[i] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < SMP_E; e++) {
            const int64_t i = base + (int64_t)e * SMP_T + threadIdx.x;
            if (i < n) f(i, v[e]);
        }
    }
}

// Wavefront sum of fixed-point values held as doubles: every partial sum is an integer below
// 2^53 (all probs add up to about 2^47), so double additions are exact in any order.  Lane
// exchanges by permlane swaps across rows and DPP row rotations within them, as wave_allsum.
__device__ __forceinline__ double smp_bits_d(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(double, (unsigned long long)hi << 32 | lo);
}
template <int OFF>
__device__ __forceinline__ double smp_xor_d(double v) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    return smp_bits_d(lane_xor_u32<OFF>((uint32_t)b), lane_xor_u32<OFF>((uint32_t)(b >> 32)));
}
template <int CTRL>
__device__ __forceinline__ double smp_dpp_d(double v) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    return smp_bits_d((uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)b, CTRL, 0xF, 0xF, true),
                      (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ unsigned long long smp_wave_sum(unsigned long long x) {
    double v = (double)x;
    v += smp_xor_d<32>(v);
    v += smp_xor_d<16>(v);
    v += smp_dpp_d<0x128>(v);
    v += smp_dpp_d<0x124>(v);
    v += smp_dpp_d<0x122>(v);
    v += smp_dpp_d<0x121>(v);
    return (unsigned long long)v;
}

// One element into the level's histogram (every lane of the wavefront calls it; `in` says
// whether this lane's key takes part).  A wavefront whose 16 or more takers share the first
// taker's bin adds them with one reduction and one atomic pair; the rest add their own.
// PACK (at most 65535 elements per bin): count and sum share one 64-bit word, the count in
// bits 48-63 -- one atomic per element instead of two.
template <bool PACK>
__device__ __forceinline__ void smp_add(uint32_t k, bool in, uint32_t dig, SmpShared& sh) {
    // (k is opaque here so the compiler does not hoist every key's 64-bit fixed-point value out
    // of the level loop: 32 of them would not fit in the registers beside the keys)
    asm volatile("" : "+v"(k));
    unsigned long long pb = __ballot(in);
    if (pb == 0) return;
    const int lane = threadIdx.x & 63;
    bool own = in;
    for (int peel = 0; peel < 4 && __popcll(pb) >= 16; peel++) {
        const int first = __builtin_amdgcn_readfirstlane(__ffsll(pb) - 1);
        const uint32_t d0 = __builtin_amdgcn_readlane(dig, first);
        const bool grp = own && dig == d0;
        const unsigned long long gb = __ballot(grp);
        if (__popcll(gb) < 16) break;
        const unsigned long long v = smp_wave_sum(grp ? smp_fx(k) : 0ull);
        if (lane == first) {
            if constexpr (PACK) {
                atomicAdd(&sh.sum[d0], (unsigned long long)__popcll(gb) << 48 | v);
            } else {
                atomicAdd(&sh.cnt[d0], (uint32_t)__popcll(gb));
                atomicAdd(&sh.sum[d0], v);
            }
        }
        own = own && !grp;
        pb &= ~gb;
    }
    if (own) {
        if constexpr (PACK) {
            atomicAdd(&sh.sum[dig], 1ull << 48 | smp_fx(k));
        } else {
            atomicAdd(&sh.cnt[dig], 1u);
            atomicAdd(&sh.sum[dig], smp_fx(k));
        }
    }
}

// First place in the order where the running sum is > t (strict) or >= t.  each(f) calls
// f(key) for every element with the same trip count in every lane (keys past n are 0).
// Every thread calls it and gets the result.
// keep: the top level's histogram is kept for a later descent (cnt0 / sum0, top_kept);
// otherwise a kept top level is reused instead of built again.
template <bool PACK, typename EachKey>
__device__ __forceinline__ SmpCross smp_cross(EachKey each, unsigned long long t, bool strict, SmpShared& sh,
                                              bool keep) {
    constexpr int PERL = SMP_NB / 64;  // bins per lane in the scan
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t prefix = 0, mask = 0;
    unsigned long long above = 0;
    for (int d = SMP_LEVELS - 1; d >= 0; d--) {
        const int s = SMP_DB * d;
        if (d == SMP_LEVELS - 1 && !keep && sh.top_kept) {
            for (int b = tid; b < SMP_NB; b += SMP_T) {
                sh.cnt[b] = sh.cnt0[b];
                sh.sum[b] = sh.sum0[b];
            }
            __syncthreads();
        } else {
            for (int b = tid; b < SMP_NB; b += SMP_T) {
                sh.cnt[b] = 0;
                sh.sum[b] = 0;
            }
            __syncthreads();
            each([&](uint32_t k) {
                smp_add<PACK>(k, k != 0u && (k & mask) == prefix, (k >> s) & (uint32_t)(SMP_NB - 1), sh);
            });
            __syncthreads();
            if (keep && d == SMP_LEVELS - 1) {
                for (int b = tid; b < SMP_NB; b += SMP_T) {  // read here, rewritten only after the next barriers
                    sh.cnt0[b] = sh.cnt[b];
                    sh.sum0[b] = sh.sum[b];
                }
                if (tid == 0) sh.top_kept = 1;
            }
        }
        if (tid < 64) {
            // lane l holds bins NB - 1 - PERL l - q, q < PERL (the running sum goes from the top
            // bin down): an exclusive scan over the lanes gives each lane its starting sum
            // (the bins are read twice, for the lane's total and then for the crossing, rather
            // than held in registers beside the 32 keys of the descents)
            unsigned long long loc = 0;
#pragma unroll 4
            for (int q = 0; q < PERL; q++) {
                const unsigned long long w = sh.sum[SMP_NB - 1 - PERL * lane - q];
                loc += PACK ? w & SMP_LOW48 : w;
            }
            unsigned long long inc = loc;
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned long long y = __shfl_up(inc, off);
                if (lane >= off) inc += y;
            }
            unsigned long long run = above + inc - loc, hit_run = 0, hit_sum = 0;
            uint32_t hit_cnt = 0;
            int hit = -1;
#pragma unroll 4
            for (int q = 0; q < PERL; q++) {
                const int b = SMP_NB - 1 - PERL * lane - q;
                const unsigned long long w = sh.sum[b];
                const uint32_t c = PACK ? (uint32_t)(w >> 48) : sh.cnt[b];
                const unsigned long long sm = PACK ? w & SMP_LOW48 : w;
                if (!c) continue;
                const unsigned long long nx = run + sm;
                if (hit < 0 && (strict ? nx > t : nx >= t)) {
                    hit = q;
                    hit_run = run;
                    hit_cnt = c;
                    hit_sum = sm;
                }
                run = nx;
            }
            const unsigned long long hb = __ballot(hit >= 0);
            if (hb == 0) {
                if (lane == 0) sh.res = SmpCross{0u, 0u, 0ull, 0, 0u, 0ull};
            } else if (lane == __ffsll(hb) - 1) {
                sh.res = SmpCross{(uint32_t)(SMP_NB - 1 - PERL * lane - hit), hit_cnt, hit_run, 1, 0u, hit_sum};
            }
        }
        __syncthreads();
        const SmpCross r = sh.res;
        __syncthreads();  // sh is rewritten by the next level
        if (!r.found) return r;
        prefix |= r.key << s;
        mask = d == 0 ? ~0u : mask | (uint32_t)(SMP_NB - 1) << s;  // all bits known after the last digit
        above = r.sum;
        if (r.rank == 1)  // the bin holds one element: it is the place
            return SmpCross{prefix, 1u, above + r.bin, 1, mask, r.bin};
        if (d == 0) {
            // r.rank elements of value v, in index order: the j-th moves the sum across t
            // (above <= t when strict, above < t otherwise: the place was not passed yet)
            const unsigned long long v = smp_fx(prefix);  // > 0: a bin of zero sum never crosses t
            unsigned long long j = v == 0 ? 1 : strict ? (t - above) / v + 1 : (t - above + v - 1) / v;
            if (j < 1) j = 1;
            if (j > r.rank) j = r.rank;
            return SmpCross{prefix, (uint32_t)j, above + j * v, 1, ~0u, v};
        }
    }
    return SmpCross{0u, 0u, 0ull, 0, 0u, 0ull};
}

// Whether place a comes after place b in the order.  Compared on the bits both know: a
// partial key is the only element of its bin, so a place that matches it there is the same
// element.
__device__ __forceinline__ bool smp_after(const SmpCross& a, const SmpCross& b) {
    const uint32_t m = a.mask & b.mask;
    if ((a.key & m) != (b.key & m)) return (a.key & m) < (b.key & m);
    return a.mask == ~0u && b.mask == ~0u && a.rank > b.rank;
}

// Index of the j-th element (1-based, index order) whose key is kv, keys in global memory:
// thread t counts its contiguous chunk, a workgroup scan places the chunk, and its owner
// walks it.
__device__ int64_t smp_nth(const uint32_t* __restrict__ key, int64_t n, uint32_t kv, uint32_t km, uint32_t j,
                           SmpShared& sh) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t c_len = (n + SMP_T - 1) / SMP_T, lo = tid * c_len, hi = lo + c_len < n ? lo + c_len : n;
    uint32_t c = 0;
    for (int64_t b = lo; b < hi; b += SMP_E) {
        uint32_t kk[SMP_E];
#pragma unroll
        for (int e = 0; e < SMP_E; e++) kk[e] = b + e < hi ? key[b + e] : 0u;
#pragma unroll
        for (int e = 0; e < SMP_E; e++) c += kk[e] != 0u && (kk[e] & km) == kv;
    }
    uint32_t inc = c;  // inclusive scan over the wavefront
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(inc, off);
        if (lane >= off) inc += y;
    }
    if (lane == 63) sh.wtot[w] = inc;
    if (tid == 0) sh.pick = 0;
    __syncthreads();
    uint32_t woff = 0;
    for (int q = 0; q < w; q++) woff += sh.wtot[q];
    const uint32_t ex = woff + inc - c;
    if (c && ex < j && j <= ex + c) {
        uint32_t need = j - ex;
        for (int64_t i = lo; i < hi; i++)
            if (key[i] != 0u && (key[i] & km) == kv && --need == 0) {
                sh.pick = i;
                break;
            }
    }
    __syncthreads();
    return sh.pick;
}

// The same for keys in LDS, element i = e * SMP_T + tid at lk[i] (rows e < re): index order
// is row e, then wavefront, then lane.  Per (row, wavefront) counts go to LDS; wavefront 0
// scans the SMP_RE * 16 counts (eight per lane) and the chosen wavefront finds its lane in
// one ballot.
__device__ __forceinline__ int64_t smp_nth_lds(const uint32_t* lk, int re, uint32_t target, uint32_t km, uint32_t j,
                                               SmpShared& sh) {
    constexpr int NW = SMP_T / 64, PER = SMP_RE * NW / 64;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    auto hit = [&](int e) {
        const uint32_t k = e < re ? lk[e * SMP_T + tid] : 0u;
        return k != 0u && (k & km) == target;
    };
#pragma unroll 4
    for (int e = 0; e < SMP_RE; e++) {
        const unsigned long long b = __ballot(hit(e));
        if (lane == 0) sh.rc[e * NW + w] = (uint32_t)__popcll(b);
    }
    if (tid == 0) sh.pick = 0;
    __syncthreads();
    if (tid < 64) {
        uint32_t c[PER], loc = 0;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            c[q] = sh.rc[lane * PER + q];
            loc += c[q];
        }
        uint32_t inc = loc;
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_up(inc, off);
            if (lane >= off) inc += y;
        }
        uint32_t run = inc - loc;
        if (run < j && j <= inc) {  // this lane's counts hold the j-th
#pragma unroll
            for (int q = 0; q < PER; q++) {
                if (run < j && j <= run + c[q]) {
                    sh.res = SmpCross{(uint32_t)(lane * PER + q), j - run, 0ull, 1, 0u, 0ull};  // (row, wavefront), rank there
                }
                run += c[q];
            }
        }
    }
    __syncthreads();
    const uint32_t rw = sh.res.key, need = sh.res.rank;
    const int e_pick = (int)(rw / NW), w_pick = (int)(rw % NW);
    if (w == w_pick) {
        const unsigned long long b = __ballot(hit(e_pick));
        const unsigned long long below = lane ? b & ((1ull << lane) - 1ull) : 0ull;
        if (((b >> lane) & 1ull) && (uint32_t)__popcll(below) + 1 == need) sh.pick = (int64_t)e_pick * SMP_T + tid;
    }
    __syncthreads();
    return sh.pick;
}

// RES: n <= SMP_T * SMP_RE, every logit and key held in registers (one load pass, no scratch);
// otherwise the keys go to `key` (n words) and every pass reads them back.
template <bool RES>
__device__ __forceinline__ int64_t smp_choose(const float* __restrict__ x, int64_t n, float temp, float top_p,
                                              float u, uint32_t* __restrict__ key, SmpShared& sh) {
    const int tid = threadIdx.x;
    // p = x / temp and its max (the fold `if a > b { a } else { b }`: the max value when no
    // p is NaN)
    float mx = -INFINITY, se = 0.f;
    int bad = 0;
    unsigned long long tot = 0;  // exact sum of every prob
    uint32_t bk = 0u;            // the largest key and its lowest index (order[0])
    int bi = 0x7fffffff;
    // RES: the keys in dynamic LDS (element i at lk[i]), re rows of SMP_T
    extern __shared__ uint32_t smp_lds_keys[];
    uint32_t* const lk = smp_lds_keys;
    const int re = (int)((n + SMP_T - 1) / SMP_T);
    if constexpr (RES) {
        float pv[SMP_RE];
#pragma unroll
        for (int e = 0; e < SMP_RE; e++) {
            const int64_t i = (int64_t)e * SMP_T + tid;
            pv[e] = i < n ? x[i] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < SMP_RE; e++) {
            if ((int64_t)e * SMP_T + tid >= n) continue;
            pv[e] = pv[e] / temp;
            bad |= pv[e] != pv[e];
            mx = mx > pv[e] ? mx : pv[e];
        }
        bad = __syncthreads_or(bad);
        mx = block_max(mx, sh.red);
        if (bad || !(fabsf(mx) <= 3.402823466e38f)) return 0;
#pragma unroll
        for (int e = 0; e < SMP_RE; e++) {
            if ((int64_t)e * SMP_T + tid >= n) continue;
            pv[e] = expf(pv[e] - mx);
            se += pv[e];
        }
        se = block_sum(se, sh.red);
#pragma unroll
        for (int e = 0; e < SMP_RE; e++) {
            const uint32_t k = (int64_t)e * SMP_T + tid < n ? __float_as_uint(pv[e] / se) : 0u;
            if (e < re) lk[e * SMP_T + tid] = k;
            tot += smp_fx(k);
            if (k > bk) {  // rows in index order: the first of equal keys stays
                bk = k;
                bi = e * SMP_T + tid;
            }
        }
    } else {
        smp_each(x, n, [&](int64_t, float xv) {
            const float p = xv / temp;
            bad |= p != p;
            mx = mx > p ? mx : p;
        });
        bad = __syncthreads_or(bad);
        mx = block_max(mx, sh.red);
        if (bad || !(fabsf(mx) <= 3.402823466e38f)) return 0;
        smp_each(x, n, [&](int64_t, float xv) { se += expf(xv / temp - mx); });
        se = block_sum(se, sh.red);
        smp_each(x, n, [&](int64_t i, float xv) {
            const uint32_t k = __float_as_uint(expf(xv / temp - mx) / se);
            key[i] = k;
            tot += smp_fx(k);
            if (k > bk) {
                bk = k;
                bi = (int)i;
            }
        });
    }
    // order[0]: the largest key, lowest index among equal ones -- the max of key << 32 | ~index
    {
        unsigned long long v = (unsigned long long)bk << 32 | (uint32_t)~(uint32_t)bi;
        auto vmax = [&](double o) {
            const unsigned long long w = __builtin_bit_cast(unsigned long long, o);
            v = w > v ? w : v;
        };
        vmax(smp_xor_d<32>(__builtin_bit_cast(double, v)));  // (bit moves only: no float arithmetic)
        vmax(smp_xor_d<16>(__builtin_bit_cast(double, v)));
        vmax(smp_dpp_d<0x128>(__builtin_bit_cast(double, v)));
        vmax(smp_dpp_d<0x124>(__builtin_bit_cast(double, v)));
        vmax(smp_dpp_d<0x122>(__builtin_bit_cast(double, v)));
        vmax(smp_dpp_d<0x121>(__builtin_bit_cast(double, v)));
        bk = (uint32_t)(v >> 32);
        bi = (int)~(uint32_t)v;
    }
    tot = smp_wave_sum(tot);
    __syncthreads();  // key[] complete for the workgroup
    if ((tid & 63) == 0) {
        sh.sum[tid >> 6] = tot;
        sh.wtot[tid >> 6] = bk;
        sh.rc[tid >> 6] = (uint32_t)bi;
    }
    __syncthreads();
    tot = 0;
    for (int q = 0; q < SMP_T / 64; q++) {
        tot += sh.sum[q];
        const uint32_t ok = sh.wtot[q];
        const int oi = (int)sh.rc[q];
        if (ok > bk || (ok == bk && oi < bi)) {
            bk = ok;
            bi = oi;
        }
    }
    __syncthreads();
    // cutoff: first running sum > top_p (a NaN top_p compares false: no cutoff; the sum of
    // all probs is about 1, so no top_p >= 2^16 is exceeded either).  When order[0] alone
    // exceeds top_p it is the cut, r <= its prob, and it is the choice: no descent.
    const bool has_cut = top_p == top_p && top_p < 65536.0f;
    const unsigned long long tcut = top_p < 0.0f ? 0ull : (unsigned long long)floor((double)top_p * SMP_SCALE);
    if (has_cut && smp_fx(bk) > tcut) return bi;
    auto each = [&](auto f) {
        if constexpr (RES) {
            // unrolled by four only: the descents inline this loop, and a fully unrolled body
            // made the kernel 108 KB of code
            for (int e0 = 0; e0 < re; e0 += 4) {  // four LDS reads in flight, then their four keys
                uint32_t kk[4];
#pragma unroll
                for (int q = 0; q < 4; q++) kk[q] = e0 + q < re ? lk[(e0 + q) * SMP_T + tid] : 0u;
#pragma unroll
                for (int q = 0; q < 4; q++) f(kk[q]);
            }
        } else {
            for (int64_t base = 0; base < n; base += SMP_ROUND) {  // the same trip counts in every lane
                uint32_t kk[SMP_E];
#pragma unroll
                for (int e = 0; e < SMP_E; e++) {
                    const int64_t i = base + (int64_t)e * SMP_T + tid;
                    kk[e] = i < n ? key[i] : 0u;
                }
#pragma unroll
                for (int e = 0; e < SMP_E; e++) f(kk[e]);
            }
        }
    };
    SmpCross cut{0u, 0u, 0ull, 0, 0u, 0ull};
    if (tid == 0) sh.top_kept = 0;
    __syncthreads();
    if (has_cut) cut = smp_cross<RES>(each, tcut, true, sh, true);
    const float cutoff_prob = (float)((double)(cut.found ? cut.sum : tot) / SMP_SCALE);
    const float r = u * cutoff_prob;
    __syncthreads();  // top_kept as the cut left it
    SmpCross pick = smp_cross<RES>(each, (unsigned long long)ceil((double)r * SMP_SCALE), false, sh, false);
    if (!pick.found || (cut.found && smp_after(pick, cut))) return bi;  // no running sum up to the cut reaches r
    if constexpr (RES) return smp_nth_lds(lk, re, pick.key, pick.mask, pick.rank, sh);
    else return smp_nth(key, n, pick.key, pick.mask, pick.rank, sh);
}

// FIN: the decode step's form -- u is draws[*step], and the choice is recorded as
// k_argmax_finish records the greedy one: token, output slot, step counter, penalty mask,
// position.  Otherwise the index goes to out[0] as a float (the [1] tensor of sample_impl).
template <bool RES, bool FIN>
__global__ __launch_bounds__(SMP_T) void k_sample_top_p(const float* __restrict__ x, int64_t n, float temp,
                                                        float top_p, float u, uint32_t* __restrict__ key,
                                                        float* __restrict__ out, SmpFin fin) {
    __shared__ SmpShared sh;
    int step0 = 0;
    if constexpr (FIN) {
        step0 = *fin.step;
        u = fin.draws[step0 < fin.max_out ? step0 : 0];
    }
    const int64_t idx = smp_choose<RES>(x, n, temp, top_p, u, key, sh);
    if (threadIdx.x == 0) {
        if constexpr (FIN) {
            st_wt(fin.tok_out, (int32_t)idx);
            if (fin.out_ids) {
                if (step0 < fin.max_out) st_wt(fin.out_ids + step0, (int32_t)idx);
                st_wt(fin.step, (int32_t)(step0 + 1));
            }
            if (fin.seen_out) st_wt(fin.seen_out + idx, (uint8_t)1);
            if (fin.pos_inc) st_wt(fin.pos_inc, (int32_t)(*fin.pos_inc + 1));
        } else {
            *out = (float)idx;
        }
    }
}

int launch_sample_top_p(const float* x, int64_t n, float temp, float top_p, float u, uint32_t* key, float* out,
                        const SmpFin* fin, hipStream_t s) {
    if (n < 1 || n > INT32_MAX) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: top-p sampling takes 1 .. 2^31 - 1 logits");
        return TL_HIP_ERR_ARG;
    }
    const bool res = n <= (int64_t)SMP_T * SMP_RE;
    if (!res && !key) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: top-p sampling over more than %d logits needs a key scratch",
                  SMP_T * SMP_RE);
        return TL_HIP_ERR_ARG;
    }
    const SmpFin f = fin ? *fin : SmpFin{};
    // the RES form keeps every key in LDS: 128 KB beside the static state (one workgroup per CU);
    // the attribute is set at each launch, so it holds on whichever device is current
    constexpr size_t lds = (size_t)SMP_T * SMP_RE * sizeof(uint32_t);
    if (res) {
        const void* kern = fin ? (const void*)k_sample_top_p<true, true> : (const void*)k_sample_top_p<true, false>;
        const hipError_t attr = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr != hipSuccess) return hip_fail(attr, "hipFuncSetAttribute(sampling LDS)");
    }
    if (fin) {
        if (res) k_sample_top_p<true, true><<<1, SMP_T, lds, s>>>(x, n, temp, top_p, u, nullptr, out, f);
        else k_sample_top_p<false, true><<<1, SMP_T, 0, s>>>(x, n, temp, top_p, u, key, out, f);
    } else {
        if (res) k_sample_top_p<true, false><<<1, SMP_T, lds, s>>>(x, n, temp, top_p, u, nullptr, out, f);
        else k_sample_top_p<false, false><<<1, SMP_T, 0, s>>>(x, n, temp, top_p, u, key, out, f);
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "top-p sampling launch");
}

int sample_key_words(int64_t n) { return n <= (int64_t)SMP_T * SMP_RE ? 0 : (int)n; }

int launch_embedding(const float* table, const int32_t* ids, float* o, int64_t n, int64_t dim,
                     hipStream_t s) {
    if (n * dim == 0) return TL_HIP_OK;
    k_embedding<<<cdiv(n * dim, 256), 256, 0, s>>>(table, ids, o, n, dim);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "embedding launch");
}

int launch_apply_rope(const float* x, const float* ct, const float* st, float* out,
                      int64_t total, int64_t hd, int64_t cos_len, int64_t sin_len, int64_t row0,
                      int64_t vpt, hipStream_t s) {
    if (total == 0 || hd == 0) return TL_HIP_OK;
    // whole float4s, one workgroup row per token: hd / 4 a power of two up to 256, 16-byte
    // aligned data, whole tokens
    const int64_t hd4 = hd / 4, tok_floats = vpt > 0 ? vpt * hd : total;
    const bool vec4 = hd % 4 == 0 && hd4 <= 256 && (hd4 & (hd4 - 1)) == 0 && total % tok_floats == 0 &&
                      total / tok_floats <= 65535 && cdiv(tok_floats / 4, 1024) <= 0x7fffffff &&
                      (((uintptr_t)x | (uintptr_t)out | (uintptr_t)ct | (uintptr_t)st) & 15) == 0;
    if (vec4) {
        const int64_t units = tok_floats / 4;
        const dim3 grid((unsigned)cdiv(units, 1024), (unsigned)(total / tok_floats));
        // head vectors up to 512 elements: 128 threads x 8 float4 ([512, 32, 128]: 4.35 -> 4.3 us)
        if (hd4 <= 128)
            k_apply_rope4<8, 128><<<grid, 128, 0, s>>>(x, ct, st, out, units, (int)hd4, row0, vpt > 0, cos_len, sin_len);
        else
            k_apply_rope4<4, 256><<<grid, 256, 0, s>>>(x, ct, st, out, units, (int)hd4, row0, vpt > 0, cos_len, sin_len);
    } else {
        int64_t np = total / 2;
        k_apply_rope<<<cdiv(np, 256), 256, 0, s>>>(x, ct, st, out, np, hd, cos_len, sin_len, row0, vpt);
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "apply_rope launch");
}

int launch_rope_table(float* out, int64_t seq_len, int64_t dim, float base, int is_sin,
                      hipStream_t s) {
    int64_t n = seq_len * (dim / 2);
    if (n == 0) return TL_HIP_OK;
    k_rope_table<<<cdiv(n, 256), 256, 0, s>>>(out, seq_len, dim, base, is_sin);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "rope table launch");
}

// The uniform draws of tl_hip_tensor_sample: splitmix64 per calling thread (the reference
// draws from rand's thread-local generator, tensor.rs:1663-1666), seeded from the OS until
// tl_hip_sample_seed fixes it; a draw is the top 53 bits scaled by 2^-53, in [0, 1), the
// construction of rand's `gen::<f64>()`.
static thread_local uint64_t g_smp_state = 0;
static thread_local bool g_smp_seeded = false;

void sample_seed(uint64_t seed) {
    g_smp_state = seed;
    g_smp_seeded = true;
}

double sample_draw() {
    if (!g_smp_seeded) {
        std::random_device rd;
        g_smp_state = ((uint64_t)rd() << 32) ^ (uint64_t)rd();
        g_smp_seeded = true;
    }
    uint64_t z = (g_smp_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) * 0x1.0p-53;
}

}  // namespace tlhip

// GpuFusedOps::fused_rotary_emb as tl_cpu computes it (fused_ops.rs:87-108): the reference
// loop over id < count / 2 writes out[id] (first element of id's pair) and out[id + half]
// (second element), later ids overwriting earlier ones on a zero-filled output.  Element i
// therefore holds the first-element value of id = i when i < count / 2, else the
// second-element value of id = i - half when that id exists, else 0 -- one thread per
// element, no write order to keep.
__global__ void k_fused_rotary(const float* __restrict__ x, const float* __restrict__ freqs, float* __restrict__ o,
                               int64_t count, int64_t half) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const int64_t h2 = count / 2;
    const bool first = i < h2, second = !first && i - half >= 0 && i - half < h2;
    float v = 0.f;
    if (first || second) {
        const int64_t id = first ? i : i - half;
        const float f = freqs[id % half], c = cosf(f), sn = sinf(f);
        const float x0 = x[id], x1 = x[id + half];
        v = first ? x0 * c - x1 * sn : x0 * sn + x1 * c;
    }
    o[i] = v;
}

// GpuFusedOps::fused_add_relu (tl_cpu fused_ops.rs:110-120): (a + b).max(0), NaN -> 0
__global__ void k_fused_add_relu(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ o,
                                 int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = fmaxf(a[i] + b[i], 0.f);
}

// GpuFusedOps::fused_bias_gelu (tl_cpu fused_ops.rs:122-131) with that crate's gelu
// (fused_ops.rs:20-22): v = x + bias[i % nbias], 0.5 v (1 + tanh(2/sqrt(pi) (v + 0.044715 v^3)))
__global__ void k_fused_bias_gelu(const float* __restrict__ x, const float* __restrict__ bias, float* __restrict__ o,
                                  int64_t n, int64_t nbias) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i] + bias[i % nbias];
    const float v3 = (v * v) * v;
    o[i] = 0.5f * v * (1.0f + tanhf(1.12837916709551257390f * (v + 0.044715f * v3)));
}

// =============================================================== C ABI wrappers ======
using namespace tlhip;

static const Tensor* CT(const tl_hip_tensor* h) { return reinterpret_cast<const Tensor*>(h); }

static bool need(const tl_hip_tensor* a, const char* what) {
    if (!a) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: %s", what);
        return false;
    }
    if (CT(a)->dtype != TL_HIP_F32) {
        set_error(TL_HIP_ERR_TYPE, "TypeMismatch: %s must be f32", what);
        return false;
    }
    return state() != nullptr;
}

static tl_hip_tensor* finish(Tensor* o, int rc) {
    if (rc != TL_HIP_OK) {
        tensor_drop(o);
        return nullptr;
    }
    return H(o);
}

static int last_launch(const char* what) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, what);
}

extern "C" {

tl_hip_tensor* tl_hip_tensor_rms_norm(const tl_hip_tensor* x, const tl_hip_tensor* w, float eps) {
    if (!need(x, "input")) return nullptr;
    const Tensor* t = CT(x);
    int64_t n = t->rank ? t->shape[t->rank - 1] : 1;
    if (w) {
        // the weight is applied by a broadcast mul (tensor.rs:549-609); only a trailing
        // [n] (or [1, n]) weight broadcasts against every row
        if (CT(w)->dtype != TL_HIP_F32 || CT(w)->numel != n) {
            set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: rms_norm weight has %lld elements, last dim is %lld",
                      (long long)CT(w)->numel, (long long)n);
            return nullptr;
        }
    }
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    int64_t rows = n ? t->numel / n : 0;
    return finish(o, launch_rmsnorm(t->f32(), nullptr, w ? CT(w)->f32() : nullptr, o->f32(), rows,
                                    n, eps, 0, cur_stream()));
}

tl_hip_tensor* tl_hip_fused_rms_norm(const tl_hip_tensor* x, const tl_hip_tensor* w, float eps) {
    if (!need(x, "input") || !need(w, "weight")) return nullptr;
    const Tensor* t = CT(x);
    int64_t n = t->rank ? t->shape[t->rank - 1] : 1;
    if (CT(w)->numel < n) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: fused_rms_norm weight shorter than last dim");
        return nullptr;
    }
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    return finish(o, launch_rmsnorm(t->f32(), nullptr, CT(w)->f32(), o->f32(), n ? t->numel / n : 0,
                                    n, eps, 1, cur_stream()));
}

tl_hip_tensor* tl_hip_fused_add_rms_norm(const tl_hip_tensor* x, const tl_hip_tensor* r,
                                         const tl_hip_tensor* w, float eps) {
    if (!need(x, "input") || !need(r, "residual") || !need(w, "weight")) return nullptr;
    const Tensor* t = CT(x);
    if (CT(r)->numel != t->numel) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: fused_add_rms_norm: shape mismatch");
        return nullptr;
    }
    int64_t n = t->rank ? t->shape[t->rank - 1] : 1;
    if (CT(w)->numel < n) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: fused_add_rms_norm weight shorter than last dim");
        return nullptr;
    }
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    return finish(o, launch_rmsnorm(t->f32(), CT(r)->f32(), CT(w)->f32(), o->f32(),
                                    n ? t->numel / n : 0, n, eps, 1, cur_stream()));
}

static tl_hip_tensor* rope_table(int64_t dim, int64_t seq_len, float base, int is_sin) {
    if (!state()) return nullptr;
    if (dim < 0 || seq_len < 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: negative rope table size");
        return nullptr;
    }
    int64_t shape[2] = {seq_len, dim};
    Tensor* o = tensor_alloc(shape, 2);
    if (!o) return nullptr;
    if (dim % 2 && o->numel) (void)hipMemsetAsync(o->data, 0, o->numel * 4, cur_stream());
    return finish(o, launch_rope_table(o->f32(), seq_len, dim, base, is_sin, cur_stream()));
}

tl_hip_tensor* tl_hip_tensor_rope_new_cos(int64_t dim, int64_t seq_len, float base) {
    return rope_table(dim, seq_len, base, 0);
}

tl_hip_tensor* tl_hip_tensor_rope_new_sin(int64_t dim, int64_t seq_len, float base) {
    return rope_table(dim, seq_len, base, 1);
}

static tl_hip_tensor* rope(const tl_hip_tensor* x, const tl_hip_tensor* c, const tl_hip_tensor* s,
                           int64_t row0, int64_t vpt) {
    if (!need(x, "input") || !need(c, "cos table") || !need(s, "sin table")) return nullptr;
    const Tensor* t = CT(x);
    int64_t hd = t->rank ? t->shape[t->rank - 1] : 0;
    if (hd % 2) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: apply_rope needs an even head_dim, got %lld",
                  (long long)hd);
        return nullptr;
    }
    if (row0 < 0 || vpt < 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: negative position");
        return nullptr;
    }
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    return finish(o, launch_apply_rope(t->f32(), CT(c)->f32(), CT(s)->f32(), o->f32(), t->numel, hd,
                                       CT(c)->numel, CT(s)->numel, row0, vpt, cur_stream()));
}

tl_hip_tensor* tl_hip_tensor_apply_rope(const tl_hip_tensor* x, const tl_hip_tensor* c,
                                        const tl_hip_tensor* s) {
    return rope(x, c, s, 0, 0);
}

tl_hip_tensor* tl_hip_tensor_apply_rope_pos(const tl_hip_tensor* x, const tl_hip_tensor* c,
                                            const tl_hip_tensor* s, int64_t pos0, int64_t vpt) {
    if (vpt <= 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: vectors_per_token must be positive");
        return nullptr;
    }
    return rope(x, c, s, pos0, vpt);
}

tl_hip_tensor* tl_hip_tensor_silu(const tl_hip_tensor* x) {
    if (!need(x, "input")) return nullptr;
    const Tensor* t = CT(x);
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    if (t->numel) k_silu<<<cdiv(t->numel, 256), 256, 0, cur_stream()>>>(t->f32(), o->f32(), t->numel);
    return finish(o, last_launch("silu launch"));
}

tl_hip_tensor* tl_hip_fused_rotary_emb(const tl_hip_tensor* x, const tl_hip_tensor* freqs, int64_t head_dim) {
    if (!need(x, "input") || !need(freqs, "freqs")) return nullptr;
    const Tensor* t = CT(x);
    const int64_t half = head_dim / 2, count = t->numel;
    // the reference indexes freqs[0 .. half) and x[0 .. count / 2 + half) (fused_ops.rs:93-100)
    if (half < 1 || CT(freqs)->numel < half || (count > 0 && count / 2 + half > count)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: fused_rotary_emb: head_dim %lld with %lld elements and %lld freqs",
                  (long long)head_dim, (long long)count, (long long)CT(freqs)->numel);
        return nullptr;
    }
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    if (count)
        k_fused_rotary<<<cdiv(count, 256), 256, 0, cur_stream()>>>(t->f32(), CT(freqs)->f32(), o->f32(), count, half);
    return finish(o, last_launch("fused rotary launch"));
}

tl_hip_tensor* tl_hip_fused_add_relu(const tl_hip_tensor* a, const tl_hip_tensor* b) {
    if (!need(a, "lhs") || !need(b, "rhs")) return nullptr;
    if (CT(a)->numel != CT(b)->numel) {  // the reference asserts equal counts (fused_ops.rs:112)
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: fused_add_relu: shape mismatch");
        return nullptr;
    }
    const Tensor* t = CT(a);
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    if (t->numel)
        k_fused_add_relu<<<cdiv(t->numel, 256), 256, 0, cur_stream()>>>(t->f32(), CT(b)->f32(), o->f32(), t->numel);
    return finish(o, last_launch("fused add-relu launch"));
}

tl_hip_tensor* tl_hip_fused_bias_gelu(const tl_hip_tensor* x, const tl_hip_tensor* bias) {
    if (!need(x, "input") || !need(bias, "bias")) return nullptr;
    if (CT(bias)->numel < 1) {  // i % 0 in the reference
        set_error(TL_HIP_ERR_ARG, "ArgumentError: fused_bias_gelu: empty bias");
        return nullptr;
    }
    const Tensor* t = CT(x);
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    if (t->numel)
        k_fused_bias_gelu<<<cdiv(t->numel, 256), 256, 0, cur_stream()>>>(t->f32(), CT(bias)->f32(), o->f32(), t->numel,
                                                                          CT(bias)->numel);
    return finish(o, last_launch("fused bias-gelu launch"));
}

tl_hip_tensor* tl_hip_fused_silu_mul(const tl_hip_tensor* g, const tl_hip_tensor* u) {
    if (!need(g, "gate") || !need(u, "up")) return nullptr;
    if (CT(g)->numel != CT(u)->numel) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: fused_silu_mul: shape mismatch");
        return nullptr;
    }
    const Tensor* t = CT(g);
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    return finish(o, launch_swiglu(t->f32(), CT(u)->f32(), o->f32(), t->numel, 1, cur_stream()));
}

static tl_hip_tensor* binary(const tl_hip_tensor* ah, const tl_hip_tensor* bh, int op) {
    if (!need(ah, "lhs") || !need(bh, "rhs")) return nullptr;
    const Tensor* a = CT(ah);
    const Tensor* b = CT(bh);
    if (a->numel == 0 || b->numel == 0) {  // tensor.rs:550-559: empty -> shape [0]
        int64_t z = 0;
        return H(tensor_alloc(&z, 1));
    }
    int nd = a->rank > b->rank ? a->rank : b->rank;
    int64_t as[TL_HIP_MAX_RANK], bs[TL_HIP_MAX_RANK], os[TL_HIP_MAX_RANK];
    for (int d = 0; d < nd; d++) {
        as[d] = d < nd - a->rank ? 1 : a->shape[d - (nd - a->rank)];
        bs[d] = d < nd - b->rank ? 1 : b->shape[d - (nd - b->rank)];
        if (as[d] != bs[d] && as[d] != 1 && bs[d] != 1) {
            set_error(TL_HIP_ERR_SHAPE,
                      "ShapeMismatch: Operands could not be broadcast together (dim %d: %lld vs %lld)",
                      d, (long long)as[d], (long long)bs[d]);
            return nullptr;
        }
        os[d] = as[d] > bs[d] ? as[d] : bs[d];
    }
    Tensor* o = tensor_alloc(os, nd);
    if (!o) return nullptr;
    hipStream_t s = cur_stream();
    if (a->numel == o->numel && b->numel == o->numel) {
        k_binop_same<<<cdiv(o->numel, 256), 256, 0, s>>>(a->f32(), b->f32(), o->f32(), o->numel, op);
    } else {
        BStrides st;
        st.nd = nd;
        int64_t so = 1, sa = 1, sb = 1;
        for (int d = nd - 1; d >= 0; d--) {
            st.out_stride[d] = so;
            st.a_stride[d] = as[d] == 1 ? 0 : sa;
            st.b_stride[d] = bs[d] == 1 ? 0 : sb;
            so *= os[d];
            sa *= as[d];
            sb *= bs[d];
        }
        k_binop_bcast<<<cdiv(o->numel, 256), 256, 0, s>>>(a->f32(), b->f32(), o->f32(), o->numel, op, st);
    }
    return finish(o, last_launch("binop launch"));
}

tl_hip_tensor* tl_hip_tensor_add(const tl_hip_tensor* a, const tl_hip_tensor* b) { return binary(a, b, 0); }
tl_hip_tensor* tl_hip_tensor_mul(const tl_hip_tensor* a, const tl_hip_tensor* b) { return binary(a, b, 1); }
tl_hip_tensor* tl_hip_tensor_sub(const tl_hip_tensor* a, const tl_hip_tensor* b) { return binary(a, b, 2); }
tl_hip_tensor* tl_hip_tensor_div(const tl_hip_tensor* a, const tl_hip_tensor* b) { return binary(a, b, 3); }

tl_hip_tensor* tl_hip_tensor_scale(const tl_hip_tensor* x, float s) {
    if (!need(x, "input")) return nullptr;
    const Tensor* t = CT(x);
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    if (t->numel) k_scale<<<cdiv(t->numel, 256), 256, 0, cur_stream()>>>(t->f32(), o->f32(), t->numel, s);
    return finish(o, last_launch("scale launch"));
}

tl_hip_tensor* tl_hip_tensor_softmax(const tl_hip_tensor* x, int64_t dim) {
    if (!need(x, "input")) return nullptr;
    const Tensor* t = CT(x);
    int64_t ax = dim < 0 ? dim + t->rank : dim;
    if (ax < 0 || ax >= t->rank) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: softmax dim %lld out of range for rank %d",
                  (long long)dim, t->rank);
        return nullptr;
    }
    int64_t outer = 1, inner = 1;
    for (int d = 0; d < ax; d++) outer *= t->shape[d];
    for (int d = ax + 1; d < t->rank; d++) inner *= t->shape[d];
    Tensor* o = tensor_alloc(t->shape, t->rank);
    if (!o) return nullptr;
    return finish(o, launch_softmax(t->f32(), o->f32(), outer, t->shape[ax], inner, cur_stream()));
}

tl_hip_tensor* tl_hip_tensor_new_causal_mask(int64_t size) {
    if (!state()) return nullptr;
    if (size < 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: negative mask size");
        return nullptr;
    }
    int64_t shape[2] = {size, size};
    Tensor* o = tensor_alloc(shape, 2);
    if (!o) return nullptr;
    if (size) k_causal_mask<<<cdiv(size * size, 256), 256, 0, cur_stream()>>>(o->f32(), size);
    return finish(o, last_launch("causal mask launch"));
}

tl_hip_tensor* tl_hip_tensor_narrow(const tl_hip_tensor* x, int64_t dim, int64_t start, int64_t len) {
    if (!need(x, "input")) return nullptr;
    const Tensor* t = CT(x);
    if (dim < 0 || dim >= t->rank) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Slice axis %lld out of bounds for tensor of rank %d",
                  (long long)dim, t->rank);
        return nullptr;
    }
    if (start < 0 || len < 0 || start + len > t->shape[dim]) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Slice range %lld:%lld out of bounds for axis %lld of size %lld",
                  (long long)start, (long long)(start + len), (long long)dim, (long long)t->shape[dim]);
        return nullptr;
    }
    int64_t shape[TL_HIP_MAX_RANK];
    for (int d = 0; d < t->rank; d++) shape[d] = t->shape[d];
    shape[dim] = len;
    Tensor* o = tensor_alloc(shape, t->rank);
    if (!o) return nullptr;
    int64_t outer = 1, inner = 1;
    for (int d = 0; d < dim; d++) outer *= t->shape[d];
    for (int d = dim + 1; d < t->rank; d++) inner *= t->shape[d];
    if (o->numel)
        k_slab_copy<<<cdiv(o->numel, 256), 256, 0, cur_stream()>>>(t->f32(), o->f32(), outer, t->shape[dim],
                                                                    start, len, len, 0, inner);
    return finish(o, last_launch("narrow launch"));
}

tl_hip_tensor* tl_hip_tensor_cat(const tl_hip_tensor* ah, const tl_hip_tensor* bh, int64_t dim) {
    if (!need(ah, "lhs") || !need(bh, "rhs")) return nullptr;
    const Tensor* a = CT(ah);
    const Tensor* b = CT(bh);
    if (dim < 0 || dim >= a->rank) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Cat axis %lld out of bounds", (long long)dim);
        return nullptr;
    }
    if (b->rank != a->rank) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Tensor 1 has different rank");
        return nullptr;
    }
    for (int d = 0; d < a->rank; d++)
        if (d != dim && a->shape[d] != b->shape[d]) {
            set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Tensor 1 has mismatching shape at dim %d (expected %lld, got %lld)",
                      d, (long long)a->shape[d], (long long)b->shape[d]);
            return nullptr;
        }
    int64_t shape[TL_HIP_MAX_RANK];
    for (int d = 0; d < a->rank; d++) shape[d] = a->shape[d];
    shape[dim] = a->shape[dim] + b->shape[dim];
    Tensor* o = tensor_alloc(shape, a->rank);
    if (!o) return nullptr;
    int64_t outer = 1, inner = 1;
    for (int d = 0; d < dim; d++) outer *= a->shape[d];
    for (int d = dim + 1; d < a->rank; d++) inner *= a->shape[d];
    hipStream_t s = cur_stream();
    if (a->numel)
        k_slab_copy<<<cdiv(a->numel, 256), 256, 0, s>>>(a->f32(), o->f32(), outer, a->shape[dim], 0,
                                                       a->shape[dim], shape[dim], 0, inner);
    if (b->numel)
        k_slab_copy<<<cdiv(b->numel, 256), 256, 0, s>>>(b->f32(), o->f32(), outer, b->shape[dim], 0,
                                                       b->shape[dim], shape[dim], a->shape[dim], inner);
    return finish(o, last_launch("cat launch"));
}

tl_hip_tensor* tl_hip_tensor_repeat_interleave(const tl_hip_tensor* x, int64_t repeats, int64_t dim) {
    if (!need(x, "input")) return nullptr;
    const Tensor* t = CT(x);
    if (dim < 0 || dim >= t->rank) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Axis %lld out of bounds for repeat_interleave (rank %d)",
                  (long long)dim, t->rank);
        return nullptr;
    }
    if (repeats < 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: negative repeats");
        return nullptr;
    }
    int64_t shape[TL_HIP_MAX_RANK];
    for (int d = 0; d < t->rank; d++) shape[d] = t->shape[d];
    shape[dim] *= repeats;
    Tensor* o = tensor_alloc(shape, t->rank);
    if (!o) return nullptr;
    int64_t inner = 1;
    for (int d = dim + 1; d < t->rank; d++) inner *= t->shape[d];
    if (o->numel)
        k_repeat_interleave<<<cdiv(o->numel, 256), 256, 0, cur_stream()>>>(t->f32(), o->f32(), o->numel,
                                                                           t->shape[dim], inner, repeats);
    return finish(o, last_launch("repeat_interleave launch"));
}

tl_hip_tensor* tl_hip_tensor_transpose(const tl_hip_tensor* x, int64_t d0, int64_t d1) {
    if (!need(x, "input")) return nullptr;
    const Tensor* t = CT(x);
    if (t->rank < 2) return tl_hip_tensor_reshape(x, t->shape, t->rank);  // tensor.rs:903-905
    if (d0 < 0 || d1 < 0 || d0 >= t->rank || d1 >= t->rank) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Transpose dims %lld and %lld are out of bounds for tensor of rank %d",
                  (long long)d0, (long long)d1, t->rank);
        return nullptr;
    }
    int64_t shape[TL_HIP_MAX_RANK], in_stride[TL_HIP_MAX_RANK];
    int64_t st = 1;
    for (int d = t->rank - 1; d >= 0; d--) {
        in_stride[d] = st;
        st *= t->shape[d];
    }
    for (int d = 0; d < t->rank; d++) shape[d] = t->shape[d];
    shape[d0] = t->shape[d1];
    shape[d1] = t->shape[d0];
    Tensor* o = tensor_alloc(shape, t->rank);
    if (!o) return nullptr;
    TStrides ts;
    ts.nd = t->rank;
    int64_t so = 1;
    for (int d = t->rank - 1; d >= 0; d--) {
        ts.out_stride[d] = so;
        so *= shape[d];
        int src_dim = d == d0 ? (int)d1 : (d == d1 ? (int)d0 : d);
        ts.in_stride[d] = in_stride[src_dim];
    }
    if (o->numel) k_permute<<<cdiv(o->numel, 256), 256, 0, cur_stream()>>>(t->f32(), o->f32(), o->numel, ts);
    return finish(o, last_launch("transpose launch"));
}

tl_hip_tensor* tl_hip_tensor_transpose_2d(const tl_hip_tensor* x) {
    if (!need(x, "input")) return nullptr;
    const Tensor* t = CT(x);
    if (t->rank != 2) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: transpose_2d needs a 2-D tensor, got rank %d", t->rank);
        return nullptr;
    }
    int64_t shape[2] = {t->shape[1], t->shape[0]};
    Tensor* o = tensor_alloc(shape, 2);
    if (!o) return nullptr;
    if (o->numel) {
        dim3 grid((unsigned)cdiv(t->shape[1], 32), (unsigned)cdiv(t->shape[0], 32));
        k_transpose2d<<<grid, 256, 0, cur_stream()>>>(t->f32(), o->f32(), t->shape[0], t->shape[1]);
    }
    return finish(o, last_launch("transpose_2d launch"));
}

tl_hip_tensor* tl_hip_tensor_matmul(const tl_hip_tensor* ah, const tl_hip_tensor* bh) {
    if (!need(ah, "lhs") || !need(bh, "rhs")) return nullptr;
    const Tensor* a = CT(ah);
    const Tensor* b = CT(bh);
    if (a->rank < 1 || b->rank < 1) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Matmul requires at least 1D tensors");
        return nullptr;
    }
    int64_t m = a->rank >= 2 ? a->shape[a->rank - 2] : 1, k = a->shape[a->rank - 1];
    int64_t k2 = b->rank >= 2 ? b->shape[b->rank - 2] : b->shape[0];
    int64_t n = b->rank >= 2 ? b->shape[b->rank - 1] : 1;
    if (k != k2) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: Matmul shape mismatch (inner dims %lld vs %lld)",
                  (long long)k, (long long)k2);
        return nullptr;
    }
    int64_t batch = 1;
    for (int d = 0; d < a->rank - 2; d++) batch *= a->shape[d];
    int64_t b_batched = b->rank > 2;
    if (b_batched && b->numel != batch * k * n) {
        // matmul_impl indexes B batch b at b * k * n (tensor.rs:1285-1288)
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: batched rhs holds %lld elements, lhs batch needs %lld",
                  (long long)b->numel, (long long)(batch * k * n));
        return nullptr;
    }
    int64_t shape[TL_HIP_MAX_RANK];
    int r = 0;
    for (int d = 0; d < a->rank - 2; d++) shape[r++] = a->shape[d];
    shape[r++] = m;
    if (b->rank >= 2) shape[r++] = n;
    Tensor* o = tensor_alloc(shape, r);
    if (!o) return nullptr;
    if (k == 0) {
        if (o->numel) (void)hipMemsetAsync(o->data, 0, o->numel * 4, cur_stream());
        return H(o);
    }
    return finish(o, launch_matmul_f32(a->f32(), b->f32(), o->f32(), batch, m, k, n, m * k,
                                       b_batched ? k * n : 0, cur_stream()));
}

tl_hip_tensor* tl_hip_tensor_embedding(const tl_hip_tensor* wh, const tl_hip_tensor* ih) {
    if (!need(wh, "weight") || !need(ih, "indices")) return nullptr;
    const Tensor* w = CT(wh);
    const Tensor* ids = CT(ih);
    int64_t vocab = w->rank ? w->shape[0] : 0;
    int64_t dim = w->rank > 1 ? w->shape[1] : 1;
    std::vector<float> hid(ids->numel);
    if (tl_hip_tensor_to_host(ih, hid.data(), ids->numel) != TL_HIP_OK) return nullptr;
    std::vector<int32_t> iid(ids->numel);
    for (int64_t i = 0; i < ids->numel; i++) {
        float f = hid[i];
        // `as i64` truncates toward zero, saturating (NaN -> 0)
        int64_t id = f != f ? 0 : (f >= 9.2e18f ? INT64_MAX : (f <= -9.2e18f ? INT64_MIN : (int64_t)f));
        if (id < 0 || id >= vocab) {
            set_error(TL_HIP_ERR_INDEX, "IndexOutOfBounds: Embedding index %lld out of range for vocab size %lld",
                      (long long)id, (long long)vocab);
            return nullptr;
        }
        iid[i] = (int32_t)id;
    }
    int64_t shape[TL_HIP_MAX_RANK];
    if (ids->rank + 1 > TL_HIP_MAX_RANK) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: indices rank too large");
        return nullptr;
    }
    for (int d = 0; d < ids->rank; d++) shape[d] = ids->shape[d];
    shape[ids->rank] = dim;
    Tensor* o = tensor_alloc(shape, ids->rank + 1);
    if (!o) return nullptr;
    if (o->numel == 0) return H(o);
    int32_t* dids = (int32_t*)dev_alloc(iid.size() * 4);
    if (!dids) {
        tensor_drop(o);
        return nullptr;
    }
    hipStream_t s = cur_stream();
    hipError_t e = hipMemcpyAsync(dids, iid.data(), iid.size() * 4, hipMemcpyHostToDevice, s);
    int rc = e == hipSuccess ? launch_embedding(w->f32(), dids, o->f32(), ids->numel, dim, s)
                             : hip_fail(e, "hipMemcpyAsync(ids)");
    if (rc == TL_HIP_OK) {
        e = hipStreamSynchronize(s);  // iid (host) must outlive the copy
        if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    }
    dev_free(dids);
    return finish(o, rc);
}

int64_t tl_hip_tensor_argmax_all(const tl_hip_tensor* x) {
    if (!need(x, "input")) return -1;
    const Tensor* t = CT(x);
    if (t->numel == 0) return 0;  // unwrap_or(0), tensor.rs:845
    int32_t* d = (int32_t*)dev_alloc(4);
    if (!d) return -1;
    hipStream_t s = cur_stream();
    int32_t h = 0;
    int rc = launch_argmax(t->f32(), t->numel, d, s);
    if (rc == TL_HIP_OK) {
        hipError_t e = hipMemcpyAsync(&h, d, 4, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "argmax readback");
    }
    dev_free(d);
    return rc == TL_HIP_OK ? (int64_t)h : -1;
}

static tl_hip_tensor* sample(const tl_hip_tensor* x, float temp, float top_p, const double* u) {
    if (!need(x, "logits")) return nullptr;
    const Tensor* t = CT(x);
    if (t->numel == 0) {
        set_error(TL_HIP_ERR_INTERNAL, "InternalError: Empty tensor for sampling");
        return nullptr;
    }
    int64_t one = 1;
    if (temp <= 0.0f) {  // greedy (a NaN temp takes the stochastic branch, as in the reference)
        int64_t idx = tl_hip_tensor_argmax_all(x);
        if (idx < 0) return nullptr;
        float v = (float)idx;
        return tl_hip_tensor_new(&v, &one, 1);
    }
    const double draw = u ? *u : sample_draw();
    Tensor* o = tensor_alloc(&one, 1);
    if (!o) return nullptr;
    // the key scratch: only for inputs past what the kernel holds in registers
    uint32_t* key = nullptr;
    if (t->numel > (int64_t)SMP_T * SMP_RE && !(key = (uint32_t*)dev_alloc((size_t)t->numel * sizeof(uint32_t)))) {
        tensor_drop(o);
        return nullptr;
    }
    // T::from_f64(u): the draw rounded to f32 (tensor.rs:1666)
    int rc = launch_sample_top_p(t->f32(), t->numel, temp, top_p, (float)draw, key, o->f32(), nullptr, cur_stream());
    if (key) dev_free(key);
    return finish(o, rc);
}

tl_hip_tensor* tl_hip_tensor_sample(const tl_hip_tensor* x, float temp, float top_p) {
    return sample(x, temp, top_p, nullptr);
}

tl_hip_tensor* tl_hip_tensor_sample_uniform(const tl_hip_tensor* x, float temp, float top_p, double u) {
    if (!(u >= 0.0 && u < 1.0)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: the uniform draw must lie in [0, 1), got %g", u);
        return nullptr;
    }
    return sample(x, temp, top_p, &u);
}

void tl_hip_sample_seed(uint64_t seed) { sample_seed(seed); }

tl_hip_tensor* tl_hip_tensor_repetition_penalty(const tl_hip_tensor* lh, const tl_hip_tensor* th,
                                                double penalty) {
    if (!need(lh, "logits") || !need(th, "tokens")) return nullptr;
    const Tensor* l = CT(lh);
    const Tensor* tk = CT(th);
    int64_t vocab = l->rank ? l->shape[l->rank - 1] : 1;
    int64_t rows = vocab ? l->numel / vocab : 0;
    std::vector<float> tok(tk->numel);
    if (tk->numel && tl_hip_tensor_to_host(th, tok.data(), tk->numel) != TL_HIP_OK) return nullptr;
    std::vector<uint8_t> seen(vocab ? vocab : 1, 0);
    for (float f : tok) {
        // `as usize` saturates: NaN and negatives give 0
        uint64_t id = !(f >= 0.0f) ? 0 : (f >= 1.8e19f ? UINT64_MAX : (uint64_t)f);
        if (id < (uint64_t)vocab) seen[id] = 1;
    }
    Tensor* o = tensor_alloc(l->shape, l->rank);
    if (!o) return nullptr;
    if (l->numel == 0) return H(o);
    uint8_t* dseen = (uint8_t*)dev_alloc(seen.size());
    if (!dseen) {
        tensor_drop(o);
        return nullptr;
    }
    hipStream_t s = cur_stream();
    hipError_t e = hipMemcpyAsync(dseen, seen.data(), seen.size(), hipMemcpyHostToDevice, s);
    int rc = e == hipSuccess ? launch_rep_penalty(l->f32(), dseen, o->f32(), rows, vocab, (float)penalty, s)
                             : hip_fail(e, "hipMemcpyAsync(seen)");
    if (rc == TL_HIP_OK) {
        e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    }
    dev_free(dseen);
    return finish(o, rc);
}

}  // extern "C"
