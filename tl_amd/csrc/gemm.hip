// Dense contractions: the quantized prefill GEMM (Y = X . W^T, W Q4_0 / Q8_0 resident) in
// two precisions, and the plain f32 batched matmul behind tensor_matmul / matmul_4d.
//
//  * k_qgemm_f32   exact dequant (d * (q - 8) in f32) into LDS, f32 FMA accumulate.
//                  The "f32 path": max-rel-err 1e-4 class against tl_cpu.
//  * k_qgemm_mfma  dequant -> f16 LDS tiles -> v_mfma_f32_16x16x32_f16, f32 accumulate.
//                  The "f16 path": 1e-2 class.  X is rounded to f16 while it is staged.
//  * k_matmul_f32  CpuTensor::matmul_impl semantics (crates/tl_cpu/src/tensor.rs:1248-1313)
//                  for [batch, m, k] x [batch?, k, n].
#include "internal.h"

namespace tlhip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Dequantise the 32 weights of one block into v[32] (f32, exact).
template <int QT>
__device__ __forceinline__ void dequant_block(const uint8_t* __restrict__ qs,
                                              const __half* __restrict__ dsc, int64_t blk,
                                              float* v) {
    float d = __half2float(dsc[blk]);
    if constexpr (QT == TL_HIP_GGML_Q4_0) {
        uint4 w = *reinterpret_cast<const uint4*>(qs + blk * 16);
        const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t byte = (q[c] >> (8 * i)) & 0xFF;
                v[4 * c + i] = d * (float)((int)(byte & 0xF) - 8);
                v[16 + 4 * c + i] = d * (float)((int)(byte >> 4) - 8);
            }
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(qs + blk * 32);
        uint4 w0 = p[0], w1 = p[1];
        const uint32_t q[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int c = 0; c < 8; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) v[4 * c + i] = d * (float)(int8_t)((q[c] >> (8 * i)) & 0xFF);
    }
}

// ------------------------------------------------------------ f32 quantized GEMM ----
// Tile 64 (x rows) x 64 (weight rows) x 32 (one quant block); 256 threads, 4x4 outputs
// per thread.  LDS holds the k-major tiles Xs[32][64] and Ws[32][64].
constexpr int F_BM = 64, F_BN = 64, F_BK = 32;

template <int QT>
__global__ __launch_bounds__(256) void k_qgemm_f32(const uint8_t* __restrict__ qs,
                                                   const __half* __restrict__ dsc,
                                                   const float* __restrict__ x,
                                                   float* __restrict__ y, int64_t m, int64_t n,
                                                   int64_t k, int64_t nb) {
    __shared__ __attribute__((aligned(16))) float Xs[F_BK][F_BM + 4];
    __shared__ __attribute__((aligned(16))) float Ws[F_BK][F_BN + 4];
    const int t = threadIdx.x;
    const int tx = t & 15, ty = t >> 4;
    const int64_t m0 = (int64_t)blockIdx.y * F_BM, n0 = (int64_t)blockIdx.x * F_BN;
    float acc[4][4] = {};
    for (int64_t kb = 0; kb < nb; kb++) {
        // X tile: 64 rows x 32 floats -> 512 float4, 2 per thread
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int idx = t + i * 256;
            int r = idx >> 3, c4 = idx & 7;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m0 + r < m) v = *reinterpret_cast<const float4*>(x + (m0 + r) * k + kb * 32 + c4 * 4);
            Xs[c4 * 4 + 0][r] = v.x;
            Xs[c4 * 4 + 1][r] = v.y;
            Xs[c4 * 4 + 2][r] = v.z;
            Xs[c4 * 4 + 3][r] = v.w;
        }
        // W tile: 64 rows x one block, threads 0..63 dequantise a row each
        if (t < 64) {
            float v[32];
            int64_t row = n0 + t < n ? n0 + t : n - 1;
            dequant_block<QT>(qs, dsc, row * nb + kb, v);
#pragma unroll
            for (int j = 0; j < 32; j++) Ws[j][t] = v[j];
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < F_BK; kk++) {
            float4 a = *reinterpret_cast<const float4*>(&Xs[kk][ty * 4]);
            float4 b = *reinterpret_cast<const float4*>(&Ws[kk][tx * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int64_t r = m0 + ty * 4 + i;
        if (r >= m) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int64_t c = n0 + tx * 4 + j;
            if (c < n) y[r * n + c] = acc[i][j];
        }
    }
}

// ------------------------------------------------------- f16 MFMA quantized GEMM ----
// Tile BM (x rows) x BN (weight rows) x 64 (two quant blocks); 4 wavefronts in a 2x2
// grid, each computing (BM/2) x (BN/2) with 16x16x32 MFMAs.  LDS rows are padded to 72
// halves (144 B) so the 16 lanes that read one operand column hit distinct bank groups.
// Operand layout of v_mfma_f32_16x16x32_f16: lane l supplies A[l % 16][8*(l/16) .. +7]
// and B[8*(l/16) .. +7][l % 16]; it receives C[4*(l/16) .. +3][l % 16].
constexpr int M_LD = 72;

template <int QT, int BM, int BN>
__global__ __launch_bounds__(256) void k_qgemm_mfma(const uint8_t* __restrict__ qs,
                                                    const __half* __restrict__ dsc,
                                                    const float* __restrict__ x,
                                                    float* __restrict__ y, int64_t m,
                                                    int64_t n, int64_t k, int64_t nb) {
    __shared__ __attribute__((aligned(16))) _Float16 As[BM * M_LD];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * M_LD];
    constexpr int TM = BM / 32, TN = BN / 32;  // 16x16 tiles per wave in m / n
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int64_t kb = 0; kb < nb; kb += 2) {
        // ---- stage X: BM rows x 64 floats (16 float4 per row) -> f16
        constexpr int XV = BM * 16 / 256;
#pragma unroll
        for (int i = 0; i < XV; i++) {
            int idx = t + i * 256;
            int r = idx >> 4, c4 = idx & 15;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            int64_t kc = kb * 32 + c4 * 4;
            if (m0 + r < m && kc < k) v = *reinterpret_cast<const float4*>(x + (m0 + r) * k + kc);
            _Float16* dst = As + r * M_LD + c4 * 4;
            dst[0] = (_Float16)v.x;
            dst[1] = (_Float16)v.y;
            dst[2] = (_Float16)v.z;
            dst[3] = (_Float16)v.w;
        }
        // ---- stage W: BN rows x 2 blocks, dequantised then rounded to f16
        for (int idx = t; idx < BN * 2; idx += 256) {
            int r = idx >> 1, bsel = idx & 1;
            int64_t row = n0 + r < n ? n0 + r : n - 1;
            _Float16* dst = Bs + r * M_LD + bsel * 32;
            if (kb + bsel < nb) {
                float v[32];
                dequant_block<QT>(qs, dsc, row * nb + kb + bsel, v);
#pragma unroll
                for (int j = 0; j < 32; j++) dst[j] = (_Float16)v[j];
            } else {
#pragma unroll
                for (int j = 0; j < 32; j++) dst[j] = (_Float16)0.f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            half8 a[TM], b[TN];
            const int kcol = ks * 32 + (lane >> 4) * 8;
#pragma unroll
            for (int i = 0; i < TM; i++)
                a[i] = *reinterpret_cast<const half8*>(As + (wm * (BM / 2) + i * 16 + (lane & 15)) * M_LD + kcol);
#pragma unroll
            for (int j = 0; j < TN; j++)
                b[j] = *reinterpret_cast<const half8*>(Bs + (wn * (BN / 2) + j * 16 + (lane & 15)) * M_LD + kcol);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            int64_t c = n0 + wn * (BN / 2) + j * 16 + (lane & 15);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int64_t r = m0 + wm * (BM / 2) + i * 16 + (lane >> 4) * 4 + e;
                if (r < m && c < n) y[r * n + c] = acc[i][j][e];
            }
        }
}

int launch_quant_gemm(const QWeight* w, const float* x, float* y, int64_t m, hipStream_t s,
                      int mode) {
    if (m < 1) return TL_HIP_OK;
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: x must be 16-byte aligned");
        return TL_HIP_ERR_ARG;
    }
    const bool q4 = w->ggml_type == TL_HIP_GGML_Q4_0;
    if (mode == 0) {
        dim3 grid((unsigned)cdiv(w->n, F_BN), (unsigned)cdiv(m, F_BM));
        if (q4)
            k_qgemm_f32<TL_HIP_GGML_Q4_0><<<grid, 256, 0, s>>>(w->qs, w->d, x, y, m, w->n, w->k, w->nb);
        else
            k_qgemm_f32<TL_HIP_GGML_Q8_0><<<grid, 256, 0, s>>>(w->qs, w->d, x, y, m, w->n, w->k, w->nb);
    } else {
        constexpr int BM = 128, BN = 64;
        dim3 grid((unsigned)cdiv(w->n, BN), (unsigned)cdiv(m, BM));
        if (q4)
            k_qgemm_mfma<TL_HIP_GGML_Q4_0, BM, BN><<<grid, 256, 0, s>>>(w->qs, w->d, x, y, m, w->n, w->k, w->nb);
        else
            k_qgemm_mfma<TL_HIP_GGML_Q8_0, BM, BN><<<grid, 256, 0, s>>>(w->qs, w->d, x, y, m, w->n, w->k, w->nb);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "quant gemm launch");
    return TL_HIP_OK;
}

// ------------------------------------------------------------- f32 batched matmul ----
// C[b, i, j] = sum_p A[b, i, p] * B[b', p, j], b' = b when B is batched (b_bstride != 0).
// 64 x 64 tiles, k-steps of 16, 4 x 4 outputs per thread; f32 FMA accumulation.
constexpr int G_B = 64, G_K = 16;

__global__ __launch_bounds__(256) void k_matmul_f32(const float* __restrict__ A,
                                                    const float* __restrict__ B,
                                                    float* __restrict__ C, int64_t m,
                                                    int64_t k, int64_t n, int64_t a_bs,
                                                    int64_t b_bs) {
    __shared__ __attribute__((aligned(16))) float As[G_K][G_B + 4];
    __shared__ __attribute__((aligned(16))) float Bs[G_K][G_B + 4];
    const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
    const int64_t bz = blockIdx.z;
    const float* Ab = A + bz * a_bs;
    const float* Bb = B + bz * b_bs;
    float* Cb = C + bz * m * n;
    const int64_t m0 = (int64_t)blockIdx.y * G_B, n0 = (int64_t)blockIdx.x * G_B;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < k; k0 += G_K) {
        // A tile 64 x 16: 1024 elements, 4 per thread
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int idx = t + i * 256;
            int r = idx >> 4, c = idx & 15;
            float v = 0.f;
            if (m0 + r < m && k0 + c < k) v = Ab[(m0 + r) * k + k0 + c];
            As[c][r] = v;
        }
        // B tile 16 x 64
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int idx = t + i * 256;
            int r = idx >> 6, c = idx & 63;
            float v = 0.f;
            if (k0 + r < k && n0 + c < n) v = Bb[(k0 + r) * n + n0 + c];
            Bs[r][c] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < G_K; kk++) {
            float4 a = *reinterpret_cast<const float4*>(&As[kk][ty * 4]);
            float4 b = *reinterpret_cast<const float4*>(&Bs[kk][tx * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int64_t r = m0 + ty * 4 + i;
        if (r >= m) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int64_t c = n0 + tx * 4 + j;
            if (c < n) Cb[r * n + c] = acc[i][j];
        }
    }
}

int launch_matmul_f32(const float* a, const float* b, float* c, int64_t batch, int64_t m,
                      int64_t k, int64_t n, int64_t a_bstride, int64_t b_bstride,
                      hipStream_t s) {
    if (batch < 1 || m < 1 || n < 1) return TL_HIP_OK;
    if (batch > 65535) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: batch %lld exceeds 65535", (long long)batch);
        return TL_HIP_ERR_ARG;
    }
    dim3 grid((unsigned)cdiv(n, G_B), (unsigned)cdiv(m, G_B), (unsigned)batch);
    k_matmul_f32<<<grid, 256, 0, s>>>(a, b, c, m, k, n, a_bstride, b_bstride);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "matmul launch");
    return TL_HIP_OK;
}

}  // namespace tlhip
