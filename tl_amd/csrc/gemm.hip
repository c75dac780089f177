// Dense contractions: the quantized prefill GEMM (Y = X . W^T, W Q4_0 / Q8_0 resident) in
// two precisions, and the plain f32 batched matmul behind tensor_matmul / matmul_4d.
//
//  * k_qgemm_f32   exact dequant (all four types) into LDS, f32 FMA accumulate.
//                  The "f32 path": max-rel-err 1e-4 class against tl_cpu.
//  * k_qgemm_mfma  dequant -> f16 LDS tiles -> v_mfma_f32_16x16x32_f16, f32 accumulate.
//                  The "f16 path": 1e-2 class.  X is rounded to f16 while it is staged.
//  * k_matmul_f32  CpuTensor::matmul_impl semantics (crates/tl_cpu/src/tensor.rs:1248-1313)
//                  for [batch, m, k] x [batch?, k, n].
#include "internal.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace tlhip {

// tile plan of the calling thread's last f16 GEMM launch (tl_hip_debug_last_gemm_plan)
static thread_local int tls_plan[3] = {0, 0, 0};

// Residency buffers of a quantized weight (layout at struct QWeight).
struct QView {
    const uint8_t* qs;
    const __half* d;
    const uint8_t* hdr;
    const uint8_t* qh;
    const int8_t* sc;
};

// Q4_K sub-block j's d * scale and dmin * min from its resident super-block header
// (q4k_hdr_sm; QTensor::get_scale_min_k4, quantized.rs:405-415); both products are exact in f32.
__device__ __forceinline__ void q4k_scale_min(const uint4& hd, int j, float* d1, float* m1) {
    uint32_t sc, mn;
    q4k_hdr_sm(hd, j, &sc, &mn);
    *d1 = __half2float(__ushort_as_half((uint16_t)(hd.x & 0xFFFF))) * (float)sc;
    *m1 = __half2float(__ushort_as_half((uint16_t)(hd.x >> 16))) * (float)mn;
}

// Dequantise the 32 weights of unit blk into v[32] (f32, bit-identical to the reference's
// dequantizers: Q4_0 d * (q - 8), Q8_0 d * q, Q4_K (d sc) q - dmin m, Q6_K (d sc) (q - 32)).
template <int QT>
__device__ __forceinline__ void dequant_block(const QView& qv, int64_t blk, float* v) {
    if constexpr (QT == TL_HIP_GGML_Q4_0) {
        const float d = __half2float(qv.d[blk]);
        uint4 w = *reinterpret_cast<const uint4*>(qv.qs + blk * 16);
        const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t byte = (q[c] >> (8 * i)) & 0xFF;
                v[4 * c + i] = d * (float)((int)(byte & 0xF) - 8);
                v[16 + 4 * c + i] = d * (float)((int)(byte >> 4) - 8);
            }
    } else if constexpr (QT == TL_HIP_GGML_Q8_0) {
        const float d = __half2float(qv.d[blk]);
        const uint4* p = reinterpret_cast<const uint4*>(qv.qs + blk * 32);
        uint4 w0 = p[0], w1 = p[1];
        const uint32_t q[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int c = 0; c < 8; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) v[4 * c + i] = d * (float)(int8_t)((q[c] >> (8 * i)) & 0xFF);
    } else if constexpr (QT == TL_HIP_GGML_Q4_K) {
        float d1, m1;
        q4k_scale_min(reinterpret_cast<const uint4*>(qv.hdr)[blk >> 3], (int)(blk & 7), &d1, &m1);
        uint4 w = *reinterpret_cast<const uint4*>(qv.qs + blk * 16);
        const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t byte = (q[c] >> (8 * i)) & 0xFF;
                v[4 * c + i] = d1 * (float)(byte & 0xF) - m1;
                v[16 + 4 * c + i] = d1 * (float)(byte >> 4) - m1;
            }
    } else {
        const float d = __half2float(qv.d[blk >> 3]);
        const float e0 = d * (float)qv.sc[2 * blk], e1 = d * (float)qv.sc[2 * blk + 1];
        uint4 w = *reinterpret_cast<const uint4*>(qv.qs + blk * 16);
        const uint2 h = reinterpret_cast<const uint2*>(qv.qh)[blk];
        const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t byte = (q[c] >> (8 * i)) & 0xFF;
                const uint32_t h0 = (h.x >> (8 * i + 2 * c)) & 3, h1 = (h.y >> (8 * i + 2 * c)) & 3;
                v[4 * c + i] = e0 * (float)((int)((byte & 0xF) | (h0 << 4)) - 32);
                v[16 + 4 * c + i] = e1 * (float)((int)((byte >> 4) | (h1 << 4)) - 32);
            }
    }
}

// ------------------------------------------------------------ f32 quantized GEMM ----
// Tile 64 (x rows) x 64 (weight rows) x 32 (one quant block); 256 threads, 4x4 outputs
// per thread.  LDS holds the k-major tiles Xs[32][64] and Ws[32][64].
constexpr int F_BM = 64, F_BN = 64, F_BK = 32;

template <int QT>
__global__ __launch_bounds__(256) void k_qgemm_f32(QView qv, const float* __restrict__ x,
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
            dequant_block<QT>(qv, row * nb + kb, v);
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
// Y[m, n] = sum_k X[m, k] W[n, k] with v_mfma_f32_16x16x32_f16 and f32 accumulation.
// Operand layout: lane l supplies A[l % 16][8*(l/16) .. +7] and B[8*(l/16) .. +7][l % 16]
// and receives C[4*(l/16) .. +3][l % 16].
//
// X is first converted to f16 once (k_x_to_f16q), with every 32-element block stored in the
// k order of the MFMA operands below.  Workgroup tile BM (x rows) x BN (weight rows), eight
// wavefronts: four (BM/2) x (BN/2) output sub-tiles in a 2 x 2 grid, each held by two
// wavefronts that split an iteration's k-steps and add their sums once at the end (two
// wavefronts per SIMD: with one, the MFMA and LDS latencies of a single instruction stream
// stay exposed).  One iteration covers 128 k = 4 quant blocks with 4 MFMAs per 16 x 16
// output tile; in MFMA t, lane group g (lanes 16g .. 16g+15) supplies block kb+g's values
// held in word t of its quant data.
//   * X rows, W quant chunks and W scales reach LDS by global_load_lds (no VGPR staging),
//     double-buffered, with the next iteration's loads in flight during the MFMAs;
//   * each lane turns its W word t into the f16 operand of MFMA t in registers (Q4_0: fp8
//     reinterpretation of the nibble bytes, Q8_0: the 0x6400 magic), times the block scale
//     d with one f16 rounding (the f16 path's rounding);
//   * the A operand is one ds_read_b128 per 16 x 32 tile.
// Measured on MI355X (M = 512): the loads alone take about 60 % of the kernel time (an
// iteration moves 37 KB per workgroup from L2), the MFMA work alone about 50 %; larger
// tiles (64 x 128, 128 x 128) and 16-accumulator wavefronts measured slower.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
constexpr int Q_KR = 4;     // quant blocks per iteration

template <int QT>
struct QWords;
template <>
struct QWords<TL_HIP_GGML_Q4_0> {
    static constexpr int BYTES = 16;
    // f16 operand of MFMA t from word t of raw (the block's word t = bytes 4t .. 4t+3, i.e.
    // elements 4t..4t+3 (low nibbles) and 16+4t..16+4t+3 (high nibbles), in that order).
    // A byte holding one nibble q is, read as an OCP fp8 E4M3 value, exactly q * 2^-9, so
    // v_cvt_scalef32_pk_f16_fp8 with scale 2^9 turns two such bytes into the f16 pair (q, q')
    // (the instruction applies only the exponent of its scale, hence the separate d); then
    // fma(q, d, -8 d) = (q - 8) d with one rounding (-8 d is exact).
    __device__ static half8 operand(const uint4& raw, int t, half2v d2, half2v m8d2) {
        const uint32_t w = t == 0 ? raw.x : t == 1 ? raw.y : t == 2 ? raw.z : raw.w;
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        const half2v p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false);
        const half2v p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true);
        const half2v p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false);
        const half2v p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true);
        const half2v v0 = __builtin_elementwise_fma(p0, d2, m8d2), v1 = __builtin_elementwise_fma(p1, d2, m8d2);
        const half2v v2 = __builtin_elementwise_fma(p2, d2, m8d2), v3 = __builtin_elementwise_fma(p3, d2, m8d2);
        return half8{v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
    }
};
template <>
struct QWords<TL_HIP_GGML_Q8_0> {
    static constexpr int BYTES = 32;
    // words 2t, 2t+1 = elements 8t .. 8t+7 as pairs (8t, 8t+2) (8t+1, 8t+3) (8t+4, 8t+6)
    // (8t+5, 8t+7); (q ^ 0x80) | 0x6400 is 1024 + q + 128.  raw = the block's 16 bytes that
    // hold k-steps 2 kh and 2 kh + 1; tt selects the step (words 2 tt, 2 tt + 1).  One
    // v_perm_b32 per pair puts bytes 0 and 2 (or 1 and 3) of the word under 0x64 bytes.
    __device__ static half8 operand(const uint4& raw, int tt, half2v d2) {
        const uint32_t src[4] = {raw.x, raw.y, raw.z, raw.w};
        const half2v off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
        half8 r;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t w = src[2 * tt + h] ^ 0x80808080u;
#pragma unroll
            for (int p = 0; p < 2; p++) {
                // selector bytes 0-3 take w's bytes, 4 the constant's 0x64
                const uint32_t bits = __builtin_amdgcn_perm(0x64646464u, w, p ? 0x04030401u : 0x04020400u);
                const half2v v = (__builtin_bit_cast(half2v, bits) + off) * d2;
                r[4 * h + 2 * p] = v.x;
                r[4 * h + 2 * p + 1] = v.y;
            }
        }
        return r;
    }
};

// Q4_K units are resident in the Q4_0 nibble order: the same operand words, built with the
// unit's (d sc, -dmin m) pair in place of (d, -8 d).
template <>
struct QWords<TL_HIP_GGML_Q4_K> : QWords<TL_HIP_GGML_Q4_0> {};

// f16 weights already in the operand order (k_dequant_f16q): block = 4 words of 8 halves,
// word t is the operand of MFMA t as stored.
template <>
struct QWords<TL_HIP_GGML_F16> {
    static constexpr int BYTES = 64;
};

// X f32 [m, k] -> f16 [m, k] with every 32-element block stored in the k-slot order of the
// MFMA operands above: unit (row, block, word t) = 8 halves, one 16-byte store.
template <int QT>
__global__ __launch_bounds__(256) void k_x_to_f16q(const float* __restrict__ x, _Float16* __restrict__ x16,
                                                   int64_t units) {
    asm volatile("" : : "s"(x), "s"(x16), "s"(units));  // arguments in one round of scalar loads
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;  // = row * nb * 4 + block * 4 + t
    if (u >= units) return;
    const int t = (int)(u & 3);
    const float4* p = reinterpret_cast<const float4*>(x + (u >> 2) * 32);
    const float4 e = p[QT == TL_HIP_GGML_Q4_0 ? t : 2 * t], f = p[QT == TL_HIP_GGML_Q4_0 ? t + 4 : 2 * t + 1];
    half8 h;
    if constexpr (QT == TL_HIP_GGML_Q4_0) {  // slots: e0 e1 e2 e3 f0 f1 f2 f3
        h[0] = (_Float16)e.x; h[1] = (_Float16)e.y; h[2] = (_Float16)e.z; h[3] = (_Float16)e.w;
        h[4] = (_Float16)f.x; h[5] = (_Float16)f.y; h[6] = (_Float16)f.z; h[7] = (_Float16)f.w;
    } else {  // slots: e0 e2 e1 e3 f0 f2 f1 f3
        h[0] = (_Float16)e.x; h[1] = (_Float16)e.z; h[2] = (_Float16)e.y; h[3] = (_Float16)e.w;
        h[4] = (_Float16)f.x; h[5] = (_Float16)f.z; h[6] = (_Float16)f.y; h[7] = (_Float16)f.w;
    }
    reinterpret_cast<half8*>(x16)[u] = h;
}

// Weights of any resident type -> f16 [n, k] in the Q4_0 operand order (unit (row, block,
// word t) = the 8 halves of elements 4t..4t+3 and 16+4t..16+4t+3), for the MFMA GEMM of the
// types without an in-register operand builder (Q4_K, Q6_K).  One thread per 32-weight unit;
// each value is the exact f32 dequantization rounded once to f16.
template <int QT>
__global__ __launch_bounds__(256) void k_dequant_f16q(QView qv, _Float16* __restrict__ w16, int64_t units) {
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    float v[32];
    dequant_block<QT>(qv, u, v);
    half8* o = reinterpret_cast<half8*>(w16) + u * 4;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        half8 h;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[e] = (_Float16)v[4 * t + e];
            h[4 + e] = (_Float16)v[16 + 4 * t + e];
        }
        o[t] = h;
    }
}

// Operand DMA: buffer loads straight into LDS through a raw (stride 0) buffer resource over
// [p, p + bytes).  A lane's SIZE bytes at voff + soff land at lds + lane * SIZE (one 64-lane
// instruction writes 64 consecutive elements).  The per-lane offset is fixed for the whole K
// loop and the iteration's advance is a scalar, so the loop spends no vector instruction on
// addresses (with flat global_load_lds each load cost two 64-bit vector adds).
__device__ __forceinline__ void buf_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void buf_dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, voff, soff, 0, 0);
}

// X-tile chunk swizzle of row r (mod 16): a bijection of the 16 chunks for every row
__device__ __forceinline__ int xsw(int r) { return ((2 * r) & 15) ^ ((r >> 3) & 1); }

// One-launch split-K form of k_qgemm_mfma: an arrival counter per tile (split plans have at
// most 512 tiles), zero at load and returned to zero by the tile's last-arriving split.
constexpr int GM_ARRIVE_MAX = 512;
constexpr int GM_FUSE_NSP = 16;
__device__ uint32_t g_gemm_arrive[GM_ARRIVE_MAX];

// FUSE (split K, 32-wide tiles, n % 4 == 0): every split stores its partial tile into its
// slice of y as agent-scope atomics (written through to the agent's point of coherence) and
// the split that finishes the tile last forms v = res + slice 0 + ... + slice nsp-1 (res
// for the residual epilogue, else 0) -- k_splitk_sum's additions in its order -- reading the
// slices with the agent-coherent cache policy, all of a 4-column unit's slices at once.
template <int QT, int BM, int BN, bool FUSE = false>
__global__ __launch_bounds__(512) void k_qgemm_mfma(const uint8_t* __restrict__ qs, const __half* __restrict__ dsc,
                                                    const _Float16* __restrict__ x16, float* y, int64_t m,
                                                    int64_t n, int64_t k, int64_t nb, GemmEpi ep,
                                                    float* __restrict__ fin = nullptr) {
    // every argument, fetched from the kernel-argument buffer in one round of scalar loads
    // (left to the compiler, three dependent rounds precede the first tile load)
    asm volatile("" : : "s"(qs), "s"(dsc), "s"(x16), "s"(y), "s"(m), "s"(n), "s"(k), "s"(nb), "s"(ep.mode),
                 "s"(ep.res), "s"(ep.out16), "s"(ep.order));
    constexpr int TM = BM / 32, TN = BN / 32;  // 16 x 16 tiles per wavefront
    constexpr int QB = QWords<QT>::BYTES;
    constexpr int QC = QB / 16;                // 16-byte chunks per quant block
    constexpr int CPR = Q_KR * QC;             // W chunks per row and iteration
    constexpr bool SCALED = QT != TL_HIP_GGML_F16;   // quant blocks carry an f16 scale
    constexpr bool K4 = QT == TL_HIP_GGML_Q4_K;      // scales: one (d sc, -dmin m) word per unit
    constexpr int XI = BM * 16 / 512;          // X chunks per thread per iteration
    constexpr int WCH = BN * CPR;              // W chunks per iteration
    constexpr int WPT = WCH >= 512 ? WCH / 512 : 1;  // W DMA instructions per issuing wavefront
    constexpr int WW = WCH >= 512 ? 8 : WCH / 64;    // wavefronts that issue W DMA
    constexpr int DW = SCALED ? BN * Q_KR / 64 : 0;  // wavefronts that issue one scale DMA instruction
    static_assert(XI >= 1 && WW >= 1 && WW * WPT * 64 == WCH && DW <= 8, "tile");
    // Every operand reaches LDS through global_load_lds (a wavefront's instruction writes 64
    //  consecutive LDS elements, one per lane), so no load in the main loop writes a VGPR.
    //  * X: row r's 16-byte chunk c (= block * 4 + word) sits at c ^ xsw(r & 15);
    //  * W: chunk-major within each group of 16 rows (chunk c of row r at
    //    16 CPR (r / 16) + 16 c + r % 16); f16 weights (16 chunks a row, the shape of the X
    //    tile) row-major with the X swizzle, which keeps a DMA instruction on 4 rows; and BN x 4
    //    scale words.
    //  Both layouts measured free of LDS bank conflicts for the fragment reads below on
    //  gfx950 (rocprofv3 SQ_LDS_BANK_CONFLICT), where a plain c ^ r row swizzle cost ~3.9
    //  extra cycles per 16-byte read.
    // Two stages, each its own LDS object: the compiler's wait insertion can then see that a
    // stage being filled by DMA is not the one being read, and the next iteration's loads
    // overlap this iteration's MFMAs (with one array indexed by stage it waits for them).
    struct Stage {
        _Float16 X[BM * 128];
        uint8_t Wq[BN * CPR * 16];
        uint32_t Wd[SCALED ? BN * Q_KR : 1];  // aligned word holding the scale
    };
    __shared__ __attribute__((aligned(16))) Stage S0, S1;
    // the wavefront index in a scalar register: the compiler cannot see that tid >> 6 is
    // uniform, and every quantity derived from it (k half, sub-tile, DMA slots, LDS
    // addresses) would otherwise sit in vector registers behind divergent branches
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = wave & 3, kh = wave >> 2;  // output sub-tile, k half
    const int wm = sub >> 1, wn = sub & 1, col = lane & 15, g = lane >> 4;
    const int64_t nt = (n + BN - 1) / BN;
    const int64_t m0 = (blockIdx.x / nt) * BM, n0 = (blockIdx.x % nt) * BN;

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Per-lane source offsets (bytes) are fixed for the whole K loop; an iteration adds one
    // uniform advance.  K is a multiple of 128 (checked at launch): no block past nb is read.
    uint32_t xoff[XI], woff[WPT] = {}, doff = 0;
#pragma unroll
    for (int u = 0; u < XI; u++) {
        const int slot = (wave * XI + u) * 64 + lane, r = slot >> 4, c = (slot & 15) ^ xsw(r & 15);
        const int64_t row = m0 + r < m ? m0 + r : m - 1;  // rows past m feed outputs that are not stored
        xoff[u] = (uint32_t)((row * k + (c >> 2) * 32 + (c & 3) * 8) * 2);
    }
    if (wave < WW) {
#pragma unroll
        for (int u = 0; u < WPT; u++) {
            const int slot = (wave * WPT + u) * 64 + lane, within = slot % (16 * CPR);
            const int r = CPR == 16 ? slot >> 4 : slot / (16 * CPR) * 16 + within % 16;
            const int c = CPR == 16 ? (slot & 15) ^ xsw(r & 15) : within / 16;
            const int64_t row = n0 + r < n ? n0 + r : n - 1;
            woff[u] = (uint32_t)((row * nb + c / QC) * QB + (c % QC) * 16);
        }
    }
    if (DW > 0 && wave >= 8 - DW) {  // the 4-byte word that holds scale (row, block)
        const int slot = (wave - (8 - DW)) * 64 + lane;
        const int64_t row = n0 + (slot >> 2) < n ? n0 + (slot >> 2) : n - 1;
        // Q4_0 / Q8_0: the word holding the f16 d of (row, block); Q4_K: its (d sc, -dmin m) word
        doff = (uint32_t)(K4 ? (row * nb + (slot & 3)) * 4 : ((row * nb + (slot & 3)) >> 1) * 4);
    }
    // buffer extents (the launch keeps every one below 2^31 bytes); a Q4_0 / Q8_0 scale array
    // carries 4 bytes of padding, so its last aligned word is whole
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x16, (uint32_t)(m * k * 2));
    const __amdgpu_buffer_rsrc_t rq = buf_rsrc(qs, (uint32_t)(n * nb * QB));
    const __amdgpu_buffer_rsrc_t rd = buf_rsrc(dsc, (uint32_t)(SCALED ? n * nb * (K4 ? 4 : 2) + (K4 ? 0 : 4) : 0));
    auto issue = [&](int64_t kb, Stage& st) {
#pragma unroll
        for (int u = 0; u < XI; u++) buf_dma16(rx, xoff[u], (uint32_t)(kb * 64), &st.X[(wave * XI + u) * 64 * 8]);
        if (wave < WW) {
#pragma unroll
            for (int u = 0; u < WPT; u++) buf_dma16(rq, woff[u], (uint32_t)(kb * QB), &st.Wq[(wave * WPT + u) * 64 * 16]);
        }
        if (DW > 0 && wave >= 8 - DW)  // kb even: whole words
            buf_dma4(rd, doff, (uint32_t)(kb * (K4 ? 4 : 2)), &st.Wd[(wave - (8 - DW)) * 64]);
    };
    uint32_t dpar[TN];  // which half of its word holds this lane's scale (kb is even)
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int r = wn * (BN / 2) + 16 * j + col;
        const int64_t row = n0 + r < n ? n0 + r : n - 1;
        dpar[j] = (uint32_t)((row * nb + g) & 1) * 16;
    }
    // This wavefront's half of the iteration: k-steps t = 2 kh, 2 kh + 1.  Every LDS read
    // (W quants, scale words, A fragments) is issued before the first use.
    auto compute = [&](const Stage& st) {
        // quant data of the wavefront's rows: the 8 bytes of its k half (4-bit types: words
        // 2 kh, 2 kh + 1), the 16 bytes of its k half (Q8_0: words 4 kh .. 4 kh + 3), or the
        // two operand words of its k-steps (f16 weights) -- picked by the wavefront's k half
        // at the read, so the operand build indexes its words with compile-time values only
        // (a word index computed from kh became divergent branches and selects: the compiler
        // cannot see that kh is uniform; Q4_0 11008 x 4096 at M = 512 78.5 -> 74.8 us)
        constexpr bool Q8 = QT == TL_HIP_GGML_Q8_0;
        constexpr int NW = Q8 ? 1 : SCALED ? QC : 2;
        uint4 wr[TN][NW];
        uint32_t dw[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int r = wn * (BN / 2) + 16 * j + col;
#pragma unroll
            for (int h = 0; h < NW; h++) {
                const int c = Q8 ? g * QC + kh : SCALED ? g * QC + h : g * QC + 2 * kh + h;
                const int pos = CPR == 16 ? r * 16 + (c ^ xsw(r & 15)) : (r >> 4) * 16 * CPR + c * 16 + (r & 15);
                if constexpr (SCALED && !Q8) {
                    const uint2 h2 = *reinterpret_cast<const uint2*>(&st.Wq[pos * 16 + 8 * kh]);
                    wr[j][h] = uint4{h2.x, h2.y, 0u, 0u};
                } else {
                    wr[j][h] = *reinterpret_cast<const uint4*>(&st.Wq[pos * 16]);
                }
            }
            if constexpr (SCALED) dw[j] = st.Wd[r * Q_KR + g];
        }
        const _Float16* xs = st.X;
        half8 a[2][TM];
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int i = 0; i < TM; i++)
                a[tt][i] = *reinterpret_cast<const half8*>(xs + (wm * (BM / 2) + 16 * i + col) * 128 + ((g * 4 + 2 * kh + tt) ^ xsw(col)) * 8);
        __builtin_amdgcn_sched_barrier(0);
        half2v d2[TN], m8d2[TN];
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if constexpr (K4) {
                // both halves broadcast by the packed FMA's operand selects (no instruction)
                const half2v u = __builtin_bit_cast(half2v, dw[j]);
                d2[j] = __builtin_shufflevector(u, u, 0, 0);
                m8d2[j] = __builtin_shufflevector(u, u, 1, 1);
            } else if constexpr (SCALED) {
                const uint32_t b = (dw[j] >> dpar[j]) & 0xFFFFu;
                d2[j] = __builtin_bit_cast(half2v, b | (b << 16));
                m8d2[j] = d2[j] * half2v{(_Float16)-8.0f, (_Float16)-8.0f};
            }
        }
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {  // k-step 2 kh + tt
#pragma unroll
            for (int j = 0; j < TN; j++) {
                half8 bop;
                if constexpr (QT == TL_HIP_GGML_Q4_0 || K4) bop = QWords<QT>::operand(wr[j][0], tt, d2[j], m8d2[j]);
                else if constexpr (QT == TL_HIP_GGML_Q8_0) bop = QWords<QT>::operand(wr[j][0], tt, d2[j]);
                else bop = __builtin_bit_cast(half8, wr[j][tt]);
#pragma unroll
                for (int i = 0; i < TM; i++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tt][i], bop, acc[i][j], 0, 0, 0);
            }
        }
    };

    // S0 holds the even iterations, S1 the odd ones; the loads of iteration it + 1 are in
    // flight while it computes.  The wait + barrier at the top of an iteration make every
    // wavefront's chunks visible and free the stage the previous iteration read.
    // Split K (gridDim.y > 1): workgroup row blockIdx.y takes iterations [it0, it1) and stores
    // its partial tile in slice blockIdx.y of y (m x n floats each); the launch makes every
    // range non-empty.
    const int64_t iters = nb / Q_KR;  // >= 1: K is a multiple of 128
    const int64_t per = (iters + gridDim.y - 1) / gridDim.y;
    const int64_t it0 = (int64_t)blockIdx.y * per, it1 = it0 + per < iters ? it0 + per : iters;
    auto step = [&](int64_t it, const Stage& cur, Stage& next) {
        __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): this iteration's DMA has landed
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        if (it + 1 < it1) issue((it + 1) * Q_KR, next);
        __builtin_amdgcn_sched_barrier(0);
        compute(cur);
    };
    issue(it0 * Q_KR, S0);
    for (int64_t it = it0; it < it1; it += 2) {
        step(it, S0, S1);
        if (it + 1 < it1) step(it + 1, S1, S0);
    }
    float* const yb = y + (int64_t)blockIdx.y * m * n;
    // The two k halves add their sums through the (now free) X tiles (sub-tiles 0, 1 in S0's,
    // 2, 3 in S1's) and share the epilogue: a wavefront finishes the 16 x 16 tiles it owns
    // (tile index i TN + j of parity kh; all of them for kh = 0 when there is one tile) and
    // hands its partial sums of the others to the wavefront that owns them.
    static_assert(2 * TM * TN * 256 * 4 <= BM * 128 * 2, "reduction space");
    constexpr bool SHARE = TM * TN >= 2;
    auto owns = [&](int i, int j) { return SHARE ? ((i * TN + j) & 1) == kh : kh == 0; };
    __syncthreads();
    float* red = reinterpret_cast<float*>(sub < 2 ? S0.X : S1.X) + (sub & 1) * TM * TN * 256;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            if (!owns(i, j)) *reinterpret_cast<floatx4*>(red + (i * TN + j) * 256 + lane * 4) = acc[i][j];
    __syncthreads();
    {
        const int64_t rpos = !FUSE && ep.mode == GEMM_ROPE_KV ? (int64_t)*ep.rk.pos : 0;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if (!owns(i, j)) continue;
                const floatx4 o = *reinterpret_cast<const floatx4*>(red + (i * TN + j) * 256 + lane * 4);
                const int64_t c = n0 + wn * (BN / 2) + 16 * j + col;
                if (ep.mode == GEMM_GLU16) {
                    // columns (2i, 2i + 1) = (gate_i, up_i) sit in lanes col, col ^ 1, each with
                    // the same four rows: after one exchange per row the even lane finishes
                    // rows 0, 1 and the odd lane rows 2, 3, so no lane idles through the SwiGLU
                    float v4[4], u4[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        v4[e] = acc[i][j][e] + o[e];
                        u4[e] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v4[e]), 0xB1,
                                                                                   0xF, 0xF, true));
                    }
                    const bool odd = (col & 1) != 0;
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const int e = odd ? 2 + h : h;
                        const float mine = odd ? v4[2 + h] : v4[h], other = odd ? u4[2 + h] : u4[h];
                        const float gate = odd ? other : mine, up = odd ? mine : other;
                        const int64_t r = m0 + wm * (BM / 2) + 16 * i + 4 * g + e;
                        if (r < m && c < n) {
                            const float a = (gate * (1.0f / (1.0f + expf(-gate)))) * up;  // silu(gate) * up
                            ep.out16[f16q_index(r, c >> 1, n >> 1, ep.order)] = (_Float16)a;
                        }
                    }
                    continue;
                }
                if (!FUSE && ep.mode == GEMM_ROPE_KV) {
                    // RoPE pairs (2i, 2i + 1) sit in lanes col, col ^ 1 as in SwiGLU; the column's
                    // place in [q | k | v] once for the lane's four rows, the table entries once
                    // when every row reads the same table row
                    float v4[4], u4[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        v4[e] = acc[i][j][e] + o[e];
                        u4[e] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v4[e]), 0xB1,
                                                                                   0xF, 0xF, true));
                    }
                    if (c < n) {
                        const RopeCol cl = rope_col(ep.rk, c);
                        const bool odd = (col & 1) != 0, rot = cl.kind != 2;
                        const int64_t rb = m0 + wm * (BM / 2) + 16 * i + 4 * g;
                        float cs = 0.f, sn = 0.f;
                        if (rot && !ep.rk.per_token) {
                            const int64_t ti = rope_tab(ep.rk, cl, 0, rpos);
                            cs = ep.rk.ct[ti];
                            sn = ep.rk.st[ti];
                        }
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const int64_t r = rb + e;
                            if (r >= m) break;
                            if (rot && ep.rk.per_token) {
                                const int64_t ti = rope_tab(ep.rk, cl, r, rpos);
                                cs = ep.rk.ct[ti];
                                sn = ep.rk.st[ti];
                            }
                            rope_kv_put(ep.rk, cl, r, rpos, odd ? u4[e] : v4[e], odd ? v4[e] : u4[e], v4[e], cs, sn);
                        }
                    }
                    continue;
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int64_t r = m0 + wm * (BM / 2) + 16 * i + 4 * g + e;
                    const float v = acc[i][j][e] + o[e];
                    if (r < m && c < n) {
                        if constexpr (FUSE)
                            __hip_atomic_store(reinterpret_cast<uint32_t*>(yb + r * n + c), __float_as_uint(v),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        else yb[r * n + c] = ep.mode == GEMM_RES ? ep.res[r * n + c] + v : v;
                    }
                }
            }
    }
    if constexpr (FUSE) {
        // arrival: every wavefront's slice stores have completed before the count is bumped
        __shared__ int s_last;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const int nsp = (int)gridDim.y;
        if (threadIdx.x == 0) {
            uint32_t* cnt = g_gemm_arrive + blockIdx.x;
            const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == (uint32_t)(nsp - 1);
            if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;  // uniform per workgroup
        const int64_t mn = m * n;
        const __amdgpu_buffer_rsrc_t rp = buf_rsrc(y, (uint32_t)(nsp * mn * 4));
        const int64_t rpos = ep.mode == GEMM_ROPE_KV ? (int64_t)*ep.rk.pos : 0;
        constexpr int UPR = BN / 4;  // 4-column units per tile row
        for (int u = threadIdx.x; u < BM * UPR; u += 512) {
            const int64_t r = m0 + u / UPR, c = n0 + 4 * (u % UPR);
            if (r < m && c < n) {
                // every slice's 16 bytes requested at once (slices past nsp lie beyond the
                // resource's range and read 0; the selects keep them out of the sum)
                const uint32_t vo = (uint32_t)((r * n + c) * 4);
                u32x4 t[GM_FUSE_NSP];
#pragma unroll
                for (int p = 0; p < GM_FUSE_NSP; p++)
                    t[p] = __builtin_amdgcn_raw_buffer_load_b128(rp, vo, (int)(p * mn * 4), CPOL_SC1);
                float4 v = ep.mode == GEMM_RES ? *reinterpret_cast<const float4*>(ep.res + r * n + c)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int p = 0; p < GM_FUSE_NSP; p++) {
                    const bool on = p < nsp;
                    v.x = on ? v.x + __uint_as_float(t[p].x) : v.x;
                    v.y = on ? v.y + __uint_as_float(t[p].y) : v.y;
                    v.z = on ? v.z + __uint_as_float(t[p].z) : v.z;
                    v.w = on ? v.w + __uint_as_float(t[p].w) : v.w;
                }
                if (ep.mode == GEMM_ROPE_KV) {  // a unit holds two whole pairs
                    rope_kv_store4(ep.rk, r, c, rpos, v);
                } else {
                    *reinterpret_cast<float4*>(fin + r * n + c) = v;
                }
            }
        }
    }
}


// ------------------------------------------------------ short-input quantized GEMM ----
// Y[m, n] = sum_k X[m, k] W[n, k] for short inputs (m <= 16 rows: chat prompts, the M = 16
// case of a prefill GEMM), reading X in f32 (no X conversion launch).  A workgroup of
// SG_WAVES wavefronts owns a tile of SG_WAVES x 16 NR weight rows (16 NR per wavefront) and
// one range of the 128-k groups of K (grid.y = the K splits).  Per group the wavefronts stage
// X once, shared: each loads its rows' part (coalesced, two rows' 512 bytes per
// instruction), rounds it to f16 and writes it to the LDS tile in the A-operand order of the
// weight type; after a barrier every wavefront reads its four 16-byte A fragments and runs
// 4 NR MFMAs (v_mfma_f32_16x16x32_f16) over its own rows.  Weights are the B operand as in
// k_qgemm_mfma: lane (col, g) holds row col's block g of the group, word t feeding MFMA t
// (QWords operand builders, one f16 rounding of the dequantized value), loaded non-temporal.
// Loads run one group ahead.  With more than one split each workgroup stores its partial
// tile in a workspace slice and k_splitk_sum_short adds the slices in K order, so the result
// does not depend on scheduling.
// Measured on MI355X (rocprofv3, M = 16): a CU's L1 takes ~64 misses in flight, each ~350-460
// cycles to L2 and back, so the number of L2 requests per CU sets the pace.  X is most of
// them when every wavefront fetches its own copy (64 bytes per k at m = 16, against 0.56
// (Q4_0) or 1.06 (Q8_0) per k and weight row), hence one shared copy per workgroup and a
// wide tile; splitting K spreads the tiles over every CU.
__global__ void k_splitk_sum(const float* __restrict__ part, float* y, const float* res, int64_t mn, int nsp);

constexpr int SG_WAVES = 4;   // wavefronts per workgroup (they split the tile's rows)
constexpr int SG_PITCH = 68;  // LDS words per X row of one 128-k group (64 + 4)
// One-launch split form: an arrival counter per tile, zero at load and returned to zero by
// the tile's last-arriving split, which adds the slices (at most SG_FUSE_NSP of them; the
// launch splits only below 512 tiles).
constexpr int SG_ARRIVE_MAX = 512;
constexpr int SG_FUSE_NSP = 8;
__device__ uint32_t g_short_arrive[SG_ARRIVE_MAX];

// FUSE: with K split, the split that finishes a tile last adds its slices (y = the final
// output, part = the slices; n % 4 == 0) instead of k_splitk_sum_short in a second launch.
// Slices are then written as agent-scope atomics (stores that write through to the agent's
// point of coherence) and read with the same cache policy (sc1: no stale line of another
// XCD's L2), and every wavefront waits for its slice stores to complete before the arrival
// count is bumped.
template <int QT, int MT, int NR, bool FUSE>
__global__ __launch_bounds__(64 * SG_WAVES) void k_qgemm_short(const uint8_t* __restrict__ qs,
                                                               const void* __restrict__ dsc,
                                                               const float* __restrict__ x, float* __restrict__ y,
                                                               int m, int64_t n, int64_t k, int64_t nb, int tiles,
                                                               int nsp, float* __restrict__ part) {
    asm volatile("" : : "s"(qs), "s"(dsc), "s"(x), "s"(y), "s"(m), "s"(n), "s"(k), "s"(nb), "s"(tiles), "s"(nsp));
    // (tile, split) from the 1-D grid so that every split of a tile runs on the XCD of its
    // tile (workgroups go to the 8 XCDs round-robin by linear id): a weight row's scale lines
    // and X then stay in one XCD's L2 (with splits spread over XCDs, 11008 x 4096 Q4_0 read
    // 1.30x its algorithmic bytes from HBM)
    const int wg = blockIdx.x, xcd = wg & 7, rest = wg >> 3;
    const int split = rest % nsp, tile = (rest / nsp) * 8 + xcd;
    if (tile >= tiles) return;  // padding of the grid to whole groups of 8 tiles (uniform)
    constexpr bool Q8 = QT == TL_HIP_GGML_Q8_0, K4 = QT == TL_HIP_GGML_Q4_K;
    constexpr int QB = Q8 ? 32 : 16, WV = QB / 16;
    constexpr int XI = MT / (2 * SG_WAVES);  // X load instructions per wavefront and group (two rows each)
    static_assert(XI >= 1, "tile");
    __shared__ __attribute__((aligned(16))) uint32_t xs[4][16 * SG_PITCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, g = lane >> 4;
    const int64_t n0 = ((int64_t)tile * SG_WAVES + wave) * 16 * NR;
    const int64_t ng = nb >> 2;  // 128-k groups (K is a multiple of 128)
    // K splits in whole two-group stages, so that no 128-byte line of a weight row is read by
    // two workgroups (split boundaries at odd groups measured 1.43x the algorithmic HBM bytes)
    const int64_t nst = (ng + 1) >> 1;
    const int64_t gb = 2 * (nst * split / nsp);
    const int64_t ge = min(2 * (nst * (split + 1) / nsp), ng);
    const int G = (int)(ge - gb);  // >= 1: the launch keeps splits <= stages

    // unit index of (row, block g of group gb) for this lane's rows; rows past n read row
    // n - 1, whose outputs are not stored
    int64_t wu[NR];
#pragma unroll
    for (int j = 0; j < NR; j++) {
        const int64_t r = n0 + 16 * j + col;
        wu[j] = (r < n ? r : n - 1) * nb + gb * 4 + g;
    }
    // X: this lane loads float4 unit xj of rows xr + 2 i (i < XI) of every group
    const int xj = lane & 31, xr = 2 * XI * wave + (lane >> 5);
    const float* xp = x + (int64_t)xr * k + gb * 128 + xj * 4;
    // LDS word pair of unit xj within its row: Q8_0 keeps the k order (elements 8t .. 8t+7 of a
    // block feed MFMA t); Q4_0 / Q4_K interleave units 8g + t and 8g + 4 + t (elements 4t..4t+3
    // and 16+4t..16+4t+3, MFMA t's nibble slots)
    const int p = Q8 ? xj : (xj & ~7) | ((xj & 3) << 1) | ((xj >> 2) & 1);

    // two slots of one stage = two 128-k groups each (both halves of every 128-byte line of a
    // weight row; loads of a stage go out back to back)
    // Scales: per four groups, lane (col, g) loads group g's four scales of its row (one 8-byte
    // load, 16 bytes of unit pairs for Q4_K) and parks them in the wavefront's LDS table;
    // a group's MFMAs read their lane's scale back (2-byte loads of 16 rows per instruction
    // were measured 1-4.5 us slower per call)
    constexpr int SCW = K4 ? 4 : 2;  // scale words per (row, group)
    __shared__ __attribute__((aligned(16))) uint32_t scs[SG_WAVES][NR][16][4][SCW];
    // A stage is two 128-k groups (both halves of every 128-byte line of a weight row).  Its
    // X, weights and scales are loaded one stage ahead of their use, in the order of use (a
    // wait for one load is a wait for every load issued before it).  Deeper rings (weights
    // four stages ahead, X with them) measured slower.
    constexpr int SG_WR = 2;
    uint4 wr[SG_WR][2][NR][WV];
    uint32_t sc[SG_WR][NR][SCW];
    float4 xv[SG_WR][2][XI];
    floatx4 acc[NR];
#pragma unroll
    for (int j = 0; j < NR; j++) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Every load below is unconditional, with clamped indices (no branch between a load and
    // its use, so the compiler's waits count loads instead of draining all of them): X rows
    // past m read row m - 1 and feed only output rows that are not stored; groups past the
    // range read its last group and feed no MFMA.
    auto load_x = [&](int st, int sl) {
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int q = min(2 * st + c, G - 1);
#pragma unroll
            for (int i = 0; i < XI; i++) {
                const int r = min(xr + 2 * i, m - 1);
                xv[sl][c][i] = *reinterpret_cast<const float4*>(xp + (int64_t)(r - xr) * k + 128 * (int64_t)q);
            }
        }
    };
    auto load_w = [&](int st, int sl) {
#pragma unroll
        for (int j = 0; j < NR; j++)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int64_t u = wu[j] + 4 * (int64_t)min(2 * st + c, G - 1);
#pragma unroll
                for (int v = 0; v < WV; v++) wr[sl][c][j][v] = ld_stream(reinterpret_cast<const uint4*>(qs + u * QB) + v);
            }
        if ((st & 1) == 0) {  // scales of groups 2 st .. 2 st + 3: lane g takes group 2 st + g
#pragma unroll
            for (int j = 0; j < NR; j++) {
                const int64_t u0 = wu[j] - g + 4 * (int64_t)min(2 * st + g, G - 1);  // unit of (row, block 0 of that group)
                if constexpr (K4) {
                    const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint32_t*>(dsc) + u0);
                    sc[sl][j][0] = v.x, sc[sl][j][1] = v.y, sc[sl][j][2] = v.z, sc[sl][j][3] = v.w;
                } else {
                    const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(dsc) + u0);
                    sc[sl][j][0] = v.x, sc[sl][j][1] = v.y;
                }
            }
        }
    };
    // this wavefront's X rows of stage st (X slot xsl) -> f16 -> LDS tiles 2 xsl, 2 xsl + 1,
    // and on even stages the scales (weight slot wsl) -> the wavefront's scale table
    auto stage = [&](int st, int wsl, int xsl) {
        if ((st & 1) == 0) {
#pragma unroll
            for (int j = 0; j < NR; j++)
#pragma unroll
                for (int w = 0; w < SCW; w++) scs[wave][j][col][g][w] = sc[wsl][j][w];
        }
#pragma unroll
        for (int c = 0; c < 2; c++) {
#pragma unroll
            for (int i = 0; i < XI; i++) {
                const float4 v = xv[xsl][c][i];
                const half2v lo = Q8 ? half2v{(_Float16)v.x, (_Float16)v.z} : half2v{(_Float16)v.x, (_Float16)v.y};
                const half2v hi = Q8 ? half2v{(_Float16)v.y, (_Float16)v.w} : half2v{(_Float16)v.z, (_Float16)v.w};
                *reinterpret_cast<uint2*>(&xs[2 * (xsl & 1) + c][(xr + 2 * i) * SG_PITCH + 2 * p]) =
                    uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
            }
        }
    };
    auto compute = [&](int st, int wsl, int xsl, bool two) {
#pragma unroll
        for (int c = 0; c < 2; c++) {
            if (c == 1 && !two) break;
            const int gq = 2 * (st & 1) + c;  // the group's entry in the scale table
            half8 a[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                a[t] = *reinterpret_cast<const half8*>(&xs[2 * (xsl & 1) + c][col * SG_PITCH + 16 * g + 4 * t]);
                if (MT < 16 && col >= MT) a[t] = half8{};
            }
#pragma unroll
            for (int j = 0; j < NR; j++) {
                half2v d2, m8d2;
                if constexpr (K4) {
                    const half2v u = __builtin_bit_cast(half2v, scs[wave][j][col][gq][g]);
                    d2 = __builtin_shufflevector(u, u, 0, 0);
                    m8d2 = __builtin_shufflevector(u, u, 1, 1);
                } else {
                    const uint32_t b = reinterpret_cast<const uint16_t*>(&scs[wave][j][col][gq][0])[g];
                    d2 = __builtin_bit_cast(half2v, b | (b << 16));
                    m8d2 = d2 * half2v{(_Float16)-8.0f, (_Float16)-8.0f};
                }
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    half8 bop;
                    if constexpr (Q8) bop = QWords<QT>::operand(wr[wsl][c][j][t >> 1], t & 1, d2);
                    else bop = QWords<QT>::operand(wr[wsl][c][j][0], t, d2, m8d2);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], bop, acc[j], 0, 0, 0);
                }
            }
        }
    };

    // stage st: its loads in slot st % 2, one stage ahead; staged (X into the LDS tiles of
    // slot st % 2), then after the barrier (which also frees those tiles' previous stage) read
    // by every wavefront.  Loads are issued only for stages that exist: clamped loads of
    // absent stages (no branch between a load and its use, exact waits) measured slower --
    // a workgroup of one stage then loads it twice.
    const int S = (G + 1) / 2;
    auto two = [&](int st) { return 2 * st + 1 < G; };
    load_x(0, 0);
    load_w(0, 0);
    for (int s0 = 0; s0 < S; s0 += 2) {
        if (s0 + 1 < S) {
            load_x(s0 + 1, 1);
            load_w(s0 + 1, 1);
        }
        stage(s0, 0, 0);
        __syncthreads();
        compute(s0, 0, 0, two(s0));
        if (s0 + 1 < S) {
            if (s0 + 2 < S) {
                load_x(s0 + 2, 0);
                load_w(s0 + 2, 0);
            }
            stage(s0 + 1, 1, 1);
            __syncthreads();
            compute(s0 + 1, 1, 1, two(s0 + 1));
        }
    }

    // lane (col, g) holds rows 4g .. 4g + 3 of column col of each sub-tile; a split stores
    // into its slice of the workspace (m x n floats per split: y, or part when FUSE)
    if constexpr (!FUSE) {
        float* const yb = y + (int64_t)split * m * n;
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int64_t cn = n0 + 16 * j + col;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = 4 * g + e;
                if (r < m && cn < n) yb[(int64_t)r * n + cn] = acc[j][e];
            }
        }
    } else {
        float* const pb = part + (int64_t)split * m * n;
#pragma unroll
        for (int j = 0; j < NR; j++) {
            const int64_t cn = n0 + 16 * j + col;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = 4 * g + e;
                if (r < m && cn < n)
                    __hip_atomic_store(reinterpret_cast<uint32_t*>(pb + (int64_t)r * n + cn), __float_as_uint(acc[j][e]),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        __shared__ int s_last;
        if (tid == 0) {
            const uint32_t old = __hip_atomic_fetch_add(g_short_arrive + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == (uint32_t)(nsp - 1);
            if (last) __hip_atomic_store(g_short_arrive + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;  // uniform per workgroup
        // y = the slices added in slice order, as k_splitk_sum_short adds them: thread t takes
        // 4-column units t, t + 256, ... of the tile's m x 64 NR outputs and requests every
        // slice's 16 bytes of a unit at once
        const int64_t mn = (int64_t)m * n;
        const __amdgpu_buffer_rsrc_t rp = buf_rsrc(part, (uint32_t)(nsp * mn * 4));
        constexpr int UPR = 4 * NR * SG_WAVES;  // 4-column units per tile row
        const int64_t c0 = (int64_t)tile * SG_WAVES * 16 * NR;
#pragma unroll
        for (int u0 = 0; u0 < MT * UPR; u0 += 64 * SG_WAVES) {
            const int u = u0 + tid, r = u / UPR;
            const int64_t cn = c0 + 4 * (u % UPR);
            if (r < m && cn < n) {
                const uint32_t vo = (uint32_t)(((int64_t)r * n + cn) * 4);
                // every load issued before the first add (slices p >= nsp lie past the buffer's
                // range and read 0; the selects keep them out of the sum)
                u32x4 t[SG_FUSE_NSP];
#pragma unroll
                for (int p = 0; p < SG_FUSE_NSP; p++)
                    t[p] = __builtin_amdgcn_raw_buffer_load_b128(rp, vo, (int)(p * mn * 4), CPOL_SC1);
                float4 v = make_float4(__uint_as_float(t[0].x), __uint_as_float(t[0].y), __uint_as_float(t[0].z),
                                       __uint_as_float(t[0].w));
#pragma unroll
                for (int p = 1; p < SG_FUSE_NSP; p++) {
                    const bool on = p < nsp;
                    v.x = on ? v.x + __uint_as_float(t[p].x) : v.x;
                    v.y = on ? v.y + __uint_as_float(t[p].y) : v.y;
                    v.z = on ? v.z + __uint_as_float(t[p].z) : v.z;
                    v.w = on ? v.w + __uint_as_float(t[p].w) : v.w;
                }
                *reinterpret_cast<float4*>(y + (int64_t)r * n + cn) = v;
            }
        }
    }
}

// y = sum of the nsp partial slices (m n floats each, 16-byte aligned) in slice order, with
// every slice's load in flight at once (NSP a power of two >= nsp)
template <int NSP>
__global__ __launch_bounds__(64) void k_splitk_sum_short(const float* __restrict__ part, float* __restrict__ y,
                                                         int64_t mn, int nsp) {
    asm volatile("" : : "s"(part), "s"(y), "s"(mn), "s"(nsp));
    const int64_t i = ((int64_t)blockIdx.x * 64 + threadIdx.x) * 4;
    if (i >= mn) return;
    float4 t[NSP];
#pragma unroll
    for (int p = 0; p < NSP; p++)
        if (p < nsp) t[p] = *reinterpret_cast<const float4*>(part + p * mn + i);
    float4 v = t[0];
#pragma unroll
    for (int p = 1; p < NSP; p++)
        if (p < nsp) {
            v.x += t[p].x;
            v.y += t[p].y;
            v.z += t[p].z;
            v.w += t[p].w;
        }
    *reinterpret_cast<float4*>(y + i) = v;
}

// Whether the short-input GEMM takes this product: 1 <= m <= 16, K in steps of 128, and a
// weight type with an in-register operand builder (Q4_K once its unit scales exist).
bool gemm_short_ok(const QWeight* w, int64_t m) {
    return m >= 1 && m <= 16 && w->nb % Q_KR == 0 &&
           (w->ggml_type == TL_HIP_GGML_Q4_0 || w->ggml_type == TL_HIP_GGML_Q8_0 ||
            (w->ggml_type == TL_HIP_GGML_Q4_K && w->us));
}

namespace {
struct ShortPlan {
    int nr;
    int64_t tiles, nsp;
};
}  // namespace

// Tile = SG_WAVES x 16 NR rows: NR = 2 (128 rows) for the 4-bit types at N >= 8192 (fewer
// tiles re-reading X), else 1 (64 rows); K split until about two workgroups per CU run (at
// most one split per two-group stage, at most 16; the partial slices need m n % 4 == 0 and a
// 16-byte aligned y).  Measured at M = 16 (us per call, Q4_0 / Q8_0): 4096^2 NR 1 8.8 / 10.2
// against NR 2 9.7 / 10.6; 11008 x 4096 NR 2 16.2 / 23.5, NR 1 17.3 / 22.8.
static ShortPlan plan_short(const QWeight* w, int64_t m, const float* y) {
    const int64_t ng = w->nb / Q_KR;
    const int cus = state() ? state()->num_cus : 256;
    const int nr = w->ggml_type != TL_HIP_GGML_Q8_0 && w->n >= 8192 ? 2 : 1;
    const int64_t tiles = cdiv(w->n, 16 * SG_WAVES * nr);
    int64_t nsp = 1;
    const bool split_ok = (m * w->n) % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    if (split_ok && tiles < 2 * cus)
        nsp = std::min<int64_t>(std::min<int64_t>(cdiv(2 * cus, tiles), (ng + 1) / 2), 16);
    return ShortPlan{nr, tiles, nsp};
}

// part_ws: workspace of nsp * m * n floats when the plan splits K and noalloc is set (else
// allocated on s).
int launch_gemm_short(const QWeight* w, const float* x, float* y, int64_t m, hipStream_t s, float* part_ws,
                      bool noalloc) {
    if (!gemm_short_ok(w, m)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: the short-input GEMM takes 1 <= m <= 16, K in steps of 128 and "
                  "Q4_0 / Q8_0 / Q4_K weights");
        return TL_HIP_ERR_ARG;
    }
    const ShortPlan pl = plan_short(w, m, y);
    float* part = nullptr;
    if (pl.nsp > 1) {
        part = noalloc ? part_ws : static_cast<float*>(dev_alloc_on((size_t)pl.nsp * m * w->n * sizeof(float), s));
        if (!part) {
            if (noalloc) set_error(TL_HIP_ERR_ARG, "ArgumentError: no workspace for the split-K partials");
            return noalloc ? TL_HIP_ERR_ARG : TL_HIP_ERR_ALLOC;
        }
    }
    float* const out = pl.nsp > 1 ? part : y;
    const unsigned grid = (unsigned)(cdiv(pl.tiles, 8) * 8 * pl.nsp);
    // one launch when no other stream can run a call that shares the arrival counters
    const bool fuse = pl.nsp > 1 && pl.nsp <= SG_FUSE_NSP && pl.tiles <= SG_ARRIVE_MAX && w->n % 4 == 0 &&
                      (size_t)pl.nsp * m * w->n * 4 < (1ull << 31) && single_stream() && one_launch_merge();
    const int ti = (int)pl.tiles, ns = (int)pl.nsp;
    const void* dsc = w->ggml_type == TL_HIP_GGML_Q4_K ? static_cast<const void*>(w->us) : static_cast<const void*>(w->d);
    tls_plan[0] = m <= 8 ? 8 : 16;
    tls_plan[1] = 16 * SG_WAVES * pl.nr;
    tls_plan[2] = (int)pl.nsp;
    const int mi = (int)m;
    auto go = [&](auto qt) {
        constexpr int QT = decltype(qt)::value;
        auto run = [&](auto mt) {
            constexpr int MT = decltype(mt)::value;
            if (fuse) {
                if (pl.nr == 1)
                    k_qgemm_short<QT, MT, 1, true><<<grid, 64 * SG_WAVES, 0, s>>>(w->qs, dsc, x, y, mi, w->n, w->k, w->nb,
                                                                                  ti, ns, part);
                else
                    k_qgemm_short<QT, MT, 2, true><<<grid, 64 * SG_WAVES, 0, s>>>(w->qs, dsc, x, y, mi, w->n, w->k, w->nb,
                                                                                  ti, ns, part);
            } else if (pl.nr == 1) {
                k_qgemm_short<QT, MT, 1, false><<<grid, 64 * SG_WAVES, 0, s>>>(w->qs, dsc, x, out, mi, w->n, w->k, w->nb,
                                                                               ti, ns, nullptr);
            } else {
                k_qgemm_short<QT, MT, 2, false><<<grid, 64 * SG_WAVES, 0, s>>>(w->qs, dsc, x, out, mi, w->n, w->k, w->nb,
                                                                               ti, ns, nullptr);
            }
        };
        if (m <= 8) run(std::integral_constant<int, 8>{});
        else run(std::integral_constant<int, 16>{});
    };
    if (w->ggml_type == TL_HIP_GGML_Q4_0) go(std::integral_constant<int, TL_HIP_GGML_Q4_0>{});
    else if (w->ggml_type == TL_HIP_GGML_Q8_0) go(std::integral_constant<int, TL_HIP_GGML_Q8_0>{});
    else go(std::integral_constant<int, TL_HIP_GGML_Q4_K>{});
    if (pl.nsp > 1) {
        const int64_t mn = m * w->n;
        const unsigned sg = (unsigned)cdiv(cdiv(mn, 4), 64);
        if (fuse) {
        } else if (pl.nsp <= 4) k_splitk_sum_short<4><<<sg, 64, 0, s>>>(part, y, mn, (int)pl.nsp);
        else if (pl.nsp <= 8) k_splitk_sum_short<8><<<sg, 64, 0, s>>>(part, y, mn, (int)pl.nsp);
        else k_splitk_sum_short<16><<<sg, 64, 0, s>>>(part, y, mn, (int)pl.nsp);
        if (!noalloc) dev_free_on(part, s);  // freed on s: reused at once only by later work on s
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "short-input gemm launch");
}

// workspace bytes of a short-input GEMM call (split-K partial slices; 0 when unsplit)
size_t gemm_short_workspace(const QWeight* w, int64_t m, const float* y) {
    const ShortPlan pl = plan_short(w, m, y);
    return pl.nsp > 1 ? (size_t)pl.nsp * m * w->n * sizeof(float) : 0;
}

// one word per Q4_K unit: f16 d * scale (low half) and f16 -(dmin * min) (high half)
__global__ __launch_bounds__(256) void k_q4k_unit_scales(const uint8_t* __restrict__ hdr, uint32_t* __restrict__ us,
                                                         int64_t units) {
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    float d1, m1;
    q4k_scale_min(reinterpret_cast<const uint4*>(hdr)[u >> 3], (int)(u & 7), &d1, &m1);
    const _Float16 a = (_Float16)d1, b = (_Float16)(-m1);
    us[u] = (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

int q4k_build_unit_scales(QWeight* w, hipStream_t s) {
    static std::mutex mu;  // one build per tensor when threads share it
    std::lock_guard<std::mutex> lk(mu);
    if (w->ggml_type != TL_HIP_GGML_Q4_K || w->us) return TL_HIP_OK;
    const int64_t units = w->n * w->nb;
    w->us = static_cast<uint32_t*>(dev_alloc_on((size_t)units * 4, s));
    if (!w->us) return TL_HIP_ERR_ALLOC;
    k_q4k_unit_scales<<<(unsigned)cdiv(units, 256), 256, 0, s>>>(w->hdr, w->us, units);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "Q4_K unit scales launch");
}

int f16q_order(int ggml_type) { return ggml_type == TL_HIP_GGML_Q8_0 ? F16Q_Q8 : F16Q_Q4; }

int launch_x_to_f16q(const float* x, _Float16* x16, int64_t m, int64_t k, int order, hipStream_t s) {
    const int64_t units = m * (k / 32) * 4;
    if (order == F16Q_Q8) k_x_to_f16q<TL_HIP_GGML_Q8_0><<<(unsigned)cdiv(units, 256), 256, 0, s>>>(x, x16, units);
    else k_x_to_f16q<TL_HIP_GGML_Q4_0><<<(unsigned)cdiv(units, 256), 256, 0, s>>>(x, x16, units);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "x -> f16 launch");
}

// Split-K sum: y = [res +] the nsp partial slices, added in slice order (the result does not
// depend on scheduling).  y may alias res; y, res and part are 16-byte aligned (the launch
// splits K only then).
__global__ __launch_bounds__(256) void k_splitk_sum(const float* __restrict__ part, float* y, const float* res,
                                                    int64_t mn, int nsp) {
    asm volatile("" : : "s"(part), "s"(y), "s"(res), "s"(mn), "s"(nsp));  // arguments in one round
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    if (i + 4 <= mn) {
        float4 v = res ? *reinterpret_cast<const float4*>(res + i) : float4{0.f, 0.f, 0.f, 0.f};
        for (int p = 0; p < nsp; p++) {
            const float4 t = *reinterpret_cast<const float4*>(part + p * mn + i);
            v.x += t.x;
            v.y += t.y;
            v.z += t.z;
            v.w += t.w;
        }
        *reinterpret_cast<float4*>(y + i) = v;
    } else {
        for (int64_t j = i; j < mn; j++) {
            float v = res ? res[j] : 0.f;
            for (int p = 0; p < nsp; p++) v += part[p * mn + j];
            y[j] = v;
        }
    }
}

// k_splitk_sum's sums (slice order, from 0) of a [q | k | v] projection, then RoPE and the
// KV append (the GEMM's ROPE_KV epilogue) instead of the store: n % 4 == 0, so a 4-column
// unit holds two whole pairs of one token row.
__global__ __launch_bounds__(256) void k_splitk_sum_rope(const float* __restrict__ part, int64_t mn, int64_t n,
                                                         int nsp, RopeKvEpi rk) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    float4 v{0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < nsp; p++) {
        const float4 t = *reinterpret_cast<const float4*>(part + p * mn + i);
        v.x += t.x;
        v.y += t.y;
        v.z += t.z;
        v.w += t.w;
    }
    const int64_t r = i / n, c = i % n, pos = *rk.pos;
    rope_kv_store4(rk, r, c, pos, v);
}

namespace {
// Launch plan of one f16 GEMM: row tile bm, column tile bn (128 x 96 or 128 x 64 wide tiles,
// x 32 narrow ones), tile count and K splits.
struct F16qPlan {
    int bm, bn;
    int64_t tiles, nsp;
};
}  // namespace

// whether a split plan of these tiles may add its slices in-kernel (the one-launch form)
static bool f16q_fuse_ok(const QWeight* w, int64_t m, int bm, int bn, int64_t tiles, int64_t nsp,
                         const GemmEpi& ep) {
    return ep.mode != GEMM_GLU16 && nsp > 1 && nsp <= GM_FUSE_NSP && bn == 32 && bm <= 64 && tiles <= GM_ARRIVE_MAX && w->n % 4 == 0 &&
           (size_t)nsp * m * w->n * 4 < (1ull << 31) && single_stream() && one_launch_merge();
}

static F16qPlan plan_f16q(const QWeight* w, int64_t m, const GemmEpi& ep, const float* y) {
    // 128 x 64 tiles when that gives at least one workgroup per CU, else 128 x 32 (twice the
    // workgroups; measured at M = 512: 2048 x 2048 18.7 -> 15.5 us).  At 256 wide tiles the
    // narrow tile gains nothing (Q4_0 4096 x 4096: 35.7 us wide, 36.4 narrow) and loses at long
    // K (4096 x 11008: Q4_0 85.2 vs 91.3 us, Q8_0 99.1 vs 111.7 us); 11008 x 4096: 84.5 vs 101.7 us.
    // f16 weights (K-quants) move 3.5x the bytes per tile: 128 x 32 only when 128 x 64 would
    // leave half the CUs idle (2560 x 2048: 16.8 us wide vs 24.8 narrow; 2048 x 2048: 16.6 vs 13.5)
    constexpr int BM = 128;
    const bool f16w = (w->ggml_type == TL_HIP_GGML_Q4_K && !w->us) || w->ggml_type == TL_HIP_GGML_Q6_K;
    const int64_t wide_tiles = cdiv(m, BM) * cdiv(w->n, 64);
    const bool wide = f16w ? wide_tiles > 128 : wide_tiles >= 256;
    // 128 x 96 tiles (4-bit types with 16-byte blocks: 79 KB of LDS, still two workgroups per
    // CU) when the 128 x 64 tiles overflow the 512 two-per-CU slots and 96-wide ones do not:
    // one wave of workgroups instead of a full one and a partial second
    const bool nib16 = w->ggml_type == TL_HIP_GGML_Q4_0 || (w->ggml_type == TL_HIP_GGML_Q4_K && w->us);
    const int64_t t96 = cdiv(m, BM) * cdiv(w->n, 96);
    const int bn = !wide ? 32 : nib16 && wide_tiles > 512 && t96 <= 512 ? 96 : 64;
    // Short inputs: 32- or 64-row tiles when M fits them, and with at most one tile per CU
    // (512 tiles for M <= 32, where the K loop's latency dominates) the K range split over up
    // to 16 workgroup rows until about 512 workgroups run (the 512-token prefill's 256-tile
    // o-projection and down projection included: 3.66 -> 3.49 ms); partial tiles go to a workspace that
    // k_splitk_sum adds up (with the residual), or the tile's last split in-kernel.  The SwiGLU
    // epilogue is not linear and keeps one workgroup per tile (split in the one-launch form,
    // with SwiGLU after the last split's sum, it measured slower: 32-token prefill 1.19 ->
    // 1.22 ms).  (Measured at M = 16 / 128: 4096 x 4096
    // 27.1 -> 13.1 / 28.9 -> 21.7 us, 4096 x 11008 63.5 -> 22.0 / 70.6 -> 36.7 us per call
    // including the X conversion; splitting the 344 tiles of 11008 x 4096 in two at M = 128
    // was slower, 37.0 -> 44.7 us, and faster at M = 16, 23.6 -> 20.5 us.)
    int bm = wide ? BM : m <= 32 ? 32 : m <= 64 ? 64 : BM;
    // f16 weights on narrow tiles: 64-row tiles while 128-row ones would leave workgroup slots
    // empty (Q4_K_M 512-token prefill -- its Q6_K parts -- 3.23 -> 3.10 ms; the 4-bit types
    // measured slower that way, Q4_0 prefill 2.79 -> 2.84 ms)
    if (f16w && !wide && bm == BM && cdiv(m, BM) * cdiv(w->n, 32) < 512) bm = 64;
    const int64_t tiles = cdiv(m, bm) * cdiv(w->n, bn);
    const int64_t iters = w->nb / Q_KR;
    int64_t nsp = 1;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(ep.res)) & 15) == 0;
    if (!wide && ep.mode != GEMM_GLU16 && vec_ok && tiles <= (m <= 32 ? 512 : 256)) {
        nsp = std::min<int64_t>(std::min<int64_t>(cdiv(512, tiles), iters), 16);
        nsp = cdiv(iters, cdiv(iters, nsp));  // every split non-empty
    } else if (nib16 && bn == 64 && ep.mode != GEMM_GLU16 && vec_ok && tiles <= 256 && iters >= 64) {
        // at most one 128 x 64 tile per CU over a long K: two K halves fill the second
        // workgroup slot of each CU (Q4_0 4096 x 11008, M = 512: 81.0 -> 75.9 us with the
        // partial sums; 4096 x 4096 unchanged; Q8_0 and f16 weights run one workgroup per
        // CU and lose: Q8_0 89.9 -> 99.1 us)
        nsp = 2;
    }
    return F16qPlan{bm, bn, tiles, nsp};
}

// part_ws / noalloc: the split-K partials go to the caller's workspace and nothing is
// allocated (weights that need an f16 copy are then rejected); otherwise the allocator
// provides the workspace.
// defer_part: a split-K launch leaves its nsp partial tiles (m x n floats each, in K order) in
// a buffer handed to the caller (*defer_part, *defer_nsp; the caller adds them -- plus ep.res
// for the residual epilogue -- and frees the buffer with dev_free_on on s); an unsplit launch
// applies the epilogue as usual and returns *defer_part = nullptr, *defer_nsp = 1, and so does a
// split launch whose last-arriving splits add the slices in-kernel (the one-launch form).
int launch_gemm_f16q(const QWeight* w, const _Float16* x16, float* y, int64_t m, const GemmEpi& ep,
                     hipStream_t s, bool noalloc, float* part_ws, float** defer_part, int* defer_nsp) {
    if (m < 1) return TL_HIP_OK;
    if (w->nb % Q_KR != 0 || (ep.mode == GEMM_GLU16 && (w->n % 64 != 0))) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: the f16 GEMM takes K in steps of 128 (SwiGLU output: N in steps "
                  "of 64)");
        return TL_HIP_ERR_ARG;
    }
    if (ep.mode == GEMM_ROPE_KV &&
        (ep.rk.hd_shift < 2 || ep.rk.hd_shift > 12 || ep.rk.hd != (1 << ep.rk.hd_shift) || ep.rk.col_off < 0 ||
         ep.rk.col_off % ep.rk.hd || w->n % ep.rk.hd ||
         ep.rk.col_off + w->n > (int64_t)(ep.rk.H + 2 * ep.rk.KV) * ep.rk.hd || !ep.rk.q || !ep.rk.kc || !ep.rk.vc ||
         !ep.rk.ct || !ep.rk.st || !ep.rk.pos)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: the RoPE / KV epilogue takes whole heads of [q | k | v] (head size "
                  "a power of two of 4-4096, hd_shift its log2) and every output");
        return TL_HIP_ERR_ARG;
    }
    const bool needs_w16 = (w->ggml_type == TL_HIP_GGML_Q4_K && !w->us) || w->ggml_type == TL_HIP_GGML_Q6_K;
    if (noalloc && needs_w16) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: a %s weight needs an f16 copy for the MFMA GEMM, which the "
                  "allocation-free entry cannot make", ggml_type_name(w->ggml_type));
        return TL_HIP_ERR_ARG;
    }
    // the kernel addresses X, the weight stream and its scales through 32-bit buffer offsets
    // (quant bytes: k / 2 per row for the 4-bit types, k for Q8_0; an f16 copy 2 k)
    const int64_t wbytes = needs_w16 ? w->n * w->k * 2 : w->ggml_type == TL_HIP_GGML_Q8_0 ? w->n * w->k : w->n * w->k / 2;
    if (m * w->k * 2 >= (int64_t(1) << 31) || wbytes >= (int64_t(1) << 31)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: the f16 GEMM takes X and weights below 2 GiB");
        return TL_HIP_ERR_ARG;
    }
    constexpr int BM = 128;
    const F16qPlan plan = plan_f16q(w, m, ep, y);
    const int bm = plan.bm, bn = plan.bn;
    const int64_t tiles = plan.tiles, nsp = plan.nsp;
    // one launch (the tile's last split adds the slices) for the split plans of short inputs
    // (32- and 64-row tiles), when no other stream can run a call that shares the arrival
    // counters.  At 128-row tiles the deferred sum is cheaper: the RMSNorm that reads the
    // residual next adds the slices with a workgroup per row (512-token prefill 2.83 ms
    // against 2.89 ms with the in-kernel sum; 32 tokens 1.30 -> 1.21 ms with it).
    const bool fuse = f16q_fuse_ok(w, m, bm, bn, tiles, nsp, ep);
    // (the RoPE / KV epilogue is applied by the kernel that forms the sums: the GEMM, the
    // tile's last split, or k_splitk_sum_rope -- never left to the caller)
    const bool defer = defer_part && nsp > 1 && !noalloc && !fuse && ep.mode != GEMM_ROPE_KV;
    if (defer_part) {
        *defer_part = nullptr;
        *defer_nsp = 1;
    }
    tls_plan[0] = bm;
    tls_plan[1] = bn;
    tls_plan[2] = (int)nsp;
    float* part = nullptr;
    if (nsp > 1) {
        part = noalloc ? part_ws : static_cast<float*>(dev_alloc_on((size_t)nsp * m * w->n * sizeof(float), s));
        if (!part) {
            if (noalloc) set_error(TL_HIP_ERR_ARG, "ArgumentError: no workspace for the split-K partials");
            return noalloc ? TL_HIP_ERR_ARG : TL_HIP_ERR_ALLOC;
        }
    }
    const GemmEpi pe = nsp > 1 ? GemmEpi{GEMM_PLAIN, nullptr, nullptr, 0} : ep;
    float* const out = nsp > 1 ? part : y;
    const dim3 grid((unsigned)tiles, (unsigned)nsp);
    auto gemm = [&](auto qt, const uint8_t* q, const __half* d) {
        constexpr int QT = decltype(qt)::value;
        constexpr bool NIB16 = QT == TL_HIP_GGML_Q4_0 || QT == TL_HIP_GGML_Q4_K;
        if (NIB16 && bn == 96) {
            if constexpr (NIB16) k_qgemm_mfma<QT, BM, 96><<<grid, 512, 0, s>>>(q, d, x16, out, m, w->n, w->k, w->nb, pe);
        } else if (bn == 64) k_qgemm_mfma<QT, BM, 64><<<grid, 512, 0, s>>>(q, d, x16, out, m, w->n, w->k, w->nb, pe);
        else if (fuse) {
            if (bm == 32) k_qgemm_mfma<QT, 32, 32, true><<<grid, 512, 0, s>>>(q, d, x16, out, m, w->n, w->k, w->nb, ep, y);
            else k_qgemm_mfma<QT, 64, 32, true><<<grid, 512, 0, s>>>(q, d, x16, out, m, w->n, w->k, w->nb, ep, y);
        } else if (bm == 32) k_qgemm_mfma<QT, 32, 32><<<grid, 512, 0, s>>>(q, d, x16, out, m, w->n, w->k, w->nb, pe);
        else if (bm == 64) k_qgemm_mfma<QT, 64, 32><<<grid, 512, 0, s>>>(q, d, x16, out, m, w->n, w->k, w->nb, pe);
        else k_qgemm_mfma<QT, BM, 32><<<grid, 512, 0, s>>>(q, d, x16, out, m, w->n, w->k, w->nb, pe);
        if (nsp > 1 && !defer && !fuse) {
            const int64_t mn = m * w->n;
            if (ep.mode == GEMM_ROPE_KV)
                k_splitk_sum_rope<<<(unsigned)cdiv(mn / 4, 256), 256, 0, s>>>(part, mn, w->n, (int)nsp, ep.rk);
            else
                k_splitk_sum<<<(unsigned)cdiv(cdiv(mn, 4), 256), 256, 0, s>>>(
                    part, y, ep.mode == GEMM_RES ? ep.res : nullptr, mn, (int)nsp);
        }
    };
    if (w->ggml_type == TL_HIP_GGML_Q4_K && w->us) {
        gemm(std::integral_constant<int, TL_HIP_GGML_Q4_K>{}, w->qs, reinterpret_cast<const __half*>(w->us));
    } else if (w->ggml_type == TL_HIP_GGML_Q4_K || w->ggml_type == TL_HIP_GGML_Q6_K) {
        // K-quants: dequantize once into f16 operand order (n * k halves), then the same
        // MFMA pipeline with the weights read as stored
        _Float16* w16 = static_cast<_Float16*>(dev_alloc_on((size_t)w->n * w->k * sizeof(_Float16), s));
        if (!w16) {
            if (part && !noalloc) dev_free_on(part, s);
            return TL_HIP_ERR_ALLOC;
        }
        const QView qv{w->qs, w->d, w->hdr, w->qh, w->sc};
        const int64_t wunits = w->n * w->nb;
        if (w->ggml_type == TL_HIP_GGML_Q4_K)
            k_dequant_f16q<TL_HIP_GGML_Q4_K><<<(unsigned)cdiv(wunits, 256), 256, 0, s>>>(qv, w16, wunits);
        else
            k_dequant_f16q<TL_HIP_GGML_Q6_K><<<(unsigned)cdiv(wunits, 256), 256, 0, s>>>(qv, w16, wunits);
        gemm(std::integral_constant<int, TL_HIP_GGML_F16>{}, reinterpret_cast<const uint8_t*>(w16), nullptr);
        dev_free_on(w16, s);
    } else if (w->ggml_type == TL_HIP_GGML_Q4_0) {
        gemm(std::integral_constant<int, TL_HIP_GGML_Q4_0>{}, w->qs, w->d);
    } else {
        gemm(std::integral_constant<int, TL_HIP_GGML_Q8_0>{}, w->qs, w->d);
    }
    hipError_t e = hipGetLastError();
    if (defer && e == hipSuccess) {  // the partials are the caller's only on success
        *defer_part = part;
        *defer_nsp = (int)nsp;
    } else if (part && !noalloc) {
        dev_free_on(part, s);  // freed on s: reused at once only by later work on s
    }
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "quant gemm launch");
}

// y = res + sum of the nsp partial slices (m n floats each) in slice order: the sum a
// deferred split-K GEMM leaves to its caller.
int launch_splitk_sum(const float* part, float* y, const float* res, int64_t mn, int nsp, hipStream_t s) {
    if (mn <= 0) return TL_HIP_OK;
    k_splitk_sum<<<(unsigned)cdiv(cdiv(mn, 4), 256), 256, 0, s>>>(part, y, res, mn, nsp);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "split-K sum launch");
}

int launch_quant_gemm(const QWeight* w, const float* x, float* y, int64_t m, hipStream_t s,
                      int mode) {
    if (m < 1) return TL_HIP_OK;
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: x must be 16-byte aligned");
        return TL_HIP_ERR_ARG;
    }
    if (mode != 0 && w->nb % Q_KR != 0) mode = 0;  // the MFMA pipeline takes K in steps of 128

    if (mode == 0) {
        dim3 grid((unsigned)cdiv(w->n, F_BN), (unsigned)cdiv(m, F_BM));
        const QView qv{w->qs, w->d, w->hdr, w->qh, w->sc};
        switch (w->ggml_type) {
            case TL_HIP_GGML_Q4_0: k_qgemm_f32<TL_HIP_GGML_Q4_0><<<grid, 256, 0, s>>>(qv, x, y, m, w->n, w->k, w->nb); break;
            case TL_HIP_GGML_Q8_0: k_qgemm_f32<TL_HIP_GGML_Q8_0><<<grid, 256, 0, s>>>(qv, x, y, m, w->n, w->k, w->nb); break;
            case TL_HIP_GGML_Q4_K: k_qgemm_f32<TL_HIP_GGML_Q4_K><<<grid, 256, 0, s>>>(qv, x, y, m, w->n, w->k, w->nb); break;
            default: k_qgemm_f32<TL_HIP_GGML_Q6_K><<<grid, 256, 0, s>>>(qv, x, y, m, w->n, w->k, w->nb); break;
        }
    } else {
        // a Q4_K tensor gets its unit scales on its first f16 GEMM (kept with the tensor)
        if (int rc = q4k_build_unit_scales(const_cast<QWeight*>(w), s)) return rc;
        // short inputs: one launch over f32 X (no conversion, no split-K partial sums)
        if (m <= 16 && gemm_short_ok(w, m)) return launch_gemm_short(w, x, y, m, s, nullptr, false);
        // X -> f16 in the operand k order (a workspace of m * k halves), then the MFMA GEMM
        _Float16* x16 = static_cast<_Float16*>(dev_alloc_on((size_t)m * w->k * sizeof(_Float16), s));
        if (!x16) return TL_HIP_ERR_ALLOC;
        int rc = launch_x_to_f16q(x, x16, m, w->k, f16q_order(w->ggml_type), s);
        if (rc == TL_HIP_OK) rc = launch_gemm_f16q(w, x16, y, m, GemmEpi{GEMM_PLAIN, nullptr, nullptr, 0}, s);
        dev_free_on(x16, s);  // freed on s: reused at once only by later work on s
        if (rc) return rc;
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


// ------------------------------------------------------ allocation-free GEMM entry ----
// The workspace of tl_hip_launch_quant_gemm_noalloc: the f16 copy of X (m * k halves, rounded
// up to 256 bytes) followed by the split-K partial tiles (nsp * m * n floats).  One array per
// GPU, held until the process ends; its device address is looked up once per device.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
constexpr int SCRATCH_MAX_DEVICES = 64;
static uint8_t* g_scratch_ptr[SCRATCH_MAX_DEVICES] = {};

// Device address of `scratch` on device dev (the host-side name is only a stand-in).
static uint8_t* scratch_on(int dev) {
    if (dev < 0 || dev >= SCRATCH_MAX_DEVICES) {
        set_error(TL_HIP_ERR_DEVICE, "DeviceError: device %d outside the scratch table", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        void* p = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p) {
            hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
            return nullptr;
        }
        g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
    }
    return g_scratch_ptr[dev];
}

int noalloc_scratch_init(int device) { return scratch_on(device) ? TL_HIP_OK : tl_hip_last_status(); }

extern "C" int tl_hip_launch_quant_gemm_noalloc(const tl_hip_qtensor* h, const float* x, float* y, int64_t m,
                                                int use_f16_mfma, void* stream) {
    if (!h || !x || !y) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: weight, x or y");
        return TL_HIP_ERR_NULL;
    }
    DeviceState* st = state();
    if (!st) return tl_hip_last_status();
    const QWeight* w = reinterpret_cast<const QWeight*>(h);
    hipStream_t s = stream ? (hipStream_t)stream : cur_stream();
    if (m < 1) return TL_HIP_OK;
    if (!use_f16_mfma || w->nb % Q_KR != 0) return launch_quant_gemm(w, x, y, m, s, 0);  // f32 path: no workspace
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: x must be 16-byte aligned");
        return TL_HIP_ERR_ARG;
    }
    const GemmEpi plain{GEMM_PLAIN, nullptr, nullptr, 0};
    // short inputs read X in f32; the scratch holds only their split-K partial slices
    const bool short_in = m <= 16 && gemm_short_ok(w, m);
    if (short_in && gemm_short_workspace(w, m, y) > NOALLOC_SCRATCH_BYTES) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: the call needs %zu bytes of scratch (split-K partials), the "
                  "allocation-free GEMM has %zu MiB", gemm_short_workspace(w, m, y), NOALLOC_SCRATCH_BYTES >> 20);
        return TL_HIP_ERR_ARG;
    }
    if (!short_in && m > (int64_t)(NOALLOC_SCRATCH_BYTES / 2 / (size_t)w->k)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: %lld x %lld input exceeds the %zu MiB scratch of the allocation-free "
                  "GEMM", (long long)m, (long long)w->k, NOALLOC_SCRATCH_BYTES >> 20);
        return TL_HIP_ERR_ARG;
    }
    const size_t x16_bytes = ((size_t)m * w->k * 2 + 255) & ~size_t(255);
    const F16qPlan plan = plan_f16q(w, m, plain, y);
    const size_t part_bytes = plan.nsp > 1 ? (size_t)plan.nsp * m * w->n * 4 : 0;
    if (!short_in && x16_bytes + part_bytes > NOALLOC_SCRATCH_BYTES) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: the call needs %zu bytes of scratch (X in f16 + split-K partials), "
                  "the allocation-free GEMM has %zu MiB", x16_bytes + part_bytes, NOALLOC_SCRATCH_BYTES >> 20);
        return TL_HIP_ERR_ARG;
    }
    if (w->ggml_type == TL_HIP_GGML_Q6_K || (w->ggml_type == TL_HIP_GGML_Q4_K && !w->us)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: a %s weight needs an f16 copy for the MFMA GEMM, which the "
                  "allocation-free entry cannot make (use_f16_mfma = 0 takes the f32 path)",
                  ggml_type_name(w->ggml_type));
        return TL_HIP_ERR_ARG;
    }
    if (note_stream_syncs(s)) {
        // the first call on a caller stream synchronises the library stream once (allocator
        // bookkeeping), which a stream under capture must not see
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
            set_error(TL_HIP_ERR_ARG, "ArgumentError: the first library call on a caller stream cannot be captured; "
                      "make one call on that stream before capturing it");
            return TL_HIP_ERR_ARG;
        }
        (void)hipGetLastError();
    }
    note_stream(s);
    uint8_t* base = scratch_on(st->device);
    if (!base) return tl_hip_last_status();
    if (short_in) return launch_gemm_short(w, x, y, m, s, reinterpret_cast<float*>(base), true);
    _Float16* x16 = reinterpret_cast<_Float16*>(base);
    int rc = launch_x_to_f16q(x, x16, m, w->k, f16q_order(w->ggml_type), s);
    if (rc == TL_HIP_OK)
        rc = launch_gemm_f16q(w, x16, y, m, plain, s, true, reinterpret_cast<float*>(base + x16_bytes));
    if (rc) return rc;
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "quant gemm launch");
}

}  // namespace tlhip

extern "C" int tl_hip_debug_last_gemm_plan(int* tile_m, int* tile_n, int* k_splits) {
    if (!tile_m || !tile_n || !k_splits) {
        tlhip::set_error(TL_HIP_ERR_NULL, "NullPointerError: output");
        return TL_HIP_ERR_NULL;
    }
    *tile_m = tlhip::tls_plan[0];
    *tile_n = tlhip::tls_plan[1];
    *k_splits = tlhip::tls_plan[2];
    return TL_HIP_OK;
}
