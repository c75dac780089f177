/*
 * tl_cpu_oracle.c -- CPU restatement of the reference's tl_cpu path for the quantized
 * LLM-inference hot path.  TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check
 * and the CPU-baseline leg of the benchmark load this library as the checker.  The
 * product (tl_amd/libtl_hip.so) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to the
 * reference repository root).  Floating-point semantics follow Rust on Linux:
 *   - f32 arithmetic, each `a * b` and `a + b` rounded separately (no FMA contraction;
 *     build with -ffp-contract=off),
 *   - Iterator::sum folds left to right,
 *   - f32::exp / powf / cos / sin / sqrt are the platform libm (glibc) expf / powf /
 *     cosf / sinf / sqrtf.
 *
 * Pinning (which check fixes each function; see tests/test_oracle.py):
 *   tlo_f16_to_f32          all 65536 bit patterns vs numpy float16 (IEEE binary16)
 *   tlo_dequantize_q4_0/q8_0 hand-built golden blocks (tests/golden/q_blocks.json) and
 *                           the closed form d*(q-8) / d*q (exact in f32)
 *   tlo_dequantize_q4_k/q6_k golden super-blocks (tests/golden/k_blocks.json) built by
 *                           packing chosen (scale, min, q) values with llama.cpp's
 *                           published block encoders; expected values come from the chosen
 *                           values, not from the decoder
 *   tlo_matmul              reference KAT [[58,64],[139,154]] (tl_cpu tests
 *                           cpu_tensor_tests.rs:488-497) + float64 brute force
 *   tlo_rms_norm            closed form of tl_cuda nn_llm_test.rs:123-132
 *   tlo_rope_new_cos/sin    pos-0 row = (1, 0) (nn_llm_test.rs:151-169), libm values
 *   tlo_apply_rope          pos-0 identity (cuda_shader_test.rs:332-355), rotation norm
 *   tlo_softmax             rows sum to 1, monotone (cpu_tensor_tests.rs:439-449)
 *   tlo_argmax_last         hand-built tie cases (last maximum wins)
 *   tlo_sample              closed forms of two- and four-element distributions (cutoff and
 *                           choice by hand), ties in index order, NaN / inf -> 0, and a
 *                           float64 restatement (numpy stable argsort, cumulative sums) on
 *                           random inputs wherever top_p and r are clear of every running sum
 *   tlo_fused_add_relu      reference KAT (tl_cuda new_ops_comprehensive_test.rs:624-632)
 *   tlo_fused_bias_gelu     reference KAT gelu(0) = 0 (new_ops_comprehensive_test.rs:687-693),
 *                           signs at +-1.1 (tl_metal fused_ops_test.rs:60-75), limits
 *                           gelu(v) -> v / 0 for large |v|, bias broadcast i % nbias
 *   tlo_fused_silu_mul      reference KATs f(0,1) = 0, f(1,1) = 0.7311 (tl_cuda
 *                           new_ops_comprehensive_test.rs:635-645), fused vs unfused within
 *                           1e-4 (tl_metal fused_ops_test.rs:42-56), float64 closed form
 *   tlo_binop               numpy float32 add / mul / sub / div with broadcasting, IEEE
 *                           specials, the ShapeMismatch rule (tests/test_oracle_model.py)
 *   tlo_fused_rotary_emb    one head vector: the textbook half-split rotation (norm of each
 *                           pair kept, f = 0 identity, f = pi/2 (x0, x1) -> (-x1, x0));
 *                           several vectors: brute-force replay of the reference loop
 *   tlo_sdpa                a causal ones-mask equals the pinned chatbot attention chain bit for
 *                           bit (tests/test_oracle_model.py); float64 softmax(QK^T/sqrt(d_k))V;
 *                           mask == 0 drops a key, a fully masked row averages V; seq_k = 1
 *                           returns the V row
 *   remaining glue ops      numpy equivalents on small inputs
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TLO_OK 0
#define TLO_ERR_ARG -1
#define TLO_ERR_SHAPE -2
#define TLO_ERR_SIZE -3
#define TLO_ERR_INDEX -4

/* IEEE binary16 -> binary32, exact (half 2.7.1 f16::to_f32 as called at
 * crates/tl_runtime/src/quantized.rs:176, 208, 249). */
float tlo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { e++; man <<= 1; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* QTensor::dequantize_f16 (crates/tl_runtime/src/quantized.rs:167-180). */
int tlo_dequantize_f16(const uint8_t* data, int64_t nbytes, float* out) {
    if (nbytes % 2 != 0) return TLO_ERR_SIZE;
    for (int64_t i = 0; i < nbytes / 2; i++) {
        uint16_t h = (uint16_t)(data[2 * i] | (data[2 * i + 1] << 8));
        out[i] = tlo_f16_to_f32(h);
    }
    return TLO_OK;
}

/* QTensor::dequantize_q4_0 (crates/tl_runtime/src/quantized.rs:182-225).  Block = f16 d
 * (LE) + 16 bytes; low nibble of byte j -> element j, high nibble -> element j+16,
 * value d * (q - 8). */
int tlo_dequantize_q4_0(const uint8_t* data, int64_t nbytes, int64_t numel, float* out) {
    if (numel % 32 != 0) return TLO_ERR_SHAPE;               /* quantized.rs:190-192 */
    int64_t nblocks = numel / 32;
    if (nbytes != nblocks * 18) return TLO_ERR_SIZE;         /* quantized.rs:195-200 */
    const uint8_t* p = data;
    for (int64_t b = 0; b < nblocks; b++) {
        float d = tlo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        p += 2;
        float* y = out + b * 32;
        for (int j = 0; j < 16; j++) {
            int x0 = (p[j] & 0x0F) - 8;
            int x1 = ((p[j] >> 4) & 0x0F) - 8;
            y[j] = d * (float)x0;
            y[j + 16] = d * (float)x1;
        }
        p += 16;
    }
    return TLO_OK;
}

/* QTensor::dequantize_q8_0 (crates/tl_runtime/src/quantized.rs:227-260): f16 d + 32 x i8,
 * value d * q. */
int tlo_dequantize_q8_0(const uint8_t* data, int64_t nbytes, int64_t numel, float* out) {
    if (numel % 32 != 0) return TLO_ERR_SHAPE;
    int64_t nblocks = numel / 32;
    if (nbytes != nblocks * 34) return TLO_ERR_SIZE;
    const uint8_t* p = data;
    for (int64_t b = 0; b < nblocks; b++) {
        float d = tlo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        p += 2;
        for (int j = 0; j < 32; j++) out[b * 32 + j] = d * (float)(int8_t)p[j];
        p += 32;
    }
    return TLO_OK;
}

/* QTensor::get_scale_min_k4 (crates/tl_runtime/src/quantized.rs:405-415): 6-bit scale and
 * min of sub-block j (0..7) from the 12 packed bytes of a Q4_K block. */
static void tlo_scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* QTensor::dequantize_q4_k (crates/tl_runtime/src/quantized.rs:337-400).  Block of 256
 * weights, 144 bytes: f16 d, f16 dmin, 12 packed scale/min bytes, 128 quant bytes.  Group g
 * (64 weights) uses quant bytes 32g..32g+31: low nibble of byte l -> weight 64g + l with
 * sub-block 2g's (scale, min), high nibble -> weight 64g + 32 + l with sub-block 2g+1's.
 * Value (d * sc) * q - dmin * m, each product rounded to f32 (all three are exact). */
int tlo_dequantize_q4_k(const uint8_t* data, int64_t nbytes, int64_t numel, float* out) {
    if (numel % 256 != 0) return TLO_ERR_SHAPE;      /* quantized.rs:342-344 */
    int64_t nblocks = numel / 256;
    if (nbytes != nblocks * 144) return TLO_ERR_SIZE; /* quantized.rs:347-352 */
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t* p = data + b * 144;
        float d = tlo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        float dmin = tlo_f16_to_f32((uint16_t)(p[2] | (p[3] << 8)));
        const uint8_t* scales = p + 4;
        const uint8_t* q = p + 16;
        float* y = out + b * 256;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t sc1, m1, sc2, m2;
            tlo_scale_min_k4(is, scales, &sc1, &m1);
            tlo_scale_min_k4(is + 1, scales, &sc2, &m2);
            float d1 = d * (float)sc1, min1 = dmin * (float)m1;
            float d2 = d * (float)sc2, min2 = dmin * (float)m2;
            for (int l = 0; l < 32; l++) y[j + l] = d1 * (float)(q[l] & 0xF) - min1;
            for (int l = 0; l < 32; l++) y[j + 32 + l] = d2 * (float)(q[l] >> 4) - min2;
            q += 32;
            is += 2;
        }
    }
    return TLO_OK;
}

/* QTensor::dequantize_q6_k (crates/tl_runtime/src/quantized.rs:268-329).  Block of 256
 * weights, 210 bytes: ql[128] (low 4 bits), qh[64] (high 2 bits), 16 int8 sub-block scales,
 * f16 d at bytes 208-209.  Per 128-weight half (ql += 64, qh += 32, scales += 8), l < 32:
 *   weight l      = ql[l] & 15      | (qh[l] >> 0 & 3) << 4, scale[l/16]
 *   weight l + 32 = ql[l + 32] & 15 | (qh[l] >> 2 & 3) << 4, scale[l/16 + 2]
 *   weight l + 64 = ql[l] >> 4      | (qh[l] >> 4 & 3) << 4, scale[l/16 + 4]
 *   weight l + 96 = ql[l + 32] >> 4 | (qh[l] >> 6 & 3) << 4, scale[l/16 + 6]
 * value (d * scale) * (q - 32), evaluated left to right as `d * sc as f32 * q as f32`. */
int tlo_dequantize_q6_k(const uint8_t* data, int64_t nbytes, int64_t numel, float* out) {
    if (numel % 256 != 0) return TLO_ERR_SHAPE;      /* quantized.rs:273-275 */
    int64_t nblocks = numel / 256;
    if (nbytes != nblocks * 210) return TLO_ERR_SIZE; /* quantized.rs:278-283 */
    for (int64_t b = 0; b < nblocks; b++) {
        const uint8_t* p = data + b * 210;
        float d = tlo_f16_to_f32((uint16_t)(p[208] | (p[209] << 8)));
        const uint8_t* ql = p;
        const uint8_t* qh = p + 128;
        const uint8_t* sc = p + 192;
        for (int half = 0; half < 2; half++) {
            float* y = out + b * 256 + half * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * (float)(int8_t)sc[is + 0] * (float)q1;
                y[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
            }
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
    return TLO_OK;
}

/* CpuTensor::transpose_impl for a 2-D tensor (crates/tl_cpu/src/tensor.rs:902-941, reached
 * from tl_device_tensor_transpose_2d, crates/tl_runtime/src/device_ffi.rs:1502). */
void tlo_transpose_2d(const float* a, int64_t rows, int64_t cols, float* out) {
    for (int64_t i = 0; i < rows; i++)
        for (int64_t j = 0; j < cols; j++) out[j * rows + i] = a[i * cols + j];
}

/* CpuTensor::transpose_impl, general rank (crates/tl_cpu/src/tensor.rs:902-941). */
int tlo_transpose(const float* a, const int64_t* shape, int rank, int d0, int d1, float* out) {
    if (rank < 2) return TLO_ERR_ARG;
    if (d0 >= rank || d1 >= rank || d0 < 0 || d1 < 0) return TLO_ERR_SHAPE;
    int64_t nshape[8], idx[8], total = 1;
    if (rank > 8) return TLO_ERR_ARG;
    for (int d = 0; d < rank; d++) { nshape[d] = shape[d]; total *= shape[d]; }
    nshape[d0] = shape[d1];
    nshape[d1] = shape[d0];
    for (int64_t f = 0; f < total; f++) {
        int64_t rem = f;
        for (int d = rank - 1; d >= 0; d--) { idx[d] = rem % shape[d]; rem /= shape[d]; }
        int64_t t = idx[d0]; idx[d0] = idx[d1]; idx[d1] = t;
        int64_t nf = 0, stride = 1;
        for (int d = rank - 1; d >= 0; d--) { nf += idx[d] * stride; stride *= nshape[d]; }
        out[nf] = a[f];
    }
    return TLO_OK;
}

/* CpuTensor::matmul_impl (crates/tl_cpu/src/tensor.rs:1248-1313).  A is [..batch, m, k]
 * (rank >= 2) or [k]; B is [..., k, n] or [k].  B is batched only when its rank > 2
 * (tensor.rs:1286-1288).  `sum` starts at 0 and adds a*b left to right (tensor.rs:1300).
 * Returns the output element count via *out_numel when non-NULL. */
int tlo_matmul(const float* A, const int64_t* ashape, int arank, const float* B,
               const int64_t* bshape, int brank, float* C) {
    if (arank < 1 || brank < 1) return TLO_ERR_SHAPE;
    int64_t m, k, k2, n;
    if (arank >= 2) { m = ashape[arank - 2]; k = ashape[arank - 1]; } else { m = 1; k = ashape[0]; }
    if (brank >= 2) { k2 = bshape[brank - 2]; n = bshape[brank - 1]; } else { k2 = bshape[0]; n = 1; }
    if (k != k2) return TLO_ERR_SHAPE;
    int64_t batch = 1;
    for (int d = 0; d < arank - 2; d++) batch *= ashape[d];
    int64_t alen = 1, blen = 1;
    for (int d = 0; d < arank; d++) alen *= ashape[d];
    for (int d = 0; d < brank; d++) blen *= bshape[d];
    for (int64_t b = 0; b < batch; b++) {
        int64_t a_off = b * m * k;
        int64_t b_bs = brank >= 2 ? k * n : bshape[0];
        int64_t b_off = brank > 2 ? b * b_bs : 0;
        for (int64_t i = 0; i < m; i++) {
            for (int64_t j = 0; j < n; j++) {
                float sum = 0.0f;
                for (int64_t p = 0; p < k; p++) {
                    int64_t ai = a_off + i * k + p;
                    int64_t bi = brank >= 2 ? b_off + p * n + j : p;
                    if (ai < alen && bi < blen) sum += A[ai] * B[bi];
                }
                C[b * m * n + i * n + j] = sum;
            }
        }
    }
    return TLO_OK;
}

/* Same per-element arithmetic as tlo_matmul for a plain 2-D product C[m,n] = A[m,k] . B[k,n]
 * (each C[i,j] is the left-to-right sum over p of A[i,p]*B[p,j], starting from 0), with
 * the loops interchanged and split over threads.  Bit-identical to tlo_matmul; used where
 * the faithful loop order is too slow (whole-model runs). */
void tlo_matmul_fast(const float* A, const float* B, float* C, int64_t m, int64_t k, int64_t n) {
    const int64_t JB = 256;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t i0 = 0; i0 < m; i0 += 4) {
        for (int64_t j0 = 0; j0 < n; j0 += JB) {
            int64_t i1 = i0 + 4 < m ? i0 + 4 : m;
            int64_t j1 = j0 + JB < n ? j0 + JB : n;
            float acc[4][256];
            for (int64_t i = i0; i < i1; i++)
                for (int64_t j = j0; j < j1; j++) acc[i - i0][j - j0] = 0.0f;
            for (int64_t p = 0; p < k; p++) {
                const float* brow = B + p * n;
                for (int64_t i = i0; i < i1; i++) {
                    float a = A[i * k + p];
                    float* ac = acc[i - i0];
                    for (int64_t j = j0; j < j1; j++) ac[j - j0] += a * brow[j];
                }
            }
            for (int64_t i = i0; i < i1; i++)
                for (int64_t j = j0; j < j1; j++) C[i * n + j] = acc[i - i0][j - j0];
        }
    }
}

/* tl_qtensor_matmul, TL_DEVICE=cpu branch (crates/tl_runtime/src/system.rs:193-222):
 * dequantize W [n,k] (quantized.rs:117-141), transpose to [k,n] (tensor.rs:902-941), then
 * matmul_impl x[m,k] . W^T (tensor.rs:1248-1313).  ggml_type: 2 = Q4_0, 8 = Q8_0,
 * 12 = Q4_K, 14 = Q6_K, 1 = F16, 0 = F32 (GGML type ids).  `fast` selects tlo_matmul_fast (bit-identical). */
int tlo_qtensor_matmul(const float* x, int64_t m, int64_t k, const uint8_t* wdata,
                       int64_t wbytes, int ggml_type, int64_t n, float* y, int fast) {
    float* w = (float*)malloc(sizeof(float) * (size_t)(n * k));
    float* wt = (float*)malloc(sizeof(float) * (size_t)(n * k));
    if (!w || !wt) { free(w); free(wt); return TLO_ERR_ARG; }
    int rc;
    if (ggml_type == 2) rc = tlo_dequantize_q4_0(wdata, wbytes, n * k, w);
    else if (ggml_type == 8) rc = tlo_dequantize_q8_0(wdata, wbytes, n * k, w);
    else if (ggml_type == 12) rc = tlo_dequantize_q4_k(wdata, wbytes, n * k, w);
    else if (ggml_type == 14) rc = tlo_dequantize_q6_k(wdata, wbytes, n * k, w);
    else if (ggml_type == 1) rc = wbytes == n * k * 2 ? tlo_dequantize_f16(wdata, wbytes, w) : TLO_ERR_SIZE;
    else if (ggml_type == 0) { rc = wbytes == n * k * 4 ? TLO_OK : TLO_ERR_SIZE; if (!rc) memcpy(w, wdata, (size_t)wbytes); }
    else rc = TLO_ERR_ARG;
    if (rc == TLO_OK) {
        tlo_transpose_2d(w, n, k, wt);
        if (fast) {
            tlo_matmul_fast(x, wt, y, m, k, n);
        } else {
            int64_t as[2] = {m, k}, bs[2] = {k, n};
            rc = tlo_matmul(x, as, 2, wt, bs, 2, y);
        }
    }
    free(w);
    free(wt);
    return rc;
}

/* tl_cpu_tensor_rms_norm (crates/tl_cpu/src/ffi.rs:2444-2486): per row of the last dim,
 * mean_sq = (sum v*v) / n; rms = sqrt(mean_sq + eps); out = x / rms; then, when a weight is
 * given, the broadcast mul_impl out * w (tensor.rs:549-609, 619-621). */
void tlo_rms_norm(const float* x, int64_t rows, int64_t n, const float* w, float eps, float* out) {
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * n;
        float s = 0.0f;
        for (int64_t i = 0; i < n; i++) s += xr[i] * xr[i];
        float ms = s / (float)n;
        float rms = sqrtf(ms + eps);
        for (int64_t i = 0; i < n; i++) {
            float v = xr[i] / rms;
            out[r * n + i] = w ? v * w[i] : v;
        }
    }
}

/* GpuFusedOps::fused_rms_norm for CpuTensor (crates/tl_cpu/src/fused_ops.rs:37-57):
 * x * (1/sqrt(sum_sq/n + eps)) * w. */
void tlo_fused_rms_norm(const float* x, int64_t rows, int64_t n, const float* w, float eps, float* out) {
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * n;
        float s = 0.0f;
        for (int64_t i = 0; i < n; i++) s += xr[i] * xr[i];
        float rcp = 1.0f / sqrtf(s / (float)n + eps);
        for (int64_t i = 0; i < n; i++) out[r * n + i] = xr[i] * rcp * w[i];
    }
}

/* GpuFusedOps::fused_add_rms_norm (crates/tl_cpu/src/fused_ops.rs:59-85). */
void tlo_fused_add_rms_norm(const float* x, const float* res, int64_t rows, int64_t n,
                            const float* w, float eps, float* out) {
    for (int64_t r = 0; r < rows; r++) {
        float s = 0.0f;
        for (int64_t i = 0; i < n; i++) {
            float v = x[r * n + i] + res[r * n + i];
            s += v * v;
        }
        float rcp = 1.0f / sqrtf(s / (float)n + eps);
        for (int64_t i = 0; i < n; i++) {
            float a = x[r * n + i] + res[r * n + i];
            out[r * n + i] = a * rcp * w[i];
        }
    }
}

/* tl_cpu_tensor_rope_new_cos / _sin (crates/tl_cpu/src/ffi.rs:2589-2629): table
 * [seq_len, dim]; freq_i = 1 / base^(2i/dim); entries 2i and 2i+1 both hold cos (sin) of
 * pos * freq_i.  (IDevice passes (dim, seq_len, base); tl_cpu device_impl.rs:1616-1632
 * swaps them into this (seq_len, dim, base) order.) */
void tlo_rope_new_cos(int64_t seq_len, int64_t dim, float base, float* out) {
    int64_t half = dim / 2, o = 0;
    for (int64_t pos = 0; pos < seq_len; pos++)
        for (int64_t i = 0; i < half; i++) {
            float freq = 1.0f / powf(base, 2.0f * (float)i / (float)dim);
            float v = cosf((float)pos * freq);
            out[o++] = v;
            out[o++] = v;
        }
}

void tlo_rope_new_sin(int64_t seq_len, int64_t dim, float base, float* out) {
    int64_t half = dim / 2, o = 0;
    for (int64_t pos = 0; pos < seq_len; pos++)
        for (int64_t i = 0; i < half; i++) {
            float freq = 1.0f / powf(base, 2.0f * (float)i / (float)dim);
            float v = sinf((float)pos * freq);
            out[o++] = v;
            out[o++] = v;
        }
}

/* tl_cpu_tensor_apply_rope (crates/tl_cpu/src/ffi.rs:2631-2686): for every vector of the
 * last dim (head_dim) and each interleaved pair (i, i+1), i even, rotate by the table's
 * entry i -- only the first head_dim entries of the table are read, so every vector uses
 * row 0 of the (narrowed) table; entries past the table's end read as cos 1, sin 0. */
void tlo_apply_rope(const float* x, int64_t total, int64_t head_dim, const float* cos_t,
                    int64_t cos_len, const float* sin_t, int64_t sin_len, float* out) {
    if (head_dim == 0 || total == 0) {
        memcpy(out, x, sizeof(float) * (size_t)total);
        return;
    }
    int64_t nv = total / head_dim;
    for (int64_t v = 0; v < nv; v++) {
        int64_t off = v * head_dim;
        for (int64_t i = 0; i < head_dim; i += 2) {
            float c = i < cos_len ? cos_t[i] : 1.0f;
            float s = i < sin_len ? sin_t[i] : 0.0f;
            float x0 = x[off + i], x1 = x[off + i + 1];
            out[off + i] = x0 * c - x1 * s;
            out[off + i + 1] = x0 * s + x1 * c;
        }
    }
}

/* tl_cpu_tensor_silu (crates/tl_cpu/src/ffi.rs:2097-2113): x * (1 / (1 + exp(-x))). */
void tlo_silu(const float* x, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * (1.0f / (1.0f + expf(-x[i])));
}

/* GpuFusedOps::fused_silu_mul (crates/tl_cpu/src/fused_ops.rs:15-35 with silu at 12-15):
 * (g / (1 + exp(-g))) * u. */
void tlo_fused_silu_mul(const float* g, const float* u, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) out[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* GpuFusedOps::fused_rotary_emb for CpuTensor (crates/tl_cpu/src/fused_ops.rs:87-108): for id
 * in 0 .. count / 2, with half = head_dim / 2, p = id % half, base = id - p, f = freqs[p]:
 *   out[base + p]        = x[base + p] cos f - x[base + p + half] sin f
 *   out[base + p + half] = x[base + p] sin f + x[base + p + half] cos f
 * in id order over a zero-filled output, cos / sin of f32 (f32::cos / f32::sin).  Past the
 * first head vector the pairs of consecutive ids overlap (base steps by half, not head_dim),
 * and later ids overwrite earlier ones; restated as the reference loop, quirk included. */
void tlo_fused_rotary_emb(const float* x, int64_t count, const float* freqs, int64_t head_dim, float* out) {
    const int64_t half = head_dim / 2;
    for (int64_t i = 0; i < count; i++) out[i] = 0.0f;
    if (half <= 0) return;
    for (int64_t id = 0; id < count / 2; id++) {
        const int64_t p = id % half, base = id - p;
        const float f = freqs[p], c = cosf(f), sn = sinf(f);
        const float x0 = x[base + p], x1 = x[base + p + half];
        out[base + p] = x0 * c - x1 * sn;
        out[base + p + half] = x0 * sn + x1 * c;
    }
}

/* GpuFusedOps::fused_add_relu for CpuTensor (crates/tl_cpu/src/fused_ops.rs:110-120):
 * (a + b).max(0.0); f32::max returns the other operand when one is NaN. */
void tlo_fused_add_relu(const float* a, const float* b, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) out[i] = fmaxf(a[i] + b[i], 0.0f);
}

/* GpuFusedOps::fused_bias_gelu for CpuTensor (crates/tl_cpu/src/fused_ops.rs:122-131) with the
 * crate's gelu (fused_ops.rs:20-22): v = x + bias[i % nbias];
 * 0.5 v (1 + tanh(FRAC_2_SQRT_PI (v + 0.044715 v^3))), v^3 = powi(3) = (v v) v.  The constant
 * is 2/sqrt(pi) as the reference writes it (the textbook tanh form has sqrt(2/pi)). */
void tlo_fused_bias_gelu(const float* x, int64_t n, const float* bias, int64_t nbias, float* out) {
    const float k = 1.12837916709551257390f;  /* f32 FRAC_2_SQRT_PI */
    for (int64_t i = 0; i < n; i++) {
        const float v = x[i] + bias[i % nbias];
        const float v3 = (v * v) * v;
        out[i] = 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * v3)));
    }
}

/* CpuTensor::elementwise_binop (crates/tl_cpu/src/tensor.rs:549-609): numpy broadcasting;
 * op 0 = add (tensor.rs:612-614), 1 = mul (619-621), 2 = sub, 3 = div.  out_shape must hold
 * max(arank, brank) entries; returns the output rank or a negative error. */
int tlo_binop(int op, const float* a, const int64_t* ashape, int arank, const float* b,
              const int64_t* bshape, int brank, float* out, int64_t* out_shape) {
    int nd = arank > brank ? arank : brank;
    if (nd > 8) return TLO_ERR_ARG;
    int64_t as[8], bs[8], ast[8], bst[8], alen = 1, blen = 1, olen = 1;
    for (int d = 0; d < arank; d++) alen *= ashape[d];
    for (int d = 0; d < brank; d++) blen *= bshape[d];
    if (alen == 0 || blen == 0) { out_shape[0] = 0; return 1; }
    for (int d = 0; d < nd; d++) {
        as[d] = d < nd - arank ? 1 : ashape[d - (nd - arank)];
        bs[d] = d < nd - brank ? 1 : bshape[d - (nd - brank)];
        if (as[d] != bs[d] && as[d] != 1 && bs[d] != 1) return TLO_ERR_SHAPE;
        out_shape[d] = as[d] > bs[d] ? as[d] : bs[d];
        olen *= out_shape[d];
    }
    int64_t sa = 1, sb = 1;
    for (int d = nd - 1; d >= 0; d--) {
        ast[d] = as[d] == 1 ? 0 : sa;
        bst[d] = bs[d] == 1 ? 0 : sb;
        sa *= as[d];
        sb *= bs[d];
    }
    for (int64_t f = 0; f < olen; f++) {
        int64_t rem = f, ai = 0, bi = 0, stride = olen;
        for (int d = 0; d < nd; d++) {
            stride /= out_shape[d];
            int64_t c = rem / stride;
            rem %= stride;
            ai += c * ast[d];
            bi += c * bst[d];
        }
        float av = ai < alen ? a[ai] : 0.0f, bv = bi < blen ? b[bi] : 0.0f, r;
        switch (op) {
            case 0: r = av + bv; break;
            case 1: r = av * bv; break;
            case 2: r = av - bv; break;
            default: r = av / bv; break;
        }
        out[f] = r;
    }
    return nd;
}

/* tl_cpu_tensor_scale (crates/tl_cpu/src/ffi.rs:2083-2094): mul_scalar_impl(s as f32). */
void tlo_scale(const float* x, int64_t n, double s, float* out) {
    float sf = (float)s;
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * sf;
}

/* CpuTensor::softmax_impl (crates/tl_cpu/src/tensor.rs:1065-1092): max pass (strict >,
 * starting at -inf), e = exp(x - max) stored and summed left to right, then x /= sum. */
int tlo_softmax(const float* x, const int64_t* shape, int rank, int axis, float* out) {
    if (axis < 0) axis += rank;
    if (axis < 0 || axis >= rank) return TLO_ERR_SHAPE;
    int64_t outer = 1, inner = 1, as = shape[axis], total = 1;
    for (int d = 0; d < axis; d++) outer *= shape[d];
    for (int d = axis + 1; d < rank; d++) inner *= shape[d];
    for (int d = 0; d < rank; d++) total *= shape[d];
    memcpy(out, x, sizeof(float) * (size_t)total);
    for (int64_t i = 0; i < outer; i++)
        for (int64_t k = 0; k < inner; k++) {
            float mx = -INFINITY;
            for (int64_t j = 0; j < as; j++) {
                float v = out[i * as * inner + j * inner + k];
                if (v > mx) mx = v;
            }
            float sum = 0.0f;
            for (int64_t j = 0; j < as; j++) {
                int64_t idx = i * as * inner + j * inner + k;
                out[idx] = expf(out[idx] - mx);
                sum += out[idx];
            }
            for (int64_t j = 0; j < as; j++) out[i * as * inner + j * inner + k] /= sum;
        }
    return TLO_OK;
}

/* tl_cpu_tensor_new_causal_mask (crates/tl_cpu/src/ffi.rs:3184-3196): [size, size], -inf
 * strictly above the diagonal, 0 elsewhere. */
void tlo_causal_mask(int64_t size, float* out) {
    for (int64_t i = 0; i < size; i++)
        for (int64_t j = 0; j < size; j++) out[i * size + j] = j > i ? -INFINITY : 0.0f;
}

/* CpuTensor::repeat_interleave_impl (crates/tl_cpu/src/tensor.rs:1178-1200). */
int tlo_repeat_interleave(const float* x, const int64_t* shape, int rank, int64_t repeats,
                          int axis, float* out) {
    if (axis < 0 || axis >= rank) return TLO_ERR_SHAPE;
    int64_t outer = 1, inner = 1, as = shape[axis], o = 0;
    for (int d = 0; d < axis; d++) outer *= shape[d];
    for (int d = axis + 1; d < rank; d++) inner *= shape[d];
    for (int64_t i = 0; i < outer; i++)
        for (int64_t j = 0; j < as; j++)
            for (int64_t r = 0; r < repeats; r++)
                for (int64_t k = 0; k < inner; k++) out[o++] = x[i * as * inner + j * inner + k];
    return TLO_OK;
}

/* CpuTensor::cat_impl for two tensors (crates/tl_cpu/src/tensor.rs:1021-1063). */
int tlo_cat(const float* a, const int64_t* ashape, const float* b, const int64_t* bshape,
            int rank, int axis, float* out) {
    if (axis < 0 || axis >= rank) return TLO_ERR_SHAPE;
    for (int d = 0; d < rank; d++)
        if (d != axis && ashape[d] != bshape[d]) return TLO_ERR_SHAPE;
    int64_t outer = 1, inner = 1, o = 0;
    for (int d = 0; d < axis; d++) outer *= ashape[d];
    for (int d = axis + 1; d < rank; d++) inner *= ashape[d];
    for (int64_t i = 0; i < outer; i++) {
        int64_t n = ashape[axis] * inner;
        memcpy(out + o, a + i * n, sizeof(float) * (size_t)n);
        o += n;
        n = bshape[axis] * inner;
        memcpy(out + o, b + i * n, sizeof(float) * (size_t)n);
        o += n;
    }
    return TLO_OK;
}

/* CpuTensor::narrow_impl / slice_impl (crates/tl_cpu/src/tensor.rs:989-1015). */
int tlo_narrow(const float* x, const int64_t* shape, int rank, int axis, int64_t start,
               int64_t len, float* out) {
    if (axis < 0 || axis >= rank) return TLO_ERR_SHAPE;
    if (start + len > shape[axis]) return TLO_ERR_SHAPE;
    int64_t outer = 1, inner = 1, as = shape[axis], o = 0;
    for (int d = 0; d < axis; d++) outer *= shape[d];
    for (int d = axis + 1; d < rank; d++) inner *= shape[d];
    for (int64_t i = 0; i < outer; i++)
        for (int64_t j = start; j < start + len; j++)
            for (int64_t k = 0; k < inner; k++) out[o++] = x[i * as * inner + j * inner + k];
    return TLO_OK;
}

/* CpuTensor::embedding_impl (crates/tl_cpu/src/tensor.rs:1094-1112): ids are f32 cast to
 * i64 (truncation); an id outside [0, vocab) is IndexOutOfBounds. */
int tlo_embedding(const float* table, int64_t vocab, int64_t dim, const float* ids, int64_t n,
                  float* out) {
    for (int64_t t = 0; t < n; t++) {
        int64_t id = (int64_t)ids[t];
        if (id < 0 || id >= vocab) return TLO_ERR_INDEX;
        memcpy(out + t * dim, table + id * dim, sizeof(float) * (size_t)dim);
    }
    return TLO_OK;
}

/* Greedy choice of CpuTensor::sample_impl with temp <= 0 (crates/tl_cpu/src/tensor.rs:
 * 1633-1637) and argmax_all_impl (tensor.rs:841-846): Iterator::max_by over partial_cmp
 * keeps the running best only when it compares Greater, so the LAST of equal maxima wins
 * and a NaN (compares Equal) moves the choice forward. */
int64_t tlo_argmax_last(const float* x, int64_t n) {
    if (n <= 0) return 0;
    int64_t best = 0;
    for (int64_t i = 1; i < n; i++)
        if (!(x[best] > x[i])) best = i;
    return best;
}

/* sort_by(|&a, &b| probs[b].partial_cmp(&probs[a]).unwrap_or(Equal)) of tensor.rs:1649-1650:
 * a stable merge sort of the indices by descending prob; an element moves ahead of an
 * earlier one only when it compares greater (a NaN compares Equal and keeps its place). */
static void sample_sort(int64_t* idx, int64_t* tmp, int64_t n, const float* pr) {
    for (int64_t w = 1; w < n; w *= 2) {
        for (int64_t lo = 0; lo < n; lo += 2 * w) {
            int64_t mid = lo + w < n ? lo + w : n, hi = lo + 2 * w < n ? lo + 2 * w : n;
            int64_t a = lo, b = mid, o = lo;
            while (a < mid && b < hi) tmp[o++] = pr[idx[a]] < pr[idx[b]] ? idx[b++] : idx[a++];
            while (a < mid) tmp[o++] = idx[a++];
            while (b < hi) tmp[o++] = idx[b++];
        }
        memcpy(idx, tmp, sizeof(int64_t) * (size_t)n);
    }
}

/* CpuTensor::sample_impl (crates/tl_cpu/src/tensor.rs:1626-1680) with rng.gen::<f64>() given
 * as u (tensor.rs:1663-1666):
 *   temp <= 0: the greedy argmax (1633-1638, tlo_argmax_last; a NaN temp is not <= 0);
 *   probs = x / temp (1642), max by the fold `if a > b {a} else {b}` from -inf (1644),
 *   sum_exp a left fold of expf(p - max) (1645), probs = expf(p - max) / sum_exp (1646);
 *   indices sorted by descending prob, stable (1649-1650);
 *   cum_prob summed in that order until it exceeds top_p: cutoff (1652-1660), else the last;
 *   r = (f32)u * cutoff_prob (1662-1666); the first index up to the cutoff whose running sum
 *   reaches r, indices[0] when none does (1667-1677).
 * Returns -1 for an empty input (the reference's InternalError). */
int64_t tlo_sample(const float* x, int64_t n, float temp, float top_p, double u) {
    if (n <= 0) return -1;
    if (temp <= 0.0f) return tlo_argmax_last(x, n);
    float* p = (float*)malloc(sizeof(float) * (size_t)n);
    int64_t* idx = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
    int64_t* tmp = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
    float mx = -INFINITY, se = 0.0f;
    for (int64_t i = 0; i < n; i++) p[i] = x[i] / temp;
    for (int64_t i = 0; i < n; i++) mx = mx > p[i] ? mx : p[i];
    for (int64_t i = 0; i < n; i++) se += expf(p[i] - mx);
    for (int64_t i = 0; i < n; i++) p[i] = expf(p[i] - mx) / se;
    for (int64_t i = 0; i < n; i++) idx[i] = i;
    sample_sort(idx, tmp, n, p);
    float cum = 0.0f;
    int64_t cutoff = n - 1;
    for (int64_t i = 0; i < n; i++) {
        cum += p[idx[i]];
        if (cum > top_p) {
            cutoff = i;
            break;
        }
    }
    const float r = (float)u * cum;
    float acc = 0.0f;
    int64_t sel = idx[0];
    for (int64_t i = 0; i <= cutoff; i++) {
        acc += p[idx[i]];
        if (acc >= r) {
            sel = idx[i];
            break;
        }
    }
    free(p);
    free(idx);
    free(tmp);
    return sel;
}

/* CpuDevice::tensor_repetition_penalty (crates/tl_cpu/src/device_impl.rs:967-1001): the
 * distinct token ids below vocab (f32 cast to usize) get val / p when val > 0, else val * p,
 * in every row of the logits. */
void tlo_repetition_penalty(const float* logits, int64_t rows, int64_t vocab, const float* tokens,
                            int64_t ntok, double penalty, float* out) {
    float p = (float)penalty;
    memcpy(out, logits, sizeof(float) * (size_t)(rows * vocab));
    unsigned char* seen = (unsigned char*)calloc((size_t)vocab, 1);
    for (int64_t t = 0; t < ntok; t++) {
        float f = tokens[t];
        /* Rust `f as usize` saturates: NaN and negatives give 0, huge values usize::MAX */
        uint64_t id = !(f >= 0.0f) ? 0 : (f >= 18446744073709551615.0f ? UINT64_MAX : (uint64_t)f);
        if (id < (uint64_t)vocab) seen[id] = 1;
    }
    for (int64_t r = 0; r < rows; r++)
        for (int64_t i = 0; i < vocab; i++) {
            if (!seen[i]) continue;
            float v = out[r * vocab + i];
            out[r * vocab + i] = v > 0.0f ? v / p : v * p;
        }
    free(seen);
}

/* CpuDevice::tensor_scaled_dot_product_attention (crates/tl_cpu/src/device_impl.rs:775-872):
 * for every (batch, head) slice, scores[i][j] = (sum_d q[i][d] k[j][d]) * (1 / sqrt(d_k)),
 * the sum from 0 left to right (scale at 800, scores 811-823); where a mask is given, a score
 * whose flat index i * seq_k + j lies inside the mask and whose mask value == 0.0 becomes -1e9
 * (825-834; every other mask value leaves the score as it is, and the same [seq_q, seq_k]
 * mask serves every slice); per row max by fold(-inf, f32::max), e = exp(s - max) summed left
 * to right, each e divided by the sum (835-849); out[i][d] = sum_l p[i][l] v[l][d] (850-861).
 * K and V hold the same (batch, head) slices as Q.  A row with seq_k = 0 gives zeros. */
void tlo_sdpa(const float* q, const float* k, const float* v, const float* mask, int64_t mask_len,
              int64_t slices, int64_t seq_q, int64_t seq_k, int64_t d_k, int64_t d_v, float* out) {
    const float scale = 1.0f / sqrtf((float)d_k);
    float* scores = (float*)malloc(sizeof(float) * (size_t)(seq_q * seq_k > 0 ? seq_q * seq_k : 1));
    for (int64_t bh = 0; bh < slices; bh++) {
        const float* Q = q + bh * seq_q * d_k;
        const float* K = k + bh * seq_k * d_k;
        const float* V = v + bh * seq_k * d_v;
        for (int64_t i = 0; i < seq_q; i++)
            for (int64_t j = 0; j < seq_k; j++) {
                float s = 0.0f;
                for (int64_t d = 0; d < d_k; d++) s += Q[i * d_k + d] * K[j * d_k + d];
                scores[i * seq_k + j] = s * scale;
            }
        if (mask)
            for (int64_t i = 0; i < seq_q; i++)
                for (int64_t j = 0; j < seq_k; j++)
                    if (mask_len > i * seq_k + j && mask[i * seq_k + j] == 0.0f) scores[i * seq_k + j] = -1e9f;
        for (int64_t i = 0; i < seq_q; i++) {
            float mx = -INFINITY;
            for (int64_t j = 0; j < seq_k; j++) mx = fmaxf(mx, scores[i * seq_k + j]);
            float sum = 0.0f;
            for (int64_t j = 0; j < seq_k; j++) {
                scores[i * seq_k + j] = expf(scores[i * seq_k + j] - mx);
                sum += scores[i * seq_k + j];
            }
            for (int64_t j = 0; j < seq_k; j++) scores[i * seq_k + j] /= sum;
        }
        float* O = out + bh * seq_q * d_v;
        for (int64_t i = 0; i < seq_q; i++)
            for (int64_t j = 0; j < d_v; j++) {
                float s = 0.0f;
                for (int64_t l = 0; l < seq_k; l++) s += scores[i * seq_k + l] * V[l * d_v + j];
                O[i * d_v + j] = s;
            }
    }
    free(scores);
}
