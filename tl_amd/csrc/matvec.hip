// Fused dequant x matvec for decode: y[m, n] = sum_k x[m, k] * W[n, k] with W resident as
// Q4_0 / Q8_0 (qs[n][nb][16|32], d[n][nb] f16), m in {1, 2} per launch.
//
// Layout of the work: a workgroup is 4 wavefronts and owns 4R consecutive rows (R per
// wavefront).  Lane l of a wavefront walks blocks l, l+64, ... of its R rows, so a load
// instruction covers 64 consecutive 16-byte quant blocks of one row (1 KiB contiguous).
// The activation row(s) are staged once per workgroup in LDS (coalesced 16-byte loads, block
// stride padded to 36 floats so the lanes of a ds_read_b128 hit distinct banks) and reused
// by all 4R rows: the weight stream is the only HBM traffic of the main loop.  The quant
// loads of the next block column are issued before the current one is consumed.
//
// Per block the lane forms d * (sum_j x_j q_j - 8 sum_j x_j) (Q4_0; Q8_0 uses q ^ 0x80 and
// 128), one byte->float conversion and one FMA per weight, f32 throughout.
//
// Prologue options:  NORM  x := (x / sqrt(mean(x^2) + eps)) * w   (the RMSNorm that precedes
//                          every projection in the chatbot, ffi.rs:2444-2486 + mul_impl)
//                    EMBED x := embedding row of the token id held in device memory
//                          (tensor.rs:1094-1112), also written out as the residual stream
// Epilogues:  EPI_PLAIN   y = v
//             EPI_RES     y = residual + v             (chatbot.tl:109, 111)
//             EPI_GLU     rows (2i, 2i+1) = (gate_i, up_i): y_i = silu(g) * u (chatbot.tl:33-38)
//             EPI_ROPE_KV rows of [q | k | v]: q, k pairs rotated by the table row of the
//                         device position (ffi.rs:2655-2681), q written out, k and v appended
//                         to the KV cache at that position (chatbot.tl:56-69)
//             EPI_ARGMAX  logits written, optional repetition penalty (device_impl.rs:967-1001),
//                         per-workgroup greedy candidates; a one-workgroup kernel reduces
//                         them (last maximum, tensor.rs:1633-1637), records the token and
//                         advances the decode position.
#include "internal.h"

namespace tlhip {

constexpr int XPAD = 36;  // floats per staged 32-float block

template <int QT>
struct QB_;
template <>
struct QB_<TL_HIP_GGML_Q4_0> {
    static constexpr int v = 16;
};
template <>
struct QB_<TL_HIP_GGML_Q8_0> {
    static constexpr int v = 32;
};

__device__ __forceinline__ float dot4b(uint32_t q, const float* x) {
    float s = x[0] * (float)(q & 0xFF);
    s = fmaf(x[1], (float)((q >> 8) & 0xFF), s);
    s = fmaf(x[2], (float)((q >> 16) & 0xFF), s);
    s = fmaf(x[3], (float)(q >> 24), s);
    return s;
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// Sum over the 64 lanes of a wavefront: DPP within rows of 16 (quad_perm 1-0-3-2 and
// 2-3-0-1, half-row and row mirrors -- VALU ops, no LDS traffic), then two cross-row
// exchanges through ds_bpermute.  Every lane receives the total.
__device__ __forceinline__ float wsum(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

template <int QT, int R>
__device__ __forceinline__ void load_rows(const MvArgs& a, int64_t row0, int64_t b,
                                          uint4 (&w)[R][QB_<QT>::v / 16], float (&dd)[R]) {
    constexpr int QB = QB_<QT>::v;
#pragma unroll
    for (int r = 0; r < R; r++) {
        int64_t row = row0 + r < a.n ? row0 + r : a.n - 1;  // clamp: loads stay in bounds
        const uint4* p = reinterpret_cast<const uint4*>(a.qs + (row * a.nb + b) * QB);
#pragma unroll
        for (int i = 0; i < QB / 16; i++) w[r][i] = p[i];
        dd[r] = __half2float(a.d[row * a.nb + b]);
    }
}

template <int QT, int R, int M, int EPI, bool NORM, bool EMBED>
__global__ __launch_bounds__(256) void k_mv(MvArgs a) {
    constexpr int QB = QB_<QT>::v;
    extern __shared__ float xs[];  // [M][nb][XPAD]
    __shared__ float ys[M][4 * R];
    __shared__ float red[M][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t nb = a.nb, k = a.k, n = a.n;
    const int64_t wg_row0 = (int64_t)blockIdx.x * 4 * R;
    const int64_t row0 = wg_row0 + wave * R;

    // (1) first block column of quant data in flight before x is staged
    uint4 w[R][QB / 16];
    float dd[R];
    if (lane < nb) load_rows<QT, R>(a, row0, lane, w, dd);

    // (2) stage x (optionally gathered and normalised) into LDS
    const int64_t k4 = k >> 2;
    const float* xsrc = EMBED ? a.x + (int64_t)(*a.embed_id) * k : a.x;
#pragma unroll
    for (int m = 0; m < M; m++) {
        const float4* xm = reinterpret_cast<const float4*>(xsrc + m * k);
        if constexpr (NORM) {
            float ss = 0.f;
            for (int64_t e = tid; e < k4; e += 256) {
                float4 v = xm[e];
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
            ss = wsum(ss);
            if (lane == 0) red[m][wave] = ss;
        }
    }
    if constexpr (NORM) __syncthreads();
#pragma unroll
    for (int m = 0; m < M; m++) {
        const float4* xm = reinterpret_cast<const float4*>(xsrc + m * k);
        float rms = 1.f;
        if constexpr (NORM) {
            float ss = (red[m][0] + red[m][1]) + (red[m][2] + red[m][3]);
            rms = sqrtf(ss / (float)k + a.eps);
        }
        for (int64_t e = tid; e < k4; e += 256) {
            float4 v = xm[e];
            if constexpr (EMBED) {
                if (blockIdx.x == 0 && a.x_out) reinterpret_cast<float4*>(a.x_out + m * k)[e] = v;
            }
            if constexpr (NORM) {
                float4 g = reinterpret_cast<const float4*>(a.norm_w)[e];
                v.x = (v.x / rms) * g.x;
                v.y = (v.y / rms) * g.y;
                v.z = (v.z / rms) * g.z;
                v.w = (v.w / rms) * g.w;
            }
            const int64_t b = e >> 3, c = e & 7;
            *reinterpret_cast<float4*>(xs + (m * nb + b) * XPAD + c * 4) = v;
        }
    }
    __syncthreads();

    // (3) main loop over this lane's block columns
    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[m][r] = 0.f;
    for (int64_t b = lane; b < nb; b += 64) {
        uint4 wn[R][QB / 16];
        float dn[R];
        const bool more = b + 64 < nb;
        if (more) load_rows<QT, R>(a, row0, b + 64, wn, dn);
#pragma unroll
        for (int m = 0; m < M; m++) {
            float xv[32];
            const float* xb = xs + (m * nb + b) * XPAD;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float4 t = *reinterpret_cast<const float4*>(xb + 4 * i);
                xv[4 * i] = t.x;
                xv[4 * i + 1] = t.y;
                xv[4 * i + 2] = t.z;
                xv[4 * i + 3] = t.w;
            }
            float sx0 = 0.f, sx1 = 0.f;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                sx0 += xv[j];
                sx1 += xv[16 + j];
            }
            const float sx = sx0 + sx1;
#pragma unroll
            for (int r = 0; r < R; r++) {
                float s0 = 0.f, s1 = 0.f;
                if constexpr (QT == TL_HIP_GGML_Q4_0) {
                    const uint32_t q[4] = {w[r][0].x, w[r][0].y, w[r][0].z, w[r][0].w};
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        s0 += dot4b(q[c] & 0x0F0F0F0Fu, xv + 4 * c);
                        s1 += dot4b((q[c] >> 4) & 0x0F0F0F0Fu, xv + 16 + 4 * c);
                    }
                    acc[m][r] = fmaf(dd[r], (s0 + s1) - 8.f * sx, acc[m][r]);
                } else {
                    const uint32_t q[8] = {w[r][0].x, w[r][0].y, w[r][0].z, w[r][0].w,
                                           w[r][1].x, w[r][1].y, w[r][1].z, w[r][1].w};
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        s0 += dot4b(q[c] ^ 0x80808080u, xv + 4 * c);
                        s1 += dot4b(q[4 + c] ^ 0x80808080u, xv + 16 + 4 * c);
                    }
                    acc[m][r] = fmaf(dd[r], (s0 + s1) - 128.f * sx, acc[m][r]);
                }
            }
        }
        if (more) {
#pragma unroll
            for (int r = 0; r < R; r++) {
#pragma unroll
                for (int i = 0; i < QB / 16; i++) w[r][i] = wn[r][i];
                dd[r] = dn[r];
            }
        }
    }

    // (4) lane partials -> row sums in LDS
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            float v = wsum(acc[m][r]);
            if (lane == 0) ys[m][wave * R + r] = v;
        }
    __syncthreads();

    // (5) epilogue
    if constexpr (EPI == EPI_PLAIN || EPI == EPI_RES) {
        for (int t = tid; t < M * 4 * R; t += 256) {
            const int m = t / (4 * R), rl = t % (4 * R);
            const int64_t row = wg_row0 + rl;
            if (row < n) {
                float v = ys[m][rl];
                if constexpr (EPI == EPI_RES) v = a.res[m * n + row] + v;
                a.y[m * n + row] = v;
            }
        }
    } else if constexpr (EPI == EPI_GLU) {
        const int64_t half_n = n / 2;
        for (int t = tid; t < M * 2 * R; t += 256) {
            const int m = t / (2 * R), p = t % (2 * R);
            const int64_t i = wg_row0 / 2 + p;
            if (i < half_n) {
                const float g = ys[m][2 * p], u = ys[m][2 * p + 1];
                a.y[m * half_n + i] = (g * (1.0f / (1.0f + expf(-g)))) * u;
            }
        }
    } else if constexpr (EPI == EPI_ROPE_KV) {
        const int64_t pos = *a.pos;
        for (int t = tid; t < 2 * R; t += 256) {
            const int64_t r0 = wg_row0 + 2 * t;
            if (r0 >= n) continue;
            const float v0 = ys[0][2 * t], v1 = ys[0][2 * t + 1];
            if (r0 < a.q_rows + a.kv_rows) {
                const bool isq = r0 < a.q_rows;
                const int64_t rr = isq ? r0 : r0 - a.q_rows;
                const int64_t i = rr % a.hd;
                const float c = a.cos_t[pos * a.hd + i], s = a.sin_t[pos * a.hd + i];
                const float o0 = v0 * c - v1 * s, o1 = v0 * s + v1 * c;
                if (isq) {
                    a.q_out[r0] = o0;
                    a.q_out[r0 + 1] = o1;
                } else {
                    const int64_t off = ((rr / a.hd) * a.max_seq + pos) * a.hd + i;
                    if (a.kv_f16) {
                        reinterpret_cast<__half*>(a.kc)[off] = __float2half(o0);
                        reinterpret_cast<__half*>(a.kc)[off + 1] = __float2half(o1);
                    } else {
                        reinterpret_cast<float*>(a.kc)[off] = o0;
                        reinterpret_cast<float*>(a.kc)[off + 1] = o1;
                    }
                }
            } else {
                const int64_t rr = r0 - a.q_rows - a.kv_rows, i = rr % a.hd;
                const int64_t off = ((rr / a.hd) * a.max_seq + pos) * a.hd + i;
                if (a.kv_f16) {
                    reinterpret_cast<__half*>(a.vc)[off] = __float2half(v0);
                    reinterpret_cast<__half*>(a.vc)[off + 1] = __float2half(v1);
                } else {
                    reinterpret_cast<float*>(a.vc)[off] = v0;
                    reinterpret_cast<float*>(a.vc)[off + 1] = v1;
                }
            }
        }
    } else if constexpr (EPI == EPI_ARGMAX) {
        // logits, penalised logits, then this workgroup's greedy candidate (the left fold of
        // tensor.rs:1633-1637 over its rows: keep the best only when strictly greater)
        if (tid < 4 * R) {
            const int64_t row = wg_row0 + tid;
            if (row < n) {
                float v = ys[0][tid];
                a.y[row] = v;
                if (a.seen && a.seen[row]) v = v > 0.0f ? v / a.penalty : v * a.penalty;
                a.plogits[row] = v;
                ys[0][tid] = v;
            }
        }
        __syncthreads();
        if (tid == 0) {
            int cnt = (int)((n - wg_row0) < 4 * R ? (n - wg_row0) : 4 * R);
            float bv = ys[0][0];
            int bi = 0, nan = bv != bv;
            for (int i = 1; i < cnt; i++) {
                float v = ys[0][i];
                nan |= v != v;
                if (!(bv > v)) {
                    bv = v;
                    bi = i;
                }
            }
            a.part_v[blockIdx.x] = bv;
            a.part_i[blockIdx.x] = (int32_t)(wg_row0 + bi);
            a.part_nan[blockIdx.x] = nan;
        }
    }
}

// Greedy token from the per-workgroup candidates of an EPI_ARGMAX matvec (one workgroup):
// the candidates are folded in workgroup order; for NaN-free input the (greater value, then
// larger index) reduction equals the left fold of tensor.rs:1633-1637, otherwise thread 0
// replays that fold over the penalised logits.  Then the decode-step bookkeeping: token
// recorded, penalty mask updated, position advanced.
__global__ __launch_bounds__(256) void k_argmax_finish(MvArgs a, int nwg) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -INFINITY;
    int bi = -1, nan = 0;
    for (int i = tid; i < nwg; i += 256) {
        const float v = a.part_v[i];
        const int ix = a.part_i[i];
        nan |= a.part_nan[i];
        if (bi < 0 || !(bv > v)) {
            bv = v;
            bi = ix;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
            bv = ov;
            bi = oi;
        }
        nan |= __shfl_xor(nan, off, 64);
    }
    __shared__ float fv[4];
    __shared__ int fi[4], fn[4];
    if (lane == 0) {
        fv[wave] = bv;
        fi[wave] = bi;
        fn[wave] = nan;
    }
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < 4; i++) {
            if (fi[i] >= 0 && (bi < 0 || fv[i] > bv || (fv[i] == bv && fi[i] > bi))) {
                bv = fv[i];
                bi = fi[i];
            }
            nan |= fn[i];
        }
        if (nan) {  // non-associative case: replay the sequential fold
            bi = 0;
            for (int64_t i = 1; i < a.n; i++)
                if (!(a.plogits[bi] > a.plogits[i])) bi = (int)i;
        }
        *a.tok_out = bi;
        if (a.out_ids) {
            const int s = *a.step;
            if (s < a.max_out) a.out_ids[s] = bi;
            *a.step = s + 1;
        }
        if (a.seen_out) a.seen_out[bi] = 1;
        if (a.pos_inc) *a.pos_inc += 1;
    }
}

// ---------------------------------------------------------------- dispatch --------------
static int pick_r(int64_t n) {
    // about 512 - 1024 workgroups of 4R rows
    if (n >= 4 * 8 * 1024) return 8;
    if (n >= 4 * 4 * 1024) return 4;
    if (n >= 4 * 2 * 512) return 2;
    return 1;
}

template <int QT, int R, int M, int EPI, bool NORM, bool EMBED>
static int run(const MvArgs& a, hipStream_t s) {
    const size_t lds = (size_t)M * a.nb * XPAD * 4;
    auto kern = k_mv<QT, R, M, EPI, NORM, EMBED>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(LDS)");
    }
    const unsigned grid = (unsigned)cdiv(a.n, 4 * R);
    kern<<<grid, 256, lds, s>>>(a);
    if constexpr (EPI == EPI_ARGMAX) k_argmax_finish<<<1, 256, 0, s>>>(a, (int)grid);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "matvec launch");
}

template <int QT, int M, int EPI, bool NORM, bool EMBED>
static int run_r(const MvArgs& a, int R, hipStream_t s) {
    switch (R) {
        case 8: return run<QT, 8, M, EPI, NORM, EMBED>(a, s);
        case 4: return run<QT, 4, M, EPI, NORM, EMBED>(a, s);
        case 2: return run<QT, 2, M, EPI, NORM, EMBED>(a, s);
        default: return run<QT, 1, M, EPI, NORM, EMBED>(a, s);
    }
}

template <int QT>
static int run_t(const MvArgs& a, int m, int epi, bool norm, bool embed, int R, hipStream_t s) {
    if (m == 2) {
        if (epi == EPI_RES) return run_r<QT, 2, EPI_RES, false, false>(a, R, s);
        return run_r<QT, 2, EPI_PLAIN, false, false>(a, R, s);
    }
    switch (epi) {
        case EPI_RES: return run_r<QT, 1, EPI_RES, false, false>(a, R, s);
        case EPI_GLU:
            return norm ? run_r<QT, 1, EPI_GLU, true, false>(a, R, s) : run_r<QT, 1, EPI_GLU, false, false>(a, R, s);
        case EPI_ROPE_KV:
            if (embed) return run_r<QT, 1, EPI_ROPE_KV, true, true>(a, R, s);
            return norm ? run_r<QT, 1, EPI_ROPE_KV, true, false>(a, R, s)
                        : run_r<QT, 1, EPI_ROPE_KV, false, false>(a, R, s);
        case EPI_ARGMAX:
            return norm ? run_r<QT, 1, EPI_ARGMAX, true, false>(a, R, s) : run_r<QT, 1, EPI_ARGMAX, false, false>(a, R, s);
        default:
            return norm ? run_r<QT, 1, EPI_PLAIN, true, false>(a, R, s) : run_r<QT, 1, EPI_PLAIN, false, false>(a, R, s);
    }
}

// Checks and launches one fused matvec.  m is 1 or 2 (2 only with EPI_PLAIN / EPI_RES
// and no prologue).
int launch_mv(const QWeight* w, MvArgs a, int m, int epi, bool norm, bool embed, hipStream_t s) {
    a.qs = w->qs;
    a.d = w->d;
    a.n = w->n;
    a.k = w->k;
    a.nb = w->nb;
    if (m < 1 || m > 2 || (m == 2 && (norm || embed || (epi != EPI_PLAIN && epi != EPI_RES)))) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: unsupported matvec variant (m=%d, epilogue %d)", m, epi);
        return TL_HIP_ERR_ARG;
    }
    if ((reinterpret_cast<uintptr_t>(a.x) & 15) != 0 || (norm && (reinterpret_cast<uintptr_t>(a.norm_w) & 15))) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: x and the norm weight must be 16-byte aligned");
        return TL_HIP_ERR_ARG;
    }
    if ((size_t)m * a.nb * XPAD * 4 > 160 * 1024) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: k = %lld too large for the LDS-staged matvec", (long long)a.k);
        return TL_HIP_ERR_ARG;
    }
    int R = pick_r(a.n);
    if ((epi == EPI_GLU || epi == EPI_ROPE_KV) && (a.n % 2)) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: paired epilogue needs an even row count");
        return TL_HIP_ERR_SHAPE;
    }
    if (w->ggml_type == TL_HIP_GGML_Q4_0) return run_t<TL_HIP_GGML_Q4_0>(a, m, epi, norm, embed, R, s);
    return run_t<TL_HIP_GGML_Q8_0>(a, m, epi, norm, embed, R, s);
}

int mv_partials(int64_t n) { return (int)cdiv(n, 4 * pick_r(n)); }

int launch_quant_matvec(const QWeight* w, const float* x, float* y, int64_t m, hipStream_t s,
                        const float* residual) {
    if (m < 1 || m > 4) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: matvec supports 1..4 rows, got %lld", (long long)m);
        return TL_HIP_ERR_ARG;
    }
    // m = 3 and 4 run as launches of up to two activation rows each
    for (int64_t m0 = 0; m0 < m; m0 += 2) {
        const int mm = (int)(m - m0 >= 2 ? 2 : 1);
        MvArgs a = {};
        a.x = x + m0 * w->k;
        a.y = y + m0 * w->n;
        a.res = residual ? residual + m0 * w->n : nullptr;
        int rc = launch_mv(w, a, mm, residual ? EPI_RES : EPI_PLAIN, false, false, s);
        if (rc) return rc;
    }
    return TL_HIP_OK;
}

}  // namespace tlhip
