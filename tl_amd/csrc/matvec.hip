// Fused dequant x matvec for decode: y[m, n] = sum_k x[m, k] * W[n, k] with W resident as
// Q4_0 / Q8_0 / Q4_K / Q6_K in 32-weight units (qs[n][nb][16|32] plus per-type scale data,
// layout at struct QWeight), m in {1, 2} per launch.
//
// Decode matvecs are small (2 - 40 MB of weights, a few microseconds each), so the kernel is
// built for memory-level parallelism: every thread issues all of its loads before it does
// any arithmetic, and the whole matrix is in flight within the first few hundred cycles.
//
// Layout of the work: a workgroup owns RW consecutive rows and S row subsets of TC threads
// (TC = the block count nb rounded up to wavefronts, at most 256).  Thread (s, t) owns block
// columns t, t + TC, ... (BT per pass) of the RW / S rows s, s + S, ...:
//   * one load instruction covers TC consecutive 16-byte quant blocks of one row;
//   * the activations are staged once per workgroup in LDS (coalesced loads, 36-float pitch
//     per 32-float block so that lane-consecutive blocks read distinct banks); each thread
//     reads its blocks from there and reuses them for its rows;
//   * the K dimension is split across the wavefronts of a subset.  Row sums are formed by a
//     transpose-reduce inside each wavefront (each exchange step halves the number of
//     values a lane carries: N - 1 exchanges for N values instead of 6 per value) and one
//     LDS pass across the wavefronts.
//   * residual, RoPE table entries and penalty flags for the epilogue are requested right
//     after the weight loads, so no memory round trip is left after the reduction.
//
// Per unit the thread forms d * (sum_j x_j q_j - 8 sum_j x_j) (Q4_0; Q8_0 uses q ^ 0x80 and
// 128), f32 throughout: one FMA per weight, plus one byte->float conversion per weight (Q8_0,
// Q6_K) or per two weights (the 4-bit types, through the fp8 pair conversion).  The K-quants use
// the same dot products with their own scale terms: Q4_K (d sc) sum x q - (dmin m) sum x
// with (sc, m) decoded from the super-block header; Q6_K rebuilds each 6-bit value as one
// byte (low nibble | high bits << 4) and forms sum over its two 16-weight halves of
// (d sc_h) (sum x q - 32 sum x).
//
// Prologue options:  NORM  x := (x / sqrt(mean(x^2) + eps)) * w   (the RMSNorm that precedes
//                          every projection in the chatbot, ffi.rs:2444-2486 + mul_impl),
//                          applied as (sum_j W_j x_j w_j) / sqrt(mean(x^2) + eps): the
//                          squares are summed alongside the dot products and the division
//                          is done once per row after the reduction
//                    EMBED x := embedding row of the token id held in device memory
//                          (tensor.rs:1094-1112), also written out as the residual stream
// Epilogues:  EPI_PLAIN   y = v
//             EPI_RES     y = residual + v             (chatbot.tl:109, 111)
//             EPI_GLU     rows (2i, 2i+1) = (gate_i, up_i): y_i = silu(g) * u (chatbot.tl:33-38)
//             EPI_ROPE_KV rows of [q | k | v] (this weight's rows start at row_off of it):
//                         q, k pairs rotated by the table row of the device position
//                         (ffi.rs:2655-2681), q written out, k and v appended to the KV cache
//                         at that position (chatbot.tl:56-69)
//             EPI_ARGMAX  logits written, optional repetition penalty (device_impl.rs:967-1001),
//                         per-workgroup greedy candidates; a one-workgroup kernel reduces
//                         them (last maximum, tensor.rs:1633-1637), records the token and
//                         advances the decode position.
#include "internal.h"

namespace tlhip {

typedef float float2v __attribute__((ext_vector_type(2)));

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
template <>
struct QB_<TL_HIP_GGML_Q4_K> {
    static constexpr int v = 16;
};
template <>
struct QB_<TL_HIP_GGML_Q6_K> {
    static constexpr int v = 16;
};

// Q4_K d * scale and dmin * min of sub-block j from its resident super-block header
// (q4k_hdr_sm; QTensor::get_scale_min_k4, quantized.rs:405-415); both products exact in f32.
__device__ __forceinline__ void k4_sm(const uint4& hd, int j, float* du, float* mu) {
    uint32_t sc, mn;
    q4k_hdr_sm(hd, j, &sc, &mn);
    *du = __half2float(__ushort_as_half((uint16_t)(hd.x & 0xFFFF))) * (float)sc;
    *mu = __half2float(__ushort_as_half((uint16_t)(hd.x >> 16))) * (float)mn;
}

// acc + sum_j x[j] * byte_j(q): one v_cvt_f32_ubyteN and one FMA per byte.  The empty asm
// hides which bits of q are known to be zero (after a nibble mask); otherwise the byte
// extraction is narrowed to a 4-bit field extract plus a ubyte0 conversion per byte.
__device__ __forceinline__ float fma4b(uint32_t q, const float* x, float acc) {
    asm("" : "+v"(q));
    acc = fmaf(x[0], (float)(q & 0xFF), acc);
    acc = fmaf(x[1], (float)((q >> 8) & 0xFF), acc);
    acc = fmaf(x[2], (float)((q >> 16) & 0xFF), acc);
    acc = fmaf(x[3], (float)(q >> 24), acc);
    return acc;
}

// Lane exchange used by the reductions.  Each form is an involution that flips lane bit OFF
// within the group of lanes agreeing on the higher bits: the permlane swaps for 32 and 16,
// the DPP row mirror (xor 15), half-row mirror (xor 7) and quad permutations (xor 2, xor 1)
// below -- VALU ops, no LDS traffic.
template <int OFF>
__device__ __forceinline__ float xchg(float v) {
    if constexpr (OFF >= 16) return lane_xor_f32<OFF>(v);
    else if constexpr (OFF == 8) return dpp_f<0x140>(v);
    else if constexpr (OFF == 4) return dpp_f<0x141>(v);
    else if constexpr (OFF == 2) return dpp_f<0x4E>(v);
    else return dpp_f<0xB1>(v);
}

template <int OFF>
__device__ __forceinline__ float fold(float t) {
    if constexpr (OFF >= 16) t = lane_pair_sum<OFF>(t);  // t + partner, with no lane select
    else t += xchg<OFF>(t);
    if constexpr (OFF > 1) return fold<OFF / 2>(t);
    else return t;
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wsum(float v) { return fold<32>(v); }

// Transpose-reduce of N values per lane (N a power of two, 2..64): after the call lane l
// holds, in v[0], the wavefront sum of value l / (64 / N).  Step OFF exchanges half of the
// values with the partner across lane bit OFF and keeps the half selected by that bit.
template <int OFF, int H, int N>
__device__ __forceinline__ void halve(float (&v)[N], int lane) {
    if constexpr (OFF >= 16) {
        // one swap of (v[i], v[i + H]) leaves a lower lane (a_l, a_partner) and an upper lane
        // (b_partner, b_l): their sum is keep + the partner's send in either half
#pragma unroll
        for (int i = 0; i < H; i++) {
            uint32_t a = __builtin_bit_cast(uint32_t, v[i]), b = __builtin_bit_cast(uint32_t, v[i + H]);
            lane_swap<OFF>(a, b);
            v[i] = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
        }
    } else {
        const bool up = (lane & OFF) != 0;
#pragma unroll
        for (int i = 0; i < H; i++) {
            const float send = up ? v[i] : v[i + H];
            const float keep = up ? v[i + H] : v[i];
            v[i] = keep + xchg<OFF>(send);
        }
    }
    if constexpr (H > 1) halve<OFF / 2, H / 2, N>(v, lane);
}

template <int N>
__device__ __forceinline__ float xreduce(float (&v)[N], int lane) {
    if constexpr (N == 1) {
        return fold<32>(v[0]);
    } else {
        halve<32, N / 2, N>(v, lane);
        constexpr int G = 64 / N;  // lanes that share a value index
        if constexpr (G > 1) return fold<G / 2>(v[0]);
        else return v[0];
    }
}

constexpr int XPAD = 36;       // floats per staged 32-float block: lane-per-block LDS reads hit distinct banks
// float4 per thread staged ahead of the weight loads: k <= 8192 at 256 threads in one pass;
// with the RMSNorm prologue (norm weights staged too) k <= 4096, and k <= 2048 when a thread
// also holds eight rows' weights -- the register budget that keeps the wide decode grids
// (704 / 1000 workgroups) resident in one pass; longer rows stage the rest in a loop
constexpr int XR = 8, XR_NORM = 4, XR_NORM8 = 2;

// Launch shape: S = 1 << s_shift row subsets of tc threads each (tc a multiple of 64 and,
// when S > 1, a power of two 1 << tc_shift).
struct MvShape {
    int tc, tc_shift, s_shift;
    // one dword for the kernel argument list: tc (<= 256) | tc_shift << 16 | s_shift << 24
    __host__ __device__ uint32_t pack() const { return (uint32_t)tc | (uint32_t)tc_shift << 16 | (uint32_t)s_shift << 24; }
    __host__ __device__ static MvShape unpack(uint32_t v) {
        return MvShape{(int)(v & 0xffffu), (int)((v >> 16) & 0xffu), (int)(v >> 24)};
    }
};

// Thread (sub, tcol) owns block columns tcol + tc * (i + BT * pass) of rows
// row0 + sub + S * j, j < RWT.  Rows per workgroup RW = S * RWT.  Offsets are 32-bit
// (checked at launch: the quant array is below 2 GiB).
// The attention records of a head merged into x: o = sum_s f_s o_s / sum_s f_s l_s,
// f_s = exp2(m_s - max_s m_s) (scores in log2 units; an empty share has m = -inf, f = 0).
// Record (h, s) sits at rec + (h * ATTN_SHARES + s) * (hd + 4): [o (hd) | m | l | 0 | 0].
// Loading and merging are separate steps so the weight loads can be issued in between.
__device__ __forceinline__ void load_shares(const float* __restrict__ rec, uint32_t e, uint32_t hd,
                                            float4 (&o)[ATTN_SHARES], float2 (&st)[ATTN_SHARES]) {
    const uint32_t h = (4 * e) / hd, d = 4 * e - h * hd;
    const float* r = rec + (size_t)h * ATTN_SHARES * (hd + 4);
#pragma unroll
    for (int s = 0; s < ATTN_SHARES; s++) {
        o[s] = *reinterpret_cast<const float4*>(r + s * (hd + 4) + d);
        st[s] = *reinterpret_cast<const float2*>(r + s * (hd + 4) + hd);
    }
}

__device__ __forceinline__ float4 merge_shares(const float4 (&o)[ATTN_SHARES], const float2 (&st)[ATTN_SHARES]) {
    float mx = st[0].x;
#pragma unroll
    for (int s = 1; s < ATTN_SHARES; s++) mx = fmaxf(mx, st[s].x);
    float4 num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int s = 0; s < ATTN_SHARES; s++) {
        const float f = __builtin_amdgcn_exp2f(st[s].x - mx);
        den = fmaf(f, st[s].y, den);
        num.x = fmaf(f, o[s].x, num.x);
        num.y = fmaf(f, o[s].y, num.y);
        num.z = fmaf(f, o[s].z, num.z);
        num.w = fmaf(f, o[s].w, num.w);
    }
    const float inv = 1.0f / den;
    return float4{num.x * inv, num.y * inv, num.z * inv, num.w * inv};
}

// The arguments the first loads need come first, as scalars and pointers, so that they are
// preloaded into SGPRs at dispatch (kernel-argument preloading covers leading non-aggregate
// arguments, up to 14 dwords: 16 user SGPRs less the argument-buffer pointer): the weight stream (qs, the scale array w1 -- d, the Q4_K headers
// or the Q6_K high bits), the activations x, the auxiliary input of the prologue (aux: the
// RMSNorm weight, or the attention records that form x; aux2: the token id of EMBED or the
// position of EPI_ROPE_KV; aux_i: the records' head dimension), and the shape.  The rest
// travels in MvArgs; the compiler's scalar loads of those fields then overlap the weight
// stream instead of holding back its first loads.
// The body runs as workgroup `bid` of its weight (k_mv: blockIdx.x; k_mv_pair: the index
// within its segment).
template <int QT, int BT, int RWT, int M, int EPI, bool NORM, bool EMBED, bool MERGE>
__device__ __forceinline__ void mv_body(const uint8_t* __restrict__ qs_p, const void* __restrict__ w1_p,
                                        const float* __restrict__ x_p, const float* __restrict__ aux_p,
                                        const int32_t* __restrict__ aux2_p, uint32_t n_p, uint32_t nb_p,
                                        uint32_t shape_p, int aux_i, MvArgs& a, const uint32_t bid) {
    constexpr int QB = QB_<QT>::v, QW = QB / 16;  // 16-byte loads per block
    constexpr int N = M * RWT;
    constexpr int RWT_SHIFT = RWT == 1 ? 0 : RWT == 2 ? 1 : RWT == 4 ? 2 : RWT == 8 ? 3 : 4;
    static_assert(N <= 64 && (N & (N - 1)) == 0 && (1 << RWT_SHIFT) == RWT, "RWT, M * RWT: powers of two");
    a.qs = qs_p;
    a.x = x_p;
    a.n = n_p;
    a.nb = nb_p;
    a.k = (int64_t)nb_p * 32;
    if constexpr (QT == TL_HIP_GGML_Q4_K) a.hdr = static_cast<const uint8_t*>(w1_p);
    else if constexpr (QT == TL_HIP_GGML_Q6_K) a.qh = static_cast<const uint8_t*>(w1_p);
    else a.d = static_cast<const __half*>(w1_p);
    if constexpr (NORM) a.norm_w = aux_p;
    if constexpr (MERGE) {
        a.attn_rec = aux_p;
        a.attn_hd = aux_i;
    }
    if constexpr (EMBED) a.embed_id = aux2_p;
    else if constexpr (EPI == EPI_ROPE_KV) a.pos = aux2_p;
    const MvShape sh = MvShape::unpack(shape_p);
    // Q6_K's scale arrays are read with the first weight loads: fetched in one round of scalar
    // loads (left to the compiler, each would wait for the round before it)
    if constexpr (QT == TL_HIP_GGML_Q6_K) asm volatile("" : : "s"(a.sc), "s"(a.d));
    extern __shared__ float xs[];  // [M][nb][XPAD] staged activations (x * norm weight with NORM)
    __shared__ float red[8][N];
    __shared__ float ssq[8][M];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR
    const int TC = sh.tc, S = 1 << sh.s_shift, RW = RWT << sh.s_shift, rw_shift = RWT_SHIFT + sh.s_shift;
    const int tcol = sh.s_shift ? (tid & (TC - 1)) : tid;
    const int sub = sh.s_shift ? __builtin_amdgcn_readfirstlane(tid >> sh.tc_shift) : 0;  // TC >= 64: uniform
    const int wps = TC >> 6;  // wavefronts per row subset
    const uint32_t nb = (uint32_t)a.nb, k = (uint32_t)a.k, n = (uint32_t)a.n;
    const uint32_t row0 = bid * (uint32_t)RW;
    const uint32_t my_row0 = row0 + sub;

    // epilogue operands, requested right after the first loads
    float pre_res = 0.f, pre_c = 0.f, pre_s = 0.f;
    uint32_t pre_pos = 0;
    int pre_seen = 0;
    float acc[M][RWT];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int r = 0; r < RWT; r++) acc[m][r] = 0.f;

    constexpr bool K4 = QT == TL_HIP_GGML_Q4_K, K6 = QT == TL_HIP_GGML_Q6_K;
    constexpr bool NIB = QT == TL_HIP_GGML_Q4_0 || K4;  // 4-bit quants in Q4_0 nibble order
    uint32_t bc[BT];
    bool valid[BT];
    uint4 w[BT][RWT][QW];
    uint16_t dh[BT][RWT];           // Q4_0 / Q8_0 / Q6_K (super-block) scale, f16 bits
    uint4 kh[BT][K4 ? RWT : 1];     // Q4_K super-block header
    uint2 h6[BT][K6 ? RWT : 1];     // Q6_K high bits
    uint32_t s6[BT][K6 ? RWT : 1];  // Q6_K scale pair
    auto set_cols = [&](uint32_t base) {
#pragma unroll
        for (int i = 0; i < BT; i++) {
            const uint32_t b = base + (uint32_t)(tcol + i * TC);
            valid[i] = b < nb;
            bc[i] = valid[i] ? b : nb - 1;  // past the end: read the last column, scale 0
        }
    };
    // Scale data is kept as loaded and decoded in the math, so nothing before the staging
    // barrier waits for the weight stream.
    auto load_w = [&]() {
#pragma unroll
        for (int i = 0; i < BT; i++) {
#pragma unroll
            for (int r = 0; r < RWT; r++) {
                uint32_t row = my_row0 + (uint32_t)(S * r);
                row = row < n ? row : n - 1;
                const uint32_t blk = __umul24(row, nb) + bc[i];
                const uint4* p = reinterpret_cast<const uint4*>(a.qs + (size_t)blk * QB);
#pragma unroll
                for (int c = 0; c < QW; c++) w[i][r][c] = ld_stream(p + c);
                if constexpr (K4) {
                    kh[i][r] = reinterpret_cast<const uint4*>(a.hdr)[blk >> 3];
                } else if constexpr (K6) {
                    h6[i][r] = reinterpret_cast<const uint2*>(a.qh)[blk];
                    s6[i][r] = reinterpret_cast<const uint16_t*>(a.sc)[blk];
                    dh[i][r] = reinterpret_cast<const uint16_t*>(a.d)[blk >> 3];
                } else {
                    dh[i][r] = reinterpret_cast<const uint16_t*>(a.d)[blk];
                }
            }
        }
    };
    auto scale = [&](int i, int r) {
        return valid[i] ? __half2float(__ushort_as_half(dh[i][r])) : 0.f;
    };

    // block dot products of one pass
    auto compute = [&]() {
#pragma unroll
        for (int i = 0; i < BT; i++) {
            float xv[M][1][32];  // this thread's block of the staged activations
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float* xb = xs + (m * nb + bc[i]) * XPAD;
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const float4 t = *reinterpret_cast<const float4*>(xb + 4 * c);
                    xv[m][0][4 * c] = t.x;
                    xv[m][0][4 * c + 1] = t.y;
                    xv[m][0][4 * c + 2] = t.z;
                    xv[m][0][4 * c + 3] = t.w;
                }
            }
            float sx[M], sxl[M], sxh[M];
#pragma unroll
            for (int m = 0; m < M; m++) {
                float sx0 = 0.f, sx1 = 0.f;
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    sx0 += xv[m][0][j];
                    sx1 += xv[m][0][16 + j];
                }
                sxl[m] = sx0;
                sxh[m] = sx1;
                sx[m] = sx0 + sx1;
            }
            // row outer, activation row inner: each quant word is unpacked once
#pragma unroll
            for (int r = 0; r < RWT; r++) {
                float s0[M], s1[M];
#pragma unroll
                for (int m = 0; m < M; m++) s0[m] = s1[m] = 0.f;
                if constexpr (NIB) {
                    // a byte n < 16 read as OCP e4m3 is exactly n * 2^-9 (exponent field 0 or 1),
                    // so one v_cvt_pk_f32_fp8 turns two nibbles into floats; the sums carry the
                    // factor 2^-9 exactly and it is removed once per unit
                    const uint32_t q[4] = {w[i][r][0].x, w[i][r][0].y, w[i][r][0].z, w[i][r][0].w};
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const uint32_t lo = q[c] & 0x0F0F0F0Fu, hi = (q[c] >> 4) & 0x0F0F0F0Fu;
                        const float2v l01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false);
                        const float2v l23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
                        const float2v h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
                        const float2v h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
#pragma unroll
                        for (int m = 0; m < M; m++) {
                            const float* xl = xv[m][0] + 4 * c;
                            const float* xh = xv[m][0] + 16 + 4 * c;
                            s0[m] = fmaf(xl[0], l01.x, s0[m]);
                            s0[m] = fmaf(xl[1], l01.y, s0[m]);
                            s0[m] = fmaf(xl[2], l23.x, s0[m]);
                            s0[m] = fmaf(xl[3], l23.y, s0[m]);
                            s1[m] = fmaf(xh[0], h01.x, s1[m]);
                            s1[m] = fmaf(xh[1], h01.y, s1[m]);
                            s1[m] = fmaf(xh[2], h23.x, s1[m]);
                            s1[m] = fmaf(xh[3], h23.y, s1[m]);
                        }
                    }
                    if constexpr (QT == TL_HIP_GGML_Q4_0) {
                        const float dd = scale(i, r);
#pragma unroll
                        for (int m = 0; m < M; m++)
                            acc[m][r] = fmaf(dd, (s0[m] + s1[m]) * 512.f - 8.f * sx[m], acc[m][r]);
                    } else {
                        // unit = sub-block bc & 7: du * sum x q - mu * sum x
                        float du, mu;
                        k4_sm(kh[i][r], (int)(bc[i] & 7), &du, &mu);
                        du = valid[i] ? du : 0.f;
                        mu = valid[i] ? mu : 0.f;
#pragma unroll
                        for (int m = 0; m < M; m++)
                            acc[m][r] = fmaf(du, (s0[m] + s1[m]) * 512.f, fmaf(-mu, sx[m], acc[m][r]));
                    }
                } else if constexpr (QT == TL_HIP_GGML_Q6_K) {
                    // 6-bit values rebuilt per byte: low nibble | high 2 bits << 4
                    const uint32_t q[4] = {w[i][r][0].x, w[i][r][0].y, w[i][r][0].z, w[i][r][0].w};
                    const uint32_t H0 = h6[i][r].x, H1 = h6[i][r].y;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const uint32_t lo = (q[c] & 0x0F0F0F0Fu) | (((H0 >> (2 * c)) & 0x03030303u) << 4);
                        const uint32_t hi = ((q[c] >> 4) & 0x0F0F0F0Fu) | (((H1 >> (2 * c)) & 0x03030303u) << 4);
#pragma unroll
                        for (int m = 0; m < M; m++) {
                            s0[m] = fma4b(lo, xv[m][0] + 4 * c, s0[m]);
                            s1[m] = fma4b(hi, xv[m][0] + 16 + 4 * c, s1[m]);
                        }
                    }
                    const float dd = scale(i, r);
                    const float e0 = dd * (float)(int8_t)(s6[i][r] & 0xFF);
                    const float e1 = dd * (float)(int8_t)(s6[i][r] >> 8);
#pragma unroll
                    for (int m = 0; m < M; m++)
                        acc[m][r] = fmaf(e0, fmaf(-32.f, sxl[m], s0[m]), fmaf(e1, fmaf(-32.f, sxh[m], s1[m]), acc[m][r]));
                } else {
                    const uint32_t q[8] = {w[i][r][0].x, w[i][r][0].y, w[i][r][0].z, w[i][r][0].w,
                                           w[i][r][1].x, w[i][r][1].y, w[i][r][1].z, w[i][r][1].w};
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const uint32_t lo = q[c] ^ 0x80808080u, hi = q[4 + c] ^ 0x80808080u;
#pragma unroll
                        for (int m = 0; m < M; m++) {
                            s0[m] = fma4b(lo, xv[m][0] + 4 * c, s0[m]);
                            s1[m] = fma4b(hi, xv[m][0] + 16 + 4 * c, s1[m]);
                        }
                    }
                    const float dd = scale(i, r);
#pragma unroll
                    for (int m = 0; m < M; m++)
                        acc[m][r] = fmaf(dd, (s0[m] + s1[m]) - 128.f * sx[m], acc[m][r]);
                }
            }
        }
    };

    // (1) first pass, with the activations (all passes) staged once per workgroup in LDS by
    // coalesced loads -- a lane reading its own 128-byte block straight from memory would
    // touch 64 cache lines per load instruction.  The first XRK float4 per thread are
    // requested before the weights of the first pass and stored once they arrive, so the
    // weight stream is in flight while the staging completes.
    if constexpr (EPI == EPI_ROPE_KV) pre_pos = (uint32_t)*a.pos;
    set_cols(0);
    {
        const float* xsrc = EMBED ? a.x + (size_t)(*a.embed_id) * k : a.x;
        const uint32_t k4 = k >> 2, nthr = (uint32_t)sh.tc << sh.s_shift;  // the workgroup size
        float s2[M];
        constexpr int XRK = MERGE ? 2 : NORM ? (RWT >= 8 ? XR_NORM8 : XR_NORM) : XR;
        float4 xr[M][XRK], gr[NORM ? XRK : 1];
        // MERGE: the attention records (written by the launch just before) are requested
        // here and merged at staging, after the weight loads are issued
        float4 ro[MERGE ? XRK : 1][ATTN_SHARES];
        float2 rs[MERGE ? XRK : 1][ATTN_SHARES];
#pragma unroll
        for (int m = 0; m < M; m++) {
            s2[m] = 0.f;
#pragma unroll
            for (int j = 0; j < XRK; j++) {
                const uint32_t e = tid + j * nthr;
                if constexpr (MERGE) {
                    if (e < k4) load_shares(a.attn_rec, e, (uint32_t)a.attn_hd, ro[j], rs[j]);
                } else {
                    if (e < k4) xr[m][j] = reinterpret_cast<const float4*>(xsrc + m * k)[e];
                }
            }
        }
        if constexpr (NORM) {
#pragma unroll
            for (int j = 0; j < XRK; j++) {
                const uint32_t e = tid + j * nthr;
                if (e < k4) gr[j] = reinterpret_cast<const float4*>(a.norm_w)[e];
            }
        }
        load_w();
        auto stage = [&](int m, uint32_t e, float4 v, float4 g) {
            if constexpr (EMBED) {
                if (bid == 0 && a.x_out) reinterpret_cast<float4*>(a.x_out)[e] = v;
            }
            if constexpr (NORM) {
                s2[m] = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, s2[m]))));
                v.x *= g.x;
                v.y *= g.y;
                v.z *= g.z;
                v.w *= g.w;
            }
            *reinterpret_cast<float4*>(xs + (m * nb + (e >> 3)) * XPAD + (e & 7) * 4) = v;
        };
#pragma unroll
        for (int m = 0; m < M; m++) {
#pragma unroll
            for (int j = 0; j < XRK; j++) {
                const uint32_t e = tid + j * nthr;
                if constexpr (MERGE) {
                    if (e < k4) {
                        const float4 v = merge_shares(ro[j], rs[j]);
                        stage(m, e, v, v);
                    }
                } else {
                    if (e < k4) stage(m, e, xr[m][j], NORM ? gr[j] : xr[m][j]);
                }
            }
            for (uint32_t e = tid + XRK * nthr; e < k4; e += nthr) {  // long rows only
                float4 v;
                if constexpr (MERGE) {
                    float4 o[ATTN_SHARES];
                    float2 st[ATTN_SHARES];
                    load_shares(a.attn_rec, e, (uint32_t)a.attn_hd, o, st);
                    v = merge_shares(o, st);
                } else {
                    v = reinterpret_cast<const float4*>(xsrc + m * k)[e];
                }
                stage(m, e, v, NORM ? reinterpret_cast<const float4*>(a.norm_w)[e] : v);
            }
        }
        if constexpr (NORM) {
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float ss = wsum(s2[m]);
                if (lane == 0) ssq[wave][m] = ss;
            }
        }
    }
    if constexpr (EPI == EPI_RES) {
        if (tid < M * RW && row0 + (tid & (RW - 1)) < n)
            pre_res = a.res[(tid >> rw_shift) * n + row0 + (tid & (RW - 1))];
    } else if constexpr (EPI == EPI_ROPE_KV) {
        // pair (row tid, row tid + 1) is rotated by the thread that forms row tid's sum
        const uint32_t r0 = row0 + tid + (uint32_t)a.row_off;
        if (tid < RW && (tid & 1) == 0 && row0 + tid < n && r0 < (uint32_t)(a.q_rows + a.kv_rows)) {
            const uint32_t i = (r0 < (uint32_t)a.q_rows ? r0 : r0 - a.q_rows) % (uint32_t)a.hd;
            pre_c = a.cos_t[pre_pos * a.hd + i];
            pre_s = a.sin_t[pre_pos * a.hd + i];
        }
    } else if constexpr (EPI == EPI_ARGMAX) {
        if (a.seen && tid < RW && row0 + tid < n) pre_seen = a.seen[row0 + tid];
    }
    __syncthreads();
    compute();
    // (2) further passes: rows of more than BT * TC blocks
    for (uint32_t base = (uint32_t)(BT * TC); base < nb; base += (uint32_t)(BT * TC)) {
        set_cols(base);
        load_w();
        compute();
    }

    // (4) thread partials -> row sums: transpose-reduce per wavefront, then across wavefronts
    float row_v = 0.f;
    {
        float v[N];
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int r = 0; r < RWT; r++) v[m * RWT + r] = acc[m][r];
        const float t = xreduce<N>(v, lane);
        constexpr int G = 64 / N;
        if ((lane & (G - 1)) == 0) red[wave][lane / G] = t;
        __syncthreads();
        if (tid < M * RW) {  // value (m, j) of subset s is row s + S * j
            const int m = tid >> rw_shift, rl = tid & (RW - 1), s = rl & (S - 1), j = rl >> sh.s_shift;
            float acc_s = 0.f;
            for (int q = s * wps; q < (s + 1) * wps; q++) acc_s += red[q][m * RWT + j];
            if constexpr (NORM) {
                float ss = 0.f;
                for (int q = 0; q < ((sh.tc << sh.s_shift) >> 6); q++) ss += ssq[q][m];
                acc_s = acc_s / sqrtf(ss / (float)k + a.eps);
            }
            if constexpr (EPI == EPI_PLAIN || EPI == EPI_RES) {
                // the thread that forms row rl's sum stores it (its residual was loaded by
                // this thread too): no LDS round trip and no second barrier
                const uint32_t row = row0 + rl;
                if (row < n) {
                    float v = acc_s;
                    if constexpr (EPI == EPI_RES) v = pre_res + v;
                    st_wt(a.y + m * n + row, v);
                }
            } else if constexpr (EPI == EPI_ARGMAX) {
                row_v = acc_s;  // row tid (m = 0, RW <= 64: wavefront 0)
            } else if constexpr (EPI == EPI_GLU) {
                // rows (2i, 2i + 1) = (gate_i, up_i) are formed in lanes tid, tid ^ 1: the gate
                // lane takes the up value with one lane exchange (no LDS round trip, no barrier)
                const float u = dpp_f<0xB1>(acc_s);  // lane tid ^ 1 (both lanes of a pair are active)
                const uint32_t half_n = n / 2, i = row0 / 2 + (rl >> 1);
                if ((rl & 1) == 0 && i < half_n) st_wt(a.y + m * half_n + i, (acc_s * (1.0f / (1.0f + expf(-acc_s)))) * u);
            } else if constexpr (EPI == EPI_ROPE_KV) {
                // dims (2j, 2j + 1) of a head are rows rl, rl + 1 (M = 1): the even lane rotates
                // the pair and writes q or the KV cache; v rows are appended as they are
                const float v1 = dpp_f<0xB1>(acc_s);  // lane tid ^ 1 (both lanes of a pair are active)
                if ((rl & 1) == 0 && row0 + rl < n) {
                    const float v0 = acc_s;
                    const int64_t pos = pre_pos;
                    const int64_t r0 = row0 + rl + a.row_off;  // row of the q | k | v projection
                    if (r0 < a.q_rows + a.kv_rows) {
                        const bool isq = r0 < a.q_rows;
                        const int64_t rr = isq ? r0 : r0 - a.q_rows;
                        const int64_t i = rr % a.hd;
                        const float c = pre_c, sn = pre_s;
                        const float o0 = v0 * c - v1 * sn, o1 = v0 * sn + v1 * c;
                        if (isq) {
                            st_wt(a.q_out + r0, o0);
                            st_wt(a.q_out + r0 + 1, o1);
                        } else {
                            const int64_t off = ((rr / a.hd) * a.max_seq + pos) * a.hd + i;
                            if (a.kv_f16) {
                                st_wt(reinterpret_cast<__half*>(a.kc) + off, __float2half(o0));
                                st_wt(reinterpret_cast<__half*>(a.kc) + off + 1, __float2half(o1));
                            } else {
                                st_wt(reinterpret_cast<float*>(a.kc) + off, o0);
                                st_wt(reinterpret_cast<float*>(a.kc) + off + 1, o1);
                            }
                        }
                    } else {
                        const int64_t rr = r0 - a.q_rows - a.kv_rows, i = rr % a.hd;
                        const int64_t off = ((rr / a.hd) * a.max_seq + pos) * a.hd + i;
                        if (a.kv_f16) {
                            st_wt(reinterpret_cast<__half*>(a.vc) + off, __float2half(v0));
                            st_wt(reinterpret_cast<__half*>(a.vc) + off + 1, __float2half(v1));
                        } else {
                            st_wt(reinterpret_cast<float*>(a.vc) + off, v0);
                            st_wt(reinterpret_cast<float*>(a.vc) + off + 1, v1);
                        }
                    }
                }
            }
        }
    }

    // (5) epilogue
    if constexpr (EPI == EPI_ARGMAX) {
        // logits, penalised logits, then this workgroup's greedy candidate (the left fold of
        // tensor.rs:1633-1637 over its rows: keep the best only when strictly greater)
        // Rows 0 .. RW - 1 sit in lanes 0 .. RW - 1 of wavefront 0 (RW <= 64).  Without NaNs the
        // fold equals (greater value, then larger index), reduced across the lanes; with a NaN
        // the flag makes k_argmax_finish replay the sequential fold over the penalised logits.
        if (wave == 0) {
            const uint32_t row = row0 + lane;
            const bool live = lane < RW && row < n;
            float v = row_v;
            if (live) {
                st_wt(a.y + row, v);
                if (pre_seen) v = v > 0.0f ? v / a.penalty : v * a.penalty;
                st_wt(a.plogits + row, v);
            }
            float bv = live ? v : -INFINITY;
            int bi = live ? lane : -1, nan = live && v != v;
            argmax_allreduce(bv, bi, nan);
            if (lane == 0) {
                st_wt(a.part_v + bid, bv);
                st_wt(a.part_i + bid, (int32_t)(row0 + bi));
                st_wt(a.part_nan + bid, (int32_t)nan);
            }
        }
    }
}

template <int QT, int BT, int RWT, int M, int EPI, bool NORM, bool EMBED, bool MERGE = false>
__global__ __launch_bounds__(512) void k_mv(const uint8_t* __restrict__ qs_p, const void* __restrict__ w1_p,
                                            const float* __restrict__ x_p, const float* __restrict__ aux_p,
                                            const int32_t* __restrict__ aux2_p, uint32_t n_p, uint32_t nb_p,
                                            uint32_t shape_p, int aux_i, MvArgs a) {
    mv_body<QT, BT, RWT, M, EPI, NORM, EMBED, MERGE>(qs_p, w1_p, x_p, aux_p, aux2_p, n_p, nb_p, shape_p, aux_i, a,
                                                     blockIdx.x);
}

// Two weights of one q | k | v projection in one launch (a layer whose q | k and v rows have
// different types, as llama.cpp's Q4_K_M mixture gives 10 of 22 TinyLlama layers): workgroups
// [0, grid1) run segment 1's matvec, the rest segment 2's, on the same staged input row
// (RMSNorm prologue, RoPE + KV-append epilogue); segment 2's workgroup 0 does not store the
// embedded row.  Both segments take the same workgroup size and K.
template <int QT1, int RWT1, int QT2, int RWT2, bool EMBED>
__global__ __launch_bounds__(512) void k_mv_pair(const uint8_t* __restrict__ qs_p, const void* __restrict__ w1_p,
                                                 const float* __restrict__ x_p, const float* __restrict__ aux_p,
                                                 const int32_t* __restrict__ aux2_p, uint32_t n_p, uint32_t nb_p,
                                                 uint32_t shape_p, uint32_t grid1, MvArgs a, MvArgs a2,
                                                 uint32_t shape2) {
    if (blockIdx.x < grid1)
        mv_body<QT1, 1, RWT1, 1, EPI_ROPE_KV, true, EMBED, false>(qs_p, w1_p, x_p, aux_p, aux2_p, n_p, nb_p, shape_p,
                                                                  0, a, blockIdx.x);
    else
        mv_body<QT2, 1, RWT2, 1, EPI_ROPE_KV, true, EMBED, false>(
            a2.qs, QT2 == TL_HIP_GGML_Q4_K ? (const void*)a2.hdr : QT2 == TL_HIP_GGML_Q6_K ? (const void*)a2.qh
                                                                                          : (const void*)a2.d,
            x_p, aux_p, aux2_p, (uint32_t)a2.n, nb_p, shape2, 0, a2, blockIdx.x - grid1);
}

// Greedy token from the per-workgroup candidates of an EPI_ARGMAX matvec (one workgroup):
// the candidates are folded in workgroup order; for NaN-free input the (greater value, then
// larger index) reduction equals the left fold of tensor.rs:1633-1637, otherwise thread 0
// replays that fold over the penalised logits.  Then the decode-step bookkeeping: token
// recorded, penalty mask updated, position advanced.
__global__ __launch_bounds__(256) void k_argmax_finish(float* part_v, int32_t* part_i, int32_t* part_nan,
                                                       int32_t* step, int32_t* pos_inc, int32_t* out_ids, int nwg,
                                                       MvArgs a) {
    // what the first loads need comes first (preloaded into SGPRs at dispatch); the fields the
    // stores at the end use are loaded from the argument buffer meanwhile
    a.part_v = part_v;
    a.part_i = part_i;
    a.part_nan = part_nan;
    a.step = step;
    a.pos_inc = pos_inc;
    a.out_ids = out_ids;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR
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
    // the step counter and the position are read with the candidates, one memory round trip
    // (read after the stores below they would each cost another)
    int step0 = 0, pos0 = 0;
    if (tid == 0) {
        if (a.out_ids) step0 = *a.step;
        if (a.pos_inc) pos0 = *a.pos_inc;
    }
    argmax_allreduce(bv, bi, nan);
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
        st_wt(a.tok_out, (int32_t)bi);
        if (a.out_ids) {
            if (step0 < a.max_out) st_wt(a.out_ids + step0, (int32_t)bi);
            st_wt(a.step, (int32_t)(step0 + 1));
        }
        if (a.seen_out) st_wt(a.seen_out + bi, (uint8_t)1);
        if (a.pos_inc) st_wt(a.pos_inc, (int32_t)(pos0 + 1));
    }
}

// ---------------------------------------------------------------- dispatch --------------
// TC = nb rounded up to wavefronts (at most 256) threads per row subset, BT block columns
// per thread and pass (2 once nb > 256), S row subsets (four wavefronts per workgroup when
// TC is one or two wavefronts; twice that when the grid stays a multiple of 256), RWT rows
// per thread: the smallest of 2, 4, 8 that keeps the grid at <= 720 workgroups (about three
// per CU), with at most 64 quant VGPRs per thread.
// (Measured on MI355X over the decode shapes: fewer, fuller workgroups lose to this because
// the per-thread block math then serialises on fewer SIMDs; many more lose to the repeated
// activation loads.)
struct MvPlan {
    int TC, S, BT, RWT;
    int64_t grid;
    MvShape shape() const {
        int tc_shift = 0, s_shift = 0;
        while ((1 << tc_shift) < TC) tc_shift++;
        while ((1 << s_shift) < S) s_shift++;
        return MvShape{TC, tc_shift, s_shift};
    }
};
constexpr int MV_MIN_RW = 2;

static MvPlan mv_plan(int64_t n, int64_t nb, int qt) {
    MvPlan p;
    p.TC = (int)(nb >= 256 ? 256 : cdiv(nb, 64) * 64);
    p.BT = nb > 256 ? 2 : 1;
    p.S = p.TC <= 128 ? 256 / p.TC : 1;  // TC of 64 or 128: a power of two
    const int qw = qt == TL_HIP_GGML_Q4_0 ? 1 : 2;  // 16-byte loads per unit incl. scale data
    int rwt = 2;
    while (rwt < 8 && cdiv(n, (int64_t)p.S * rwt) > 720) rwt *= 2;
    while (rwt > 2 && rwt * p.BT * qw > 16) rwt /= 2;
    p.RWT = rwt;
    // 512-thread workgroups (twice the row subsets, the activations staged once for twice the
    // rows) when the grid stays a whole number of workgroups per CU -- a multiple of 256.
    // Measured on MI355X: Q4_0 / Q4_K 4096^2 4.19 -> 4.07 / 4.72 -> 4.61 us, 4096 x 11008 Q4_0
    // 10.69 -> 10.17, Q8_0 15.2 -> 12.2 us (Q8_0 / Q6_K 4096^2 +1 %); at 344 workgroups
    // (11008 x 4096) the doubled form loses 19 %, and the decode shapes keep 256 threads.
    const int64_t g2 = cdiv(n, (int64_t)p.S * 2 * rwt);
    if ((p.TC & (p.TC - 1)) == 0 && p.S * p.TC == 256 && g2 >= 256 && g2 % 256 == 0) p.S *= 2;
    p.grid = cdiv(n, (int64_t)p.S * rwt);
    return p;
}

template <int QT, int BT, int RWT, int M, int EPI, bool NORM, bool EMBED, bool MERGE = false>
static int run(const MvArgs& a, const MvPlan& p, hipStream_t s) {
    const size_t lds = (size_t)M * a.nb * XPAD * sizeof(float);
    auto kern = k_mv<QT, BT, RWT, M, EPI, NORM, EMBED, MERGE>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(LDS)");
    }
    const MvShape sh = p.shape();
    const void* w1 = QT == TL_HIP_GGML_Q4_K ? (const void*)a.hdr : QT == TL_HIP_GGML_Q6_K ? (const void*)a.qh
                                                                                       : (const void*)a.d;
    kern<<<(unsigned)p.grid, p.S * p.TC, lds, s>>>(a.qs, w1, a.x, NORM ? a.norm_w : MERGE ? a.attn_rec : nullptr,
                                                  EMBED ? a.embed_id : EPI == EPI_ROPE_KV ? a.pos : nullptr,
                                                  (uint32_t)a.n, (uint32_t)a.nb, sh.pack(), MERGE ? a.attn_hd : 0, a);
    if constexpr (EPI == EPI_ARGMAX) {
        if (a.smp_temp > 0.0f) {  // top-p sampling of the penalised logits instead of the greedy finish
            const SmpFin fin{a.smp_draws, a.tok_out, a.out_ids, a.step, a.seen_out, a.pos_inc, a.max_out};
            const int rc = launch_sample_top_p(a.plogits, a.n, a.smp_temp, a.smp_top_p, 0.0f, a.smp_key, nullptr, &fin, s);
            if (rc) return rc;
        } else {
            k_argmax_finish<<<1, 256, 0, s>>>(a.part_v, a.part_i, a.part_nan, a.step, a.pos_inc, a.out_ids,
                                              (int)p.grid, a);
        }
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "matvec launch");
}

// (BT, RWT) combinations the plan can produce: Q4_0 (1, 8|4|2), (2, 8|4|2);
// Q8_0 (1, 8|4|2), (2, 4|2).
template <int QT, int M, int EPI, bool NORM, bool EMBED, bool MERGE = false>
static int run_p(const MvArgs& a, const MvPlan& p, hipStream_t s) {
    if (p.BT == 1) {
        if (p.RWT == 8) return run<QT, 1, 8, M, EPI, NORM, EMBED, MERGE>(a, p, s);
        if (p.RWT == 4) return run<QT, 1, 4, M, EPI, NORM, EMBED, MERGE>(a, p, s);
        return run<QT, 1, 2, M, EPI, NORM, EMBED, MERGE>(a, p, s);
    }
    if constexpr (QT == TL_HIP_GGML_Q4_0)
        if (p.RWT == 8) return run<QT, 2, 8, M, EPI, NORM, EMBED, MERGE>(a, p, s);
    if (p.RWT == 4) return run<QT, 2, 4, M, EPI, NORM, EMBED, MERGE>(a, p, s);
    return run<QT, 2, 2, M, EPI, NORM, EMBED, MERGE>(a, p, s);
}

template <int QT>
static int run_t(const MvArgs& a, int m, int epi, bool norm, bool embed, const MvPlan& p, hipStream_t s) {
    if (m == 2) {
        if (epi == EPI_RES) return run_p<QT, 2, EPI_RES, false, false>(a, p, s);
        return run_p<QT, 2, EPI_PLAIN, false, false>(a, p, s);
    }
    switch (epi) {
        case EPI_RES:
            if (a.attn_rec) return run_p<QT, 1, EPI_RES, false, false, true>(a, p, s);
            return run_p<QT, 1, EPI_RES, false, false>(a, p, s);
        case EPI_GLU:
            return norm ? run_p<QT, 1, EPI_GLU, true, false>(a, p, s) : run_p<QT, 1, EPI_GLU, false, false>(a, p, s);
        case EPI_ROPE_KV:
            if (embed) return run_p<QT, 1, EPI_ROPE_KV, true, true>(a, p, s);
            return norm ? run_p<QT, 1, EPI_ROPE_KV, true, false>(a, p, s)
                        : run_p<QT, 1, EPI_ROPE_KV, false, false>(a, p, s);
        case EPI_ARGMAX:
            return norm ? run_p<QT, 1, EPI_ARGMAX, true, false>(a, p, s) : run_p<QT, 1, EPI_ARGMAX, false, false>(a, p, s);
        default:
            return norm ? run_p<QT, 1, EPI_PLAIN, true, false>(a, p, s) : run_p<QT, 1, EPI_PLAIN, false, false>(a, p, s);
    }
}

// Checks and launches one fused matvec.  m is 1 or 2 (2 only with EPI_PLAIN / EPI_RES
// and no prologue).
int launch_mv(const QWeight* w, MvArgs a, int m, int epi, bool norm, bool embed, hipStream_t s) {
    a.qs = w->qs;
    a.d = w->d;
    a.hdr = w->hdr;
    a.qh = w->qh;
    a.sc = w->sc;
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
    if (a.n < 1 || a.nb < 1) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: empty matvec weight");
        return TL_HIP_ERR_SHAPE;
    }
    if ((uint64_t)a.n * a.nb * (w->ggml_type == TL_HIP_GGML_Q8_0 ? 32 : 16) >= (1ull << 31)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: quant weight of %lld x %lld exceeds the 2 GiB decode matvec limit",
                  (long long)a.n, (long long)a.k);
        return TL_HIP_ERR_ARG;
    }
    const MvPlan p = mv_plan(a.n, a.nb, w->ggml_type);
    if ((size_t)m * a.nb * XPAD * sizeof(float) > 150 * 1024) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: k = %lld too large for the LDS-staged matvec", (long long)a.k);
        return TL_HIP_ERR_ARG;
    }
    if ((epi == EPI_GLU || epi == EPI_ROPE_KV) && (a.n % 2)) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: paired epilogue needs an even row count");
        return TL_HIP_ERR_SHAPE;
    }
    if (a.attn_rec && (m != 1 || epi != EPI_RES || norm || embed || a.attn_hd < 4 || a.attn_hd % 4 ||
                       a.k % a.attn_hd || (reinterpret_cast<uintptr_t>(a.attn_rec) & 15))) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: attention-record input needs m = 1, the residual epilogue, "
                  "head size a multiple of 4 dividing k, 16-byte aligned records");
        return TL_HIP_ERR_ARG;
    }
    switch (w->ggml_type) {
        case TL_HIP_GGML_Q4_0: return run_t<TL_HIP_GGML_Q4_0>(a, m, epi, norm, embed, p, s);
        case TL_HIP_GGML_Q8_0: return run_t<TL_HIP_GGML_Q8_0>(a, m, epi, norm, embed, p, s);
        case TL_HIP_GGML_Q4_K: return run_t<TL_HIP_GGML_Q4_K>(a, m, epi, norm, embed, p, s);
        default: return run_t<TL_HIP_GGML_Q6_K>(a, m, epi, norm, embed, p, s);
    }
}

// One launch for a two-weight q | k | v projection (k_mv_pair): Q4_K rows, then Q6_K rows, or
// the reverse, with the RMSNorm prologue and the RoPE + KV epilogue; a holds the shared
// arguments and segment 1's row offset, row_off2 segment 2's.  Returns -1 without launching
// when the pair is not covered (other types or plans, or the checks of launch_mv fail): the
// caller then launches each weight on its own.
int launch_mv_pair(const QWeight* w1, const QWeight* w2, MvArgs a, int64_t row_off2, bool embed, hipStream_t s) {
    const int t1 = w1->ggml_type, t2 = w2->ggml_type;
    const bool kq = (t1 == TL_HIP_GGML_Q4_K && t2 == TL_HIP_GGML_Q6_K) || (t1 == TL_HIP_GGML_Q6_K && t2 == TL_HIP_GGML_Q4_K);
    if (!kq || w1->nb != w2->nb || w1->n % 2 || w2->n % 2 || (reinterpret_cast<uintptr_t>(a.x) & 15) ||
        (reinterpret_cast<uintptr_t>(a.norm_w) & 15) || !a.norm_w)
        return -1;
    for (const QWeight* w : {w1, w2})
        if ((uint64_t)w->n * w->nb * 16 >= (1ull << 31)) return -1;
    if ((size_t)w1->nb * XPAD * sizeof(float) > 64 * 1024) return -1;  // default LDS limit: no attribute call
    const MvPlan p1 = mv_plan(w1->n, w1->nb, t1), p2 = mv_plan(w2->n, w2->nb, t2);
    if (p1.BT != 1 || p2.BT != 1 || p1.S * p1.TC != p2.S * p2.TC || p1.TC != p2.TC || (p1.RWT != 2 && p1.RWT != 4) ||
        (p2.RWT != 2 && p2.RWT != 4))
        return -1;
    MvArgs a1 = a, b = a;
    for (auto [ar, w] : {std::pair<MvArgs*, const QWeight*>{&a1, w1}, {&b, w2}}) {
        ar->qs = w->qs;
        ar->d = w->d;
        ar->hdr = w->hdr;
        ar->qh = w->qh;
        ar->sc = w->sc;
        ar->n = w->n;
        ar->k = w->k;
        ar->nb = w->nb;
    }
    b.row_off = row_off2;
    b.x_out = nullptr;  // the embedded row is stored once, by segment 1
    const size_t lds = (size_t)a.nb * XPAD * sizeof(float);
    const unsigned grid = (unsigned)(p1.grid + p2.grid), threads = (unsigned)(p1.S * p1.TC);
    const void* x1 = t1 == TL_HIP_GGML_Q4_K ? (const void*)a1.hdr : (const void*)a1.qh;
    const int32_t* aux2 = embed ? a.embed_id : a.pos;
    const uint32_t sh1 = p1.shape().pack(), sh2 = p2.shape().pack(), g1 = (uint32_t)p1.grid;
#define TLH_PAIR(Q1, R1, Q2, R2)                                                                              \
    if (t1 == Q1 && p1.RWT == R1 && p2.RWT == R2) {                                                            \
        if (embed)                                                                                             \
            k_mv_pair<Q1, R1, Q2, R2, true><<<grid, threads, lds, s>>>(a1.qs, x1, a.x, a.norm_w, aux2,           \
                                                                      (uint32_t)a1.n, (uint32_t)a1.nb, sh1, g1,  \
                                                                      a1, b, sh2);                               \
        else                                                                                                   \
            k_mv_pair<Q1, R1, Q2, R2, false><<<grid, threads, lds, s>>>(a1.qs, x1, a.x, a.norm_w, aux2,          \
                                                                       (uint32_t)a1.n, (uint32_t)a1.nb, sh1, g1, \
                                                                       a1, b, sh2);                              \
        hipError_t e = hipGetLastError();                                                                      \
        return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "matvec pair launch");                                \
    }
    TLH_PAIR(TL_HIP_GGML_Q4_K, 2, TL_HIP_GGML_Q6_K, 2)
    TLH_PAIR(TL_HIP_GGML_Q4_K, 4, TL_HIP_GGML_Q6_K, 2)
    TLH_PAIR(TL_HIP_GGML_Q4_K, 2, TL_HIP_GGML_Q6_K, 4)
    TLH_PAIR(TL_HIP_GGML_Q4_K, 4, TL_HIP_GGML_Q6_K, 4)
    TLH_PAIR(TL_HIP_GGML_Q6_K, 2, TL_HIP_GGML_Q4_K, 2)
    TLH_PAIR(TL_HIP_GGML_Q6_K, 4, TL_HIP_GGML_Q4_K, 2)
    TLH_PAIR(TL_HIP_GGML_Q6_K, 2, TL_HIP_GGML_Q4_K, 4)
    TLH_PAIR(TL_HIP_GGML_Q6_K, 4, TL_HIP_GGML_Q4_K, 4)
#undef TLH_PAIR
    return -1;
}

// Whether the LDS-staged matvec takes an m-row product with this weight (rows staged two at
// a time must fit 150 KiB of LDS; the quant array stays below 2 GiB).
bool matvec_fits(const QWeight* w, int64_t m) {
    const int64_t mm = m >= 2 ? 2 : 1;
    return m >= 1 && m <= 4 && w->n >= 1 && w->nb >= 1 &&
           (uint64_t)w->n * w->nb * (w->ggml_type == TL_HIP_GGML_Q8_0 ? 32 : 16) < (1ull << 31) &&
           (size_t)mm * w->nb * XPAD * sizeof(float) <= 150 * 1024;
}

// ------------------------------------------------------------ one-launch read floor ----
// The loads of k_mv with its launch plan and access pattern -- thread (sub, tcol) reads unit
// columns tcol + TC i of rows row0 + sub + S r, quant bytes and scale data as the matvec does --
// and nothing else: the XOR of the loaded words goes to an empty asm statement, which keeps
// the loads (and the wait for them) without a store.  The time of a launch that only moves
// the weight stream the way the matvec moves it.
template <int QT, int BT, int RWT>
__global__ __launch_bounds__(512) void k_read_floor(const uint8_t* __restrict__ qs, const void* __restrict__ w1,
                                                    const int8_t* __restrict__ sc, const __half* __restrict__ d6,
                                                    uint32_t n_p, uint32_t nb_p, uint32_t shape_p) {
    constexpr int QB = QB_<QT>::v, QW = QB / 16;
    MvArgs a = {};
    a.qs = qs;
    a.n = n_p;
    a.nb = nb_p;
    a.d = QT == TL_HIP_GGML_Q6_K ? d6 : static_cast<const __half*>(w1);
    a.hdr = static_cast<const uint8_t*>(w1);
    a.qh = static_cast<const uint8_t*>(w1);
    a.sc = sc;
    const MvShape sh = MvShape::unpack(shape_p);
    const int tid = threadIdx.x;
    const int TC = sh.tc, S = 1 << sh.s_shift;
    const int tcol = sh.s_shift ? (tid & (TC - 1)) : tid;
    const int sub = sh.s_shift ? __builtin_amdgcn_readfirstlane(tid >> sh.tc_shift) : 0;  // TC >= 64: uniform
    const uint32_t nb = (uint32_t)a.nb, n = (uint32_t)a.n;
    const uint32_t my_row0 = blockIdx.x * (uint32_t)(RWT << sh.s_shift) + sub;
    uint32_t acc = 0;
    for (uint32_t base = 0; base < nb; base += (uint32_t)(BT * TC)) {
        uint4 w[BT][RWT][QW];
        uint4 extra[BT][RWT];
#pragma unroll
        for (int i = 0; i < BT; i++) {
            const uint32_t b0 = base + (uint32_t)(tcol + i * TC);
            const uint32_t b = b0 < nb ? b0 : nb - 1;
#pragma unroll
            for (int r = 0; r < RWT; r++) {
                uint32_t row = my_row0 + (uint32_t)(S * r);
                row = row < n ? row : n - 1;
                const uint32_t blk = __umul24(row, nb) + b;
                const uint4* p = reinterpret_cast<const uint4*>(a.qs + (size_t)blk * QB);
#pragma unroll
                for (int c = 0; c < QW; c++) w[i][r][c] = ld_stream(p + c);
                if constexpr (QT == TL_HIP_GGML_Q4_K) {
                    extra[i][r] = reinterpret_cast<const uint4*>(a.hdr)[blk >> 3];
                } else if constexpr (QT == TL_HIP_GGML_Q6_K) {
                    const uint2 hq = reinterpret_cast<const uint2*>(a.qh)[blk];
                    extra[i][r] = uint4{hq.x, hq.y, reinterpret_cast<const uint16_t*>(a.sc)[blk],
                                        reinterpret_cast<const uint16_t*>(a.d)[blk >> 3]};
                } else {
                    extra[i][r] = uint4{reinterpret_cast<const uint16_t*>(a.d)[blk], 0u, 0u, 0u};
                }
            }
        }
#pragma unroll
        for (int i = 0; i < BT; i++)
#pragma unroll
            for (int r = 0; r < RWT; r++) {
#pragma unroll
                for (int c = 0; c < QW; c++) acc ^= w[i][r][c].x ^ w[i][r][c].y ^ w[i][r][c].z ^ w[i][r][c].w;
                acc ^= extra[i][r].x ^ extra[i][r].y ^ extra[i][r].z ^ extra[i][r].w;
            }
    }
    asm volatile("" : : "v"(acc));
}

template <int QT>
static int run_floor(const MvArgs& a, const MvPlan& p, hipStream_t s) {
    const dim3 grid((unsigned)p.grid), block((unsigned)(p.S * p.TC));
    const MvShape sh = p.shape();
    const void* w1 = QT == TL_HIP_GGML_Q4_K ? (const void*)a.hdr : QT == TL_HIP_GGML_Q6_K ? (const void*)a.qh
                                                                                       : (const void*)a.d;
    const uint32_t n = (uint32_t)a.n, nb = (uint32_t)a.nb;
#define TLH_FLOOR(B, R) k_read_floor<QT, B, R><<<grid, block, 0, s>>>(a.qs, w1, a.sc, a.d, n, nb, sh.pack())
    if (p.BT == 1) {
        if (p.RWT == 8) TLH_FLOOR(1, 8);
        else if (p.RWT == 4) TLH_FLOOR(1, 4);
        else TLH_FLOOR(1, 2);
    } else {
        if (p.RWT == 8) TLH_FLOOR(2, 8);
        else if (p.RWT == 4) TLH_FLOOR(2, 4);
        else TLH_FLOOR(2, 2);
    }
#undef TLH_FLOOR
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "read floor launch");
}

int launch_read_floor(const QWeight* w, hipStream_t s) {
    if (w->n < 1 || w->nb < 1 ||
        (uint64_t)w->n * w->nb * (w->ggml_type == TL_HIP_GGML_Q8_0 ? 32 : 16) >= (1ull << 31)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: weight outside the decode matvec's limits");
        return TL_HIP_ERR_ARG;
    }
    MvArgs a = {};
    a.qs = w->qs;
    a.d = w->d;
    a.hdr = w->hdr;
    a.qh = w->qh;
    a.sc = w->sc;
    a.n = w->n;
    a.k = w->k;
    a.nb = w->nb;
    const MvPlan p = mv_plan(w->n, w->nb, w->ggml_type);
    switch (w->ggml_type) {
        case TL_HIP_GGML_Q4_0: return run_floor<TL_HIP_GGML_Q4_0>(a, p, s);
        case TL_HIP_GGML_Q8_0: return run_floor<TL_HIP_GGML_Q8_0>(a, p, s);
        case TL_HIP_GGML_Q4_K: return run_floor<TL_HIP_GGML_Q4_K>(a, p, s);
        default: return run_floor<TL_HIP_GGML_Q6_K>(a, p, s);
    }
}

// Upper bound on the workgroups (= argmax partial slots) of a matvec over n rows.
int mv_partials(int64_t n) { return (int)cdiv(n, MV_MIN_RW); }

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
