// Single-query decode attention with grouped KV heads over a KV cache (f16 or f32), the
// replacement of the chatbot's transpose / cat_4d / repeat_interleave / matmul_4d / scale /
// softmax / matmul_4d chain (examples/apps/tinyllama/chatbot.tl:63-87): K and V are read in
// place, and the Hq/Hkv query heads of a group share every K/V row loaded (no
// repeat_interleave copy).  A causal prefill of n queries over one shared cache is the same
// computation with per-query lengths (AttnLen.len_step = 1).  Three forms, all f32 arithmetic:
//   * k_attn_qh  short caches (decode of the chatbot's model): one workgroup per query head;
//   * k_attn_gq  f16 caches, 4 or 8 query heads per KV head, head_dim 64 / 128: one workgroup
//                per (split of 128 or 64 positions, KV head, query), every row read once for
//                all heads of the group, then k_attn_merge_gq (flash-decoding);
//   * k_attn     the general form (f32 caches, other group sizes), split the same way, then
//                k_attn_merge.
// A split's record is (o, max, sum); the merge forms
// out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M); a single split writes its result.
#include "internal.h"

namespace tlhip {

template <typename KVT>
struct KVLoad;

template <>
struct KVLoad<__half> {
    template <int DL>
    __device__ static void load(const __half* p, float* out) {
        static_assert(DL % 8 == 0, "f16 rows are read 16 bytes at a time");
#pragma unroll
        for (int i = 0; i < DL / 8; i++) {
            uint4 w = reinterpret_cast<const uint4*>(p)[i];
            const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                __half2 h2 = *reinterpret_cast<const __half2*>(&u[j]);
                float2 f = __half22float2(h2);
                out[8 * i + 2 * j] = f.x;
                out[8 * i + 2 * j + 1] = f.y;
            }
        }
    }
};

template <>
struct KVLoad<float> {
    template <int DL>
    __device__ static void load(const float* p, float* out) {
#pragma unroll
        for (int i = 0; i < DL / 4; i++) {
            float4 v = reinterpret_cast<const float4*>(p)[i];
            out[4 * i] = v.x;
            out[4 * i + 1] = v.y;
            out[4 * i + 2] = v.z;
            out[4 * i + 3] = v.w;
        }
    }
};

constexpr int ATT_MAX_CHUNK = 1024;
constexpr int ATT_MAX_SPLITS = 256;
// One-launch grouped split form: arrival counters per (batch item, KV head), zero at load and
// returned to zero by the workgroup that arrives last, which merges the item's split records
// (at most ATT_FUSE_MAX: one workgroup reading more records costs more than a merge launch).
constexpr int ATT_ARRIVE_MAX = 4096;
constexpr int ATT_FUSE_MAX = 8;
__device__ uint32_t g_attn_arrive[ATT_ARRIVE_MAX];

constexpr int ATT_PF = 2;  // 32-position steps whose K/V rows are requested up front

// Cached length of batch item b: (len_dev ? *len_dev + len_add : L) + b * len_step.
// Decode uses len_step 0; a causal prefill of n queries over one shared cache
// (kv_bstride 0) uses len_step 1, so query i sees positions 0 .. base + i.
struct AttnLen {
    int64_t L;
    const int32_t* len_dev;
    int len_add, len_step;
    __device__ int64_t of(int b) const {
        return (len_dev ? (int64_t)(*len_dev) + len_add : L) + (int64_t)b * len_step;
    }
};

struct AttnArgs {
    const float* q;  // [B, Hq, D]
    const void* k;   // [B?, Hkv, lmax, D]
    const void* v;
    float* out;      // [B, Hq, D]
    float* ws;       // [B, Hkv, nsplit, G, D + 2]
    int hkv;
    int64_t lmax, kv_bstride;
    AttnLen len;
    int chunk, nsplit;
    float scale;
};

// Every AttnArgs field the kernels' prologues read, fetched from the kernel-argument buffer in
// one round of scalar loads: left to the compiler, loads placed after the prologue's branches
// wait for an earlier round to return (three or four dependent memory round trips before the
// first K load).
__device__ __forceinline__ void attn_args_prefetch(const AttnArgs& a) {
    asm volatile("" : : "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.out), "s"(a.ws), "s"(a.hkv), "s"(a.lmax), "s"(a.kv_bstride),
                 "s"(a.len.L), "s"(a.len.len_dev), "s"(a.len.len_add), "s"(a.len.len_step), "s"(a.chunk),
                 "s"(a.nsplit), "s"(a.scale));
}

template <int D, int G, typename KVT>
__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
    attn_args_prefetch(a);
    constexpr int DL = D / 8;  // dims per lane
    __shared__ float sc[G][ATT_MAX_CHUNK];
    __shared__ float stat[G][2];
    __shared__ float part[4][G][D];
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR
    const int grp = lane >> 3, sub = lane & 7;
    int64_t L = a.len.of(b);
    if (L > a.lmax) L = a.lmax;
    const int64_t p0 = (int64_t)split * a.chunk;
    const int64_t p1 = p0 + a.chunk < L ? p0 + a.chunk : (L > p0 ? L : p0);
    const int hq = a.hkv * G;
    const KVT* kb = reinterpret_cast<const KVT*>(a.k) + (int64_t)b * a.kv_bstride + (int64_t)h * a.lmax * D;
    const KVT* vb = reinterpret_cast<const KVT*>(a.v) + (int64_t)b * a.kv_bstride + (int64_t)h * a.lmax * D;
    const int64_t rec0 = (((int64_t)b * a.hkv + h) * a.nsplit) * G * (D + 2);

    if (p0 < p1) {
        // K / V rows of the first steps, then q
        float kpre[ATT_PF][DL], vpre[ATT_PF][DL];
#pragma unroll
        for (int it = 0; it < ATT_PF; it++) {
            int64_t p = p0 + it * 32 + wave * 8 + grp;
            int64_t pc = p < p1 ? p : p1 - 1;
            KVLoad<KVT>::template load<DL>(kb + pc * D + sub * DL, kpre[it]);
            KVLoad<KVT>::template load<DL>(vb + pc * D + sub * DL, vpre[it]);
        }
        float qv[G][DL];
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float* qp = a.q + ((int64_t)b * hq + h * G + g) * D + sub * DL;
#pragma unroll
            for (int i = 0; i < DL; i += 4) {
                float4 t = *reinterpret_cast<const float4*>(qp + i);
                qv[g][i] = t.x;
                qv[g][i + 1] = t.y;
                qv[g][i + 2] = t.z;
                qv[g][i + 3] = t.w;
            }
        }
        auto scores = [&](int64_t base, const float* kv) {
            const int64_t p = base + wave * 8 + grp;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < DL; i++) s = fmaf(qv[g][i], kv[i], s);
                s = sum8_dpp(s);
                if (sub == 0 && p < p1) sc[g][p - p0] = s * a.scale;
            }
        };
#pragma unroll
        for (int it = 0; it < ATT_PF; it++)
            if (p0 + it * 32 < p1) scores(p0 + it * 32, kpre[it]);
        for (int64_t base = p0 + ATT_PF * 32; base < p1; base += 32) {
            int64_t p = base + wave * 8 + grp;
            int64_t pc = p < p1 ? p : p1 - 1;
            float kv[DL];
            KVLoad<KVT>::template load<DL>(kb + pc * D + sub * DL, kv);
            scores(base, kv);
        }
        __syncthreads();
        // per-head chunk max and exp-sum (wavefront w handles heads w, w + 4)
        const int cn = (int)(p1 - p0);
        for (int g = wave; g < G; g += 4) {
            float mx = -INFINITY;
            for (int i = lane; i < cn; i += 64) mx = fmaxf(mx, sc[g][i]);
            mx = wave_allmax(mx);
            float sum = 0.f;
            for (int i = lane; i < cn; i += 64) {
                float e = expf(sc[g][i] - mx);
                sc[g][i] = e;
                sum += e;
            }
            sum = wave_allsum(sum);
            if (lane == 0) {
                stat[g][0] = mx;
                stat[g][1] = sum;
            }
        }
        __syncthreads();
        // exp-weighted V
        float o[G][DL];
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < DL; i++) o[g][i] = 0.f;
        auto accum = [&](int64_t base, const float* vv) {
            const int64_t p = base + wave * 8 + grp;
            if (p < p1) {
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float e = sc[g][p - p0];
#pragma unroll
                    for (int i = 0; i < DL; i++) o[g][i] = fmaf(e, vv[i], o[g][i]);
                }
            }
        };
#pragma unroll
        for (int it = 0; it < ATT_PF; it++)
            if (p0 + it * 32 < p1) accum(p0 + it * 32, vpre[it]);
        for (int64_t base = p0 + ATT_PF * 32; base < p1; base += 32) {
            int64_t p = base + wave * 8 + grp;
            float vv[DL];
            if (p < p1) KVLoad<KVT>::template load<DL>(vb + p * D + sub * DL, vv);
            accum(base, vv);
        }
        // reduce over the 8 position groups of the wavefront (lane bits 3..5)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < DL; i++) {
                float v = o[g][i];
                v += dpp_f<0x128>(v);  // row_ror:8 = xor 8 within 16 lanes
                v = lane_pair_sum<16>(v);
                v = lane_pair_sum<32>(v);
                o[g][i] = v;
            }
        if (grp == 0) {
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int i = 0; i < DL; i++) part[wave][g][sub * DL + i] = o[g][i];
        }
        __syncthreads();
        if (a.nsplit == 1) {  // the only split: normalise and store
            for (int idx = tid; idx < G * D; idx += 256) {
                const int g = idx / D, d = idx % D;
                const float s = (part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]);
                a.out[((int64_t)b * hq + h * G + g) * D + d] = s / stat[g][1];
            }
            return;
        }
        float* wr = a.ws + rec0 + (int64_t)split * G * (D + 2);
        for (int idx = tid; idx < G * D; idx += 256) {
            const int g = idx / D, d = idx % D;
            wr[g * (D + 2) + d] = (part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]);
        }
        if (tid < G) {
            wr[tid * (D + 2) + D] = stat[tid][0];
            wr[tid * (D + 2) + D + 1] = stat[tid][1];
        }
    }
}

// Merge of the split records of one (batch, kv head): the (max, sum) pairs of the active
// splits are read in parallel into LDS, then each output element sums its o_s in split order.
template <int D, int G>
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs a) {
    attn_args_prefetch(a);
    __shared__ float sm[G][ATT_MAX_SPLITS], sf[G][ATT_MAX_SPLITS], sden[G];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int64_t L = a.len.of(b);
    if (L > a.lmax) L = a.lmax;
    const int nact = (int)((L + a.chunk - 1) / a.chunk);
    const int64_t stride = (int64_t)G * (D + 2);
    const float* base = a.ws + (((int64_t)b * a.hkv + h) * a.nsplit) * stride;
    for (int idx = tid; idx < G * nact; idx += 256) {
        const int g = idx / nact, s = idx % nact;
        sm[g][s] = base[s * stride + g * (D + 2) + D];
        sf[g][s] = base[s * stride + g * (D + 2) + D + 1];
    }
    __syncthreads();
    // per head: M = max_s m_s, weights f_s = e^(m_s - M), den = sum_s l_s f_s
    for (int g = wave; g < G; g += 4) {
        float M = -INFINITY;
        for (int s = lane; s < nact; s += 64) M = fmaxf(M, sm[g][s]);
        M = wave_allmax(M);
        float den = 0.f;
        for (int s = lane; s < nact; s += 64) {
            const float f = expf(sm[g][s] - M);
            den = fmaf(sf[g][s], f, den);
            sm[g][s] = f;
        }
        den = wave_allsum(den);
        if (lane == 0) sden[g] = den;
    }
    __syncthreads();
    const int hq = a.hkv * G;
    for (int idx = tid; idx < G * D; idx += 256) {
        const int g = idx / D, d = idx % D;
        const float* r = base + g * (D + 2) + d;
        float num = 0.f;
#pragma unroll 4
        for (int s = 0; s < nact; s++) num = fmaf(r[s * stride], sm[g][s], num);
        a.out[((int64_t)b * hq + h * G + g) * D + d] = num / sden[g];
    }
}

// ---- shared helpers ---------------------------------------------------------------------
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = lane_pair_max<16>(v);  // permlane swaps: no LDS round trip
    v = lane_pair_max<32>(v);
    return v;
}
__device__ __forceinline__ float wave_sum64(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    v = lane_pair_sum<16>(v);
    v = lane_pair_sum<32>(v);
    return v;
}

template <typename KVT>
__device__ __forceinline__ void cvt8(const uint4& w, float* f);
template <>
__device__ __forceinline__ void cvt8<__half>(const uint4& w, float* f) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float2 t = __half22float2(*reinterpret_cast<const __half2*>(&u[j]));
        f[2 * j] = t.x;
        f[2 * j + 1] = t.y;
    }
}

// ---- grouped-query split form: one workgroup per (split of 128 positions, kv head, item) --
// Every K / V row of the split is read exactly once (coalesced: D/8 consecutive lanes share a
// row, 16 bytes each) and serves all G query heads of its KV head -- no per-head re-reads.
// The rows of a wavefront's 32 positions are requested at kernel start.
//   scores: lane (row r, slice kl) forms the partial dot products of its 8 dims with the G
//           q vectors for each of its rows; one transpose-reduce over the D/8 lanes of a row
//           leaves N / (D/8) finished scores per lane, which go to LDS;
//   softmax over the split's 128 positions per head (one wavefront per head);
//   P.V:    the same lanes accumulate p_g * v for their rows and all heads, then a second
//           transpose-reduce over the rows of the wavefront and an LDS sum over the four
//           wavefronts give the split's (o, max, sum) record; k_attn_merge combines splits
//           (a single split writes the output directly).
template <int OFF>
__device__ __forceinline__ float xchg_lo(float v) {  // partner across lane bit OFF within 16 lanes
    if constexpr (OFF == 8) return dpp_f<0x140>(v);      // row mirror (15 - i)
    else if constexpr (OFF == 4) return dpp_f<0x141>(v); // half-row mirror (7 - i)
    else if constexpr (OFF == 2) return dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]
    else return dpp_f<0xB1>(v);                          // quad_perm [1,0,3,2]
}
template <int OFF>
__device__ __forceinline__ float xchg_hi(float v) {  // exact xor of lane bit OFF (OFF >= 8)
    if constexpr (OFF == 8) return dpp_f<0x128>(v);  // row_ror:8 = xor 8 within 16 lanes
    else return lane_xor_f32<OFF>(v);                // permlane swaps
}

// Transpose-reduce of N values over the lanes that differ in lane bits LO .. OFF (powers of
// two, the first call's OFF the highest): each step sends half of the values across one bit
// and keeps the half its own bit selects.  Afterwards value j of the lane whose bits
// LO .. OFF read r holds the group sum of original value j + r * N / (2 OFF / LO).  Partners
// below 16 lanes apart may also differ in lower bits (the DPP mirrors): every lane of a
// group holds the same value indices when they exchange, so only the stepped bit matters.
template <int OFF, int LO, int H, int N, bool HIGH>
__device__ __forceinline__ void tr_halve(float (&v)[N], int lane) {
    const bool up = (lane & OFF) != 0;
#pragma unroll
    for (int i = 0; i < H; i++) {
        const float send = up ? v[i] : v[i + H];
        const float keep = up ? v[i + H] : v[i];
        if constexpr (HIGH) v[i] = keep + xchg_hi<OFF>(send);
        else v[i] = keep + xchg_lo<OFF>(send);
    }
    if constexpr (OFF > LO) tr_halve<OFF / 2, LO, H / 2, N, HIGH>(v, lane);
}

// PW positions per wavefront, 4 PW per workgroup (split).  FUSE false: the split records are
// merged by k_attn_merge_gq; true: the workgroup that completes the last split of a (batch
// item, KV head) merges them in the same launch.
template <int D, int G, int PW, bool FUSE>
__global__ __launch_bounds__(256) void k_attn_gq(AttnArgs a) {
    attn_args_prefetch(a);
    constexpr int GQ_PW = PW, GQ_CH = 4 * PW;
    constexpr int LPR = D / 8;          // lanes per row (16 bytes of f16 each)
    constexpr int RPI = 64 / LPR;       // rows per load instruction
    constexpr int NI = GQ_PW / RPI;     // load instructions per wavefront (K and V each)
    constexpr int NS = NI * G;          // partial scores per lane
    constexpr int NSL = NS / LPR;       // finished scores per lane
    constexpr int NO = G * 8;           // output partials per lane
    constexpr int NOL = NO / RPI;       // output sums per lane after the row reduction
    static_assert(NS % LPR == 0 && NO % RPI == 0, "shape");
    __shared__ float S[G][GQ_CH];
    __shared__ float stat[G][2];
    __shared__ float part[4][G][D];
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR
    const int kl = lane % LPR, kr = lane / LPR;
    int64_t L = a.len.of(b);
    if (L > a.lmax) L = a.lmax;
    const int64_t p0 = (int64_t)split * GQ_CH;
    if (p0 >= L) return;  // inactive split (uniform per workgroup)
    const int hq = a.hkv * G;
    const __half* kb = reinterpret_cast<const __half*>(a.k) + (int64_t)b * a.kv_bstride + (int64_t)h * a.lmax * D;
    const __half* vb = reinterpret_cast<const __half*>(a.v) + (int64_t)b * a.kv_bstride + (int64_t)h * a.lmax * D;

    uint4 kraw[NI], vraw[NI];
    const int64_t pw = p0 + wave * GQ_PW + kr;  // this lane's row of instruction 0
#pragma unroll
    for (int i = 0; i < NI; i++) {
        int64_t p = pw + i * RPI;
        p = p < L ? p : L - 1;
        kraw[i] = *reinterpret_cast<const uint4*>(kb + p * D + kl * 8);
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
        int64_t p = pw + i * RPI;
        p = p < L ? p : L - 1;
        vraw[i] = *reinterpret_cast<const uint4*>(vb + p * D + kl * 8);
    }
    float q[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float* qp = a.q + ((int64_t)b * hq + h * G + g) * D + kl * 8;
        const float4 t0 = reinterpret_cast<const float4*>(qp)[0], t1 = reinterpret_cast<const float4*>(qp)[1];
        q[g][0] = t0.x; q[g][1] = t0.y; q[g][2] = t0.z; q[g][3] = t0.w;
        q[g][4] = t1.x; q[g][5] = t1.y; q[g][6] = t1.z; q[g][7] = t1.w;
    }

    // scores
    {
        float sc[NS];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            float kf[8];
            cvt8<__half>(kraw[i], kf);
#pragma unroll
            for (int g = 0; g < G; g++) {
                float t = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) t = fmaf(q[g][e], kf[e], t);
                sc[i * G + g] = t;
            }
        }
        tr_halve<LPR / 2, 1, NS / 2, NS, false>(sc, lane);
#pragma unroll
        for (int j = 0; j < NSL; j++) {
            const int f = kl * NSL + j, i = f / G, g = f % G;
            const int pl = wave * GQ_PW + i * RPI + kr;  // position within the split
            S[g][pl] = p0 + pl < L ? sc[j] * a.scale : -INFINITY;
        }
    }
    __syncthreads();
    // softmax statistics of the split, one wavefront per head
    for (int g = wave; g < G; g += 4) {
        constexpr int PL = GQ_CH / 64;  // positions per lane
        float sv[PL], mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < PL; u++) {
            sv[u] = S[g][lane + 64 * u];
            mx = fmaxf(mx, sv[u]);
        }
        const float m = wave_max64(mx);  // position p0 is always valid: m is finite
        float es = 0.f;
#pragma unroll
        for (int u = 0; u < PL; u++) {
            sv[u] = expf(sv[u] - m);
            S[g][lane + 64 * u] = sv[u];
            es += sv[u];
        }
        const float l = wave_sum64(es);
        if (lane == 0) {
            stat[g][0] = m;
            stat[g][1] = l;
        }
    }
    __syncthreads();
    // P.V for this lane's rows and all heads
    float o[NO];
#pragma unroll
    for (int j = 0; j < NO; j++) o[j] = 0.f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        float vf[8];
        cvt8<__half>(vraw[i], vf);
        const int pl = wave * GQ_PW + i * RPI + kr;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float e = S[g][pl];
#pragma unroll
            for (int d = 0; d < 8; d++) o[g * 8 + d] = fmaf(e, vf[d], o[g * 8 + d]);
        }
    }
    tr_halve<32, LPR, NO / 2, NO, true>(o, lane);
#pragma unroll
    for (int j = 0; j < NOL; j++) {
        const int f = kr * NOL + j, g = f / 8, d = f % 8;
        part[wave][g][kl * 8 + d] = o[j];
    }
    __syncthreads();
    if (L <= GQ_CH) {  // the item's only split: normalise and store (the merge skips the item)
        for (int idx = tid; idx < G * D; idx += 256) {
            const int g = idx / D, d = idx % D;
            const float v = (part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]);
            a.out[((int64_t)b * hq + h * G + g) * D + d] = v / stat[g][1];
        }
        return;
    }
    float* wr = a.ws + (((int64_t)b * a.hkv + h) * a.nsplit + split) * G * (D + 2);
    if constexpr (!FUSE) {  // record [G][D + 2]: o, then max and sum, per head
        for (int idx = tid; idx < G * D; idx += 256) {
            const int g = idx / D, d = idx % D;
            wr[g * (D + 2) + d] = (part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]);
        }
        if (tid < G) {
            wr[tid * (D + 2) + D] = stat[tid][0];
            wr[tid * (D + 2) + D + 1] = stat[tid][1];
        }
    } else {
        // Record [G][D] of o, then [G] (max, sum) pairs, 16-byte aligned (G (D + 2) floats per
        // split), written with the agent-coherent cache policy (through to the agent's point
        // of coherence) in 16-byte stores.
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(wr, G * (D + 2) * 4);
        for (int u = tid; u < G * D / 4; u += 256) {
            const int g = 4 * u / D, d = 4 * u % D;
            u32x4 v;
            v.x = __float_as_uint((part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]));
            v.y = __float_as_uint((part[0][g][d + 1] + part[1][g][d + 1]) + (part[2][g][d + 1] + part[3][g][d + 1]));
            v.z = __float_as_uint((part[0][g][d + 2] + part[1][g][d + 2]) + (part[2][g][d + 2] + part[3][g][d + 2]));
            v.w = __float_as_uint((part[0][g][d + 3] + part[1][g][d + 3]) + (part[2][g][d + 3] + part[3][g][d + 3]));
            __builtin_amdgcn_raw_buffer_store_b128(v, rw, 16 * u, 0, CPOL_SC1);
        }
        if (tid < G) {
            const u32x2 ml = {__float_as_uint(stat[tid][0]), __float_as_uint(stat[tid][1])};
            __builtin_amdgcn_raw_buffer_store_b64(ml, rw, 4 * (G * D + 2 * tid), 0, CPOL_SC1);
        }
        // Arrival.  Every wave waits until its record stores have completed (reached the
        // agent's point of coherence) before the barrier, so the counter is bumped only once
        // the whole record is visible to every XCD: the release order of an agent-scope
        // fence without its L2 write-back, which only plain stores need.  The last arriver
        // reads the records with the same cache policy, issued after its bump has returned.
        __shared__ int s_last;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // splits holding positions; the grid has a.nsplit <= ATT_FUSE_MAX of them
        const int nact = (int)min((L + GQ_CH - 1) / GQ_CH, (int64_t)a.nsplit);
        if (tid == 0) {
            uint32_t* c = g_attn_arrive + ((int64_t)b * a.hkv + h);
            const uint32_t old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == (uint32_t)(nact - 1);
            if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;  // uniform per workgroup
        // Merge of the nact records: out = sum_s o_s w_s / sum_s l_s w_s, w_s = e^(m_s - max m).
        // A thread takes four consecutive outputs of one head and requests their o values and
        // the head's (max, sum) of every split at once (records past nact lie beyond the
        // resource's range and read 0; the selects drop them).
        constexpr int RB = G * (D + 2) * 4;  // bytes per split record
        const float* rb = a.ws + (((int64_t)b * a.hkv + h) * a.nsplit) * G * (D + 2);
        const __amdgpu_buffer_rsrc_t rr = buf_rsrc(rb, (uint32_t)(nact * RB));
        const int hq = a.hkv * G;
        for (int u = tid; u < G * D / 4; u += 256) {
            const int g = 4 * u / D, d = 4 * u % D;
            u32x4 o[ATT_FUSE_MAX];
            u32x2 ml[ATT_FUSE_MAX];
#pragma unroll
            for (int sp = 0; sp < ATT_FUSE_MAX; sp++) {
                o[sp] = __builtin_amdgcn_raw_buffer_load_b128(rr, 16 * u, sp * RB, CPOL_SC1);
                ml[sp] = __builtin_amdgcn_raw_buffer_load_b64(rr, 4 * (G * D + 2 * g), sp * RB, CPOL_SC1);
            }
            float M = __uint_as_float(ml[0].x);  // split 0 always holds positions
#pragma unroll
            for (int sp = 1; sp < ATT_FUSE_MAX; sp++) M = sp < nact ? fmaxf(M, __uint_as_float(ml[sp].x)) : M;
            float den = 0.f;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int sp = 0; sp < ATT_FUSE_MAX; sp++) {
                const float e = sp < nact ? expf(__uint_as_float(ml[sp].x) - M) : 0.f;
                den = fmaf(__uint_as_float(ml[sp].y), e, den);
                acc.x = fmaf(__uint_as_float(o[sp].x), e, acc.x);
                acc.y = fmaf(__uint_as_float(o[sp].y), e, acc.y);
                acc.z = fmaf(__uint_as_float(o[sp].z), e, acc.z);
                acc.w = fmaf(__uint_as_float(o[sp].w), e, acc.w);
            }
            const float rd = 1.0f / den;
            *reinterpret_cast<float4*>(a.out + ((int64_t)b * hq + h * G + g) * D + d) =
                make_float4(acc.x * rd, acc.y * rd, acc.z * rd, acc.w * rd);
        }
    }
}

// ---- short-cache form: one workgroup per (query head, batch item) ------------------------
// W wavefronts each take 64 consecutive positions per round (W * 64 per round, one round
// for the decode lengths it is used for).  K rows are read coalesced: LPR consecutive lanes
// share a row (16 bytes each), so one load instruction covers 64 / LPR whole rows; the score
// of a position is the LPR-lane sum of the partial dot products.  V rows are read by lane
// (dim group dg = lane / 8, position slot = lane % 8), eight full rows per instruction.
// Scores pass to the P.V lanes through LDS; each lane turns one of them into a probability
// (scores kept in log2 units, so one hardware exp2 per lane and round).  Softmax is online
// across rounds; the wavefronts' (max, sum, o) records are merged through LDS at the end, with
// the per-wavefront weights formed once.  All arithmetic f32.
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {  // over aligned groups of LPR lanes
    static_assert(LPR == 8 || LPR == 16 || LPR == 32, "row width");
    v += dpp_f<0xB1>(v);   // xor 1
    v += dpp_f<0x4E>(v);   // xor 2
    v += dpp_f<0x141>(v);  // half-row mirror: the other four of the eight
    if constexpr (LPR >= 16) v += dpp_f<0x140>(v);  // row mirror: the other eight of sixteen
    if constexpr (LPR >= 32) v = lane_pair_sum<16>(v);
    return v;
}

template <typename KVT>
__device__ __forceinline__ void cvt16(const uint4& w, float* f);  // 16 bytes -> floats
template <>
__device__ __forceinline__ void cvt16<__half>(const uint4& w, float* f) {
    cvt8<__half>(w, f);
}
template <>
__device__ __forceinline__ void cvt16<float>(const uint4& w, float* f) {
    f[0] = __uint_as_float(w.x);
    f[1] = __uint_as_float(w.y);
    f[2] = __uint_as_float(w.z);
    f[3] = __uint_as_float(w.w);
}

// The arguments the first loads need lead, as scalars and pointers preloaded into SGPRs at
// dispatch (14 dwords: the KV-head count, G and the share count share one); the rest of AttnArgs (the split
// record buffer, the output, the score scale, the host length) is loaded from the argument
// buffer while the first K / V loads are in flight.
template <int D, typename KVT, int W>
__global__ __launch_bounds__(64 * W) void k_attn_qh(const float* __restrict__ q_p, const void* __restrict__ k_p,
                                                    const void* __restrict__ v_p, const int32_t* __restrict__ len_dev,
                                                    int64_t kv_bstride, int lmax_p, uint32_t hkv_g, int len_add,
                                                    int len_step, AttnArgs a) {
    a.q = q_p;
    a.k = k_p;
    a.v = v_p;
    a.kv_bstride = kv_bstride;
    a.lmax = lmax_p;
    a.hkv = (int)(hkv_g & 0xffffu);
    a.len.len_dev = len_dev;
    a.len.len_add = len_add;
    a.len.len_step = len_step;
    const int G = (int)((hkv_g >> 16) & 0xffu);
    const uint32_t ns = hkv_g >> 24;  // = gridDim.z, without a load of the dispatch packet
    constexpr int C = 64;                  // positions per wavefront and round
    constexpr int EPC = 16 / sizeof(KVT);  // elements per 16-byte load
    constexpr int LPR = D / EPC;           // lanes per K row
    constexpr int PPI = 64 / LPR;          // K rows per load instruction
    constexpr int NI = C / PPI;            // K load instructions per round (= LPR)
    constexpr int DL = D / 8;              // dims per lane in P.V
    constexpr int VC = DL / EPC;           // 16-byte loads of a lane's V slice
    static_assert(NI == LPR, "one score per lane and round");
    __shared__ float P[W][C];
    __shared__ float wm[W], wl[W], wf[W];
    __shared__ float wo[W][D];
    const int qh = blockIdx.x, b = blockIdx.y;
    const int h = qh / G;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR
    const int kl = lane % LPR, kr = lane / LPR;  // K: slice and row within an instruction
    const int slot = lane & 7, dg = lane >> 3;   // V: position slot and dim group
    const int hq = a.hkv * G;
    const float* qp = a.q + ((int64_t)b * hq + qh) * D;
    float qv[EPC];  // this lane's slice of q, requested before the cached length is known
#pragma unroll
    for (int e = 0; e < EPC; e += 4) {
        const float4 t = *reinterpret_cast<const float4*>(qp + kl * EPC + e);
        qv[e] = t.x;
        qv[e + 1] = t.y;
        qv[e + 2] = t.z;
        qv[e + 3] = t.w;
    }
    int64_t L64 = a.len.of(b);
    if (L64 > a.lmax) L64 = a.lmax;
    const uint32_t L = (uint32_t)L64;  // lmax * D < 2^31 (attention_qh_supported): 32-bit offsets
    // gridDim.z > 1: this workgroup covers positions [p0, p1), a share of whole rounds (the
    // first share is never empty), and leaves an unnormalised partial record
    uint32_t p0 = 0, p1 = L;
    if (ns > 1) {
        const uint32_t per = ((L + ns - 1) / ns + C - 1) / C * C;
        p0 = blockIdx.z * per < L ? blockIdx.z * per : L;
        p1 = p0 + per < L ? p0 + per : L;
    }
    const KVT* kb = reinterpret_cast<const KVT*>(a.k) + (int64_t)b * a.kv_bstride + (int64_t)h * a.lmax * D;
    const KVT* vb = reinterpret_cast<const KVT*>(a.v) + (int64_t)b * a.kv_bstride + (int64_t)h * a.lmax * D;
    const float sl2 = a.scale * 1.44269504088896341f;  // scores in log2 units: exp(x) = exp2(x log2 e)
    float m = -INFINITY, l = 0.f, o[DL];
#pragma unroll
    for (int i = 0; i < DL; i++) o[i] = 0.f;

    for (uint32_t base = p0 + (uint32_t)wave * C; base < p1; base += (uint32_t)W * C) {
        uint4 kraw[NI], vraw[8][VC];
#pragma unroll
        for (int c = 0; c < NI; c++) {
            uint32_t p = base + c * PPI + kr;
            p = p < p1 ? p : p1 - 1;
            kraw[c] = *reinterpret_cast<const uint4*>(kb + p * D + kl * EPC);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t p = base + slot + 8 * j;
            p = p < p1 ? p : p1 - 1;
#pragma unroll
            for (int c = 0; c < VC; c++) vraw[j][c] = reinterpret_cast<const uint4*>(vb + p * D + dg * DL)[c];
        }
        // scores: position base + c * PPI + kr lives in register s[c] of its LPR lanes
        float s[NI];
#pragma unroll
        for (int c = 0; c < NI; c++) {
            float kf[EPC];
            cvt16<KVT>(kraw[c], kf);
            float t = 0.f;
#pragma unroll
            for (int e = 0; e < EPC; e++) t = fmaf(qv[e], kf[e], t);
            s[c] = row_sum<LPR>(t) * sl2;
        }
        // one probability per lane: lane kl of a row group takes position base + kl * PPI + kr
        float sk = s[0];
#pragma unroll
        for (int c = 1; c < NI; c++) sk = kl == c ? s[c] : sk;
        const bool in = base + kl * PPI + kr < p1;
        const float mn = fmaxf(m, wave_max64(in ? sk : -INFINITY));  // position base is valid: finite
        const float pk = in ? __builtin_amdgcn_exp2f(sk - mn) : 0.f;
        const float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first round (m = -inf)
        l = l * alpha + wave_sum64(pk);
        m = mn;
        P[wave][kl * PPI + kr] = pk;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < DL; i++) o[i] *= alpha;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float pj = P[wave][slot + 8 * j];
            float vf[DL];
#pragma unroll
            for (int c = 0; c < VC; c++) cvt16<KVT>(vraw[j][c], vf + c * EPC);
#pragma unroll
            for (int i = 0; i < DL; i++) o[i] = fmaf(pj, vf[i], o[i]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int i = 0; i < DL; i++) o[i] = sum8_dpp(o[i]);
    if (slot == 0) {
#pragma unroll
        for (int i = 0; i < DL; i++) wo[wave][dg * DL + i] = o[i];
    }
    if (lane == 0) {
        wm[wave] = m;
        wl[wave] = l;
    }
    __syncthreads();
    // record of a split: [o (D floats, relative to M) | M | l | 0 | 0], D + 4 floats
    float* rec = ns > 1 ? a.ws + (((int64_t)b * hq + qh) * ns + blockIdx.z) * (D + 4) : nullptr;
    if (wave == 0) {  // per-wavefront weights exp2(m_w - M) / sum_w l_w exp2(m_w - M)
        const bool act = lane < W && wl[lane < W ? lane : 0] > 0.f;  // idle wavefronts add nothing
        const float mw = act ? wm[lane] : -INFINITY;
        const float M = wave_max64(mw);  // -inf for an empty share: every weight 0, l = 0
        const float f = act ? __builtin_amdgcn_exp2f(mw - M) : 0.f;
        const float den = wave_sum64(act ? f * wl[lane] : 0.f);
        if (lane < W) wf[lane] = rec ? f : f / den;
        if (rec && lane == 0) {
            st_wt(rec + D, M);
            st_wt(rec + D + 1, den);
            st_wt(rec + D + 2, 0.f);
            st_wt(rec + D + 3, 0.f);
        }
    }
    __syncthreads();
    for (int d = tid; d < D; d += 64 * W) {
        float num = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) num = fmaf(wo[w][d], wf[w], num);
        if (rec) st_wt(rec + d, num);
        else st_wt(a.out + ((int64_t)b * hq + qh) * D + d, num);
    }
}

// ---- causal prefill form (f16 cache, f16 MFMA): one workgroup per (block of queries, KV head,
// head half).  The workgroup's 128 / HS rows are (query, head) pairs of its QB = 128 / G
// queries and G / HS of the KV head's G heads; wavefront w owns RT = 2 / HS 16-row tiles
// (HS = 2: twice the workgroups, each KV tile staged by both halves).  Per 64-position
// KV tile (K row-major, V transposed, both in LDS):
//   S^T = K Q^T   (v_mfma_f32_16x16x32_f16: A = K rows from LDS, B = q from registers), so a
//                 lane holds row l % 16's scores for positions 4 (l / 16) .. +3 of each
//                 16-position block -- every per-row quantity stays in the lane that owns it;
//   online softmax per row (the row's 64 scores sit in the four lanes l % 16 + 16 g);
//   O^T += V^T P^T with the k slots ordered as the scores already lie in the lanes
//                 (slot group g, element e <-> position 32 ks + 16 (e / 4) + 4 g + e % 4),
//                 so P never leaves the registers; V^T is read as two 8-byte runs.
// Query i of the call sits at position pos0 + i and attends positions 0 .. pos0 + i.  Scores,
// softmax and accumulation in f32; q, P, K, V enter the MFMAs in f16 (the f16 path).
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float floatx4v __attribute__((ext_vector_type(4)));

template <int D, int G, int HS>
__global__ __launch_bounds__(256) void k_attn_prefill(const float* __restrict__ q, const __half* __restrict__ kc,
                                                      const __half* __restrict__ vc, float* __restrict__ out,
                                                      int n, int hkv, int64_t lmax, const int32_t* __restrict__ pos_dev,
                                                      int64_t pos_host, float scale, _Float16* __restrict__ out16,
                                                      int order) {
    // arguments in one round of scalar loads (left to the compiler: three dependent rounds)
    asm volatile("" : : "s"(q), "s"(kc), "s"(vc), "s"(out), "s"(n), "s"(hkv), "s"(lmax), "s"(pos_dev), "s"(pos_host),
                 "s"(scale), "s"(out16), "s"(order));
    constexpr int QB = 128 / G;   // queries per workgroup
    constexpr int GH = G / HS;    // heads per workgroup
    constexpr int RT = 2 / HS;    // 16-row tiles per wavefront
    constexpr int KT = 64;        // positions per KV tile
    constexpr int KS = D / 32;    // MFMA k-steps over the head dim
    constexpr int CPR = D / 8;    // 16-byte chunks per K row
    __shared__ __attribute__((aligned(16))) _Float16 Ks[KT * D];  // row-major, chunk c of row r at c ^ (r & (CPR - 1))
    __shared__ __attribute__((aligned(16))) _Float16 Vt[D * KT];  // [dim][pos], 8-byte run j of dim d at j ^ (d & 15)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR
    const int col = lane & 15, g = lane >> 4;
    const int qb = blockIdx.x, h = blockIdx.y / HS, hs = blockIdx.y % HS;
    const int hq = hkv * G;
    const int64_t pos0 = pos_dev ? (int64_t)*pos_dev : pos_host;
    const __half* kb = kc + (int64_t)h * lmax * D;
    const __half* vb = vc + (int64_t)h * lmax * D;

    // this lane's rows (one per 16-row tile): query qi, head hh
    int qi[RT], hh[RT];
    int64_t prow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = 16 * RT * wave + 16 * rt + col;
        qi[rt] = qb * QB + r / GH;
        hh[rt] = h * G + hs * GH + r % GH;
        prow[rt] = pos0 + (qi[rt] < n ? qi[rt] : n - 1);
    }
    // B operand of S^T: q[row][32 ks + 8 g .. +7] * scale * log2(e), in f16: scores in log2
    // units, so the softmax exponentials are single hardware exp2 instructions
    const float sl2 = scale * 1.44269504088896341f;
    half8v qop[RT][KS];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int qq = qi[rt] < n ? qi[rt] : n - 1;
        const float* qp = q + ((int64_t)qq * hq + hh[rt]) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const float4 a = reinterpret_cast<const float4*>(qp + 32 * ks + 8 * g)[0];
            const float4 b = reinterpret_cast<const float4*>(qp + 32 * ks + 8 * g)[1];
            qop[rt][ks] = half8v{(_Float16)(a.x * sl2), (_Float16)(a.y * sl2), (_Float16)(a.z * sl2),
                                 (_Float16)(a.w * sl2), (_Float16)(b.x * sl2), (_Float16)(b.y * sl2),
                                 (_Float16)(b.z * sl2), (_Float16)(b.w * sl2)};
        }
    }
    floatx4v o[RT][D / 16];  // O^T tiles: [row tile][dim tile], lane: dims 4 g .. +3 of row col
    float mrow[RT], lrow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) o[rt][dt] = floatx4v{0.f, 0.f, 0.f, 0.f};
        mrow[rt] = -INFINITY;
        lrow[rt] = 0.f;
    }

    const int64_t last = pos0 + (int64_t)((qb + 1) * QB < n ? (qb + 1) * QB : n);  // positions needed
    const int ntiles = (int)((last + KT - 1) / KT);
    // K / V tile rows as raw 16-byte chunks, one tile ahead: the loads of tile + 1 are in
    // flight while tile computes.  Rows at or past `last` are zeros: they are masked out, and
    // a zero P times a non-finite V would still poison O.
    constexpr int TU = KT * CPR / 256;  // chunks per thread and tile
    uint4 kn[TU], vn[TU];
    auto fetch = [&](int tile) {
#pragma unroll
        for (int i = 0; i < TU; i++) {
            const int u = tid + 256 * i, r = u / CPR, c = u % CPR;
            const int64_t p = (int64_t)tile * KT + r;
            kn[i] = vn[i] = make_uint4(0u, 0u, 0u, 0u);
            if (p < last) {
                kn[i] = *reinterpret_cast<const uint4*>(kb + p * D + 8 * c);
                vn[i] = *reinterpret_cast<const uint4*>(vb + p * D + 8 * c);
            }
        }
    };
    fetch(0);
    for (int tile = 0; tile < ntiles; tile++) {
        const int64_t t0 = (int64_t)tile * KT;
        __syncthreads();  // the previous tile's readers are done
        // K tile row-major (chunk swizzle), V tile transposed into Vt
#pragma unroll
        for (int i = 0; i < TU; i++) {
            const int u = tid + 256 * i, r = u / CPR, c = u % CPR;
            *reinterpret_cast<uint4*>(&Ks[r * D + 8 * (c ^ (r & (CPR - 1)))]) = kn[i];
            const _Float16* vh = reinterpret_cast<const _Float16*>(&vn[i]);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int d = 8 * c + e;
                Vt[d * KT + 4 * ((r >> 2) ^ (d & 15)) + (r & 3)] = vh[e];
            }
        }
        if (tile + 1 < ntiles) fetch(tile + 1);
        __syncthreads();
        // S^T = K Q^T over the tile: [pos tile pt][row tile rt]
        floatx4v st[4][RT];
#pragma unroll
        for (int pt = 0; pt < 4; pt++)
#pragma unroll
            for (int rt = 0; rt < RT; rt++) st[pt][rt] = floatx4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pt = 0; pt < 4; pt++) {
            const int r = 16 * pt + col;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const int c = 4 * ks + g;
                const half8v a = *reinterpret_cast<const half8v*>(&Ks[r * D + 8 * (c ^ (r & (CPR - 1)))]);
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
                    st[pt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qop[rt][ks], st[pt][rt], 0, 0, 0);
            }
        }
        // causal mask, online softmax per row (row col's scores: this lane and lanes col + 16 g)
        half8v pop[2][RT];  // B operand of O^T: [k-step][row tile]
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            float mx = -INFINITY;
#pragma unroll
            for (int pt = 0; pt < 4; pt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int64_t p = t0 + 16 * pt + 4 * g + i;
                    if (p > prow[rt]) st[pt][rt][i] = -INFINITY;
                    mx = fmaxf(mx, st[pt][rt][i]);
                }
            mx = lane_pair_max<16>(mx);
            mx = lane_pair_max<32>(mx);
            const float mn = fmaxf(mrow[rt], mx);  // finite: position 0 is in every row's range
            const float alpha = __builtin_amdgcn_exp2f(mrow[rt] - mn);  // 0 on the first tile
            float sum = 0.f;
#pragma unroll
            for (int pt = 0; pt < 4; pt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float e = __builtin_amdgcn_exp2f(st[pt][rt][i] - mn);  // 0 for masked
                    st[pt][rt][i] = e;
                    sum += e;
                }
            sum = lane_pair_sum<16>(sum);
            sum = lane_pair_sum<32>(sum);
            lrow[rt] = lrow[rt] * alpha + sum;
            mrow[rt] = mn;
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++) o[rt][dt] *= alpha;
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) pop[ks][rt][e] = (_Float16)st[2 * ks + e / 4][rt][e % 4];
        }
        // O^T += V^T P^T: A = V^T[dim tile][k slots], two 8-byte runs per k-step
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
            const int d = 16 * dt + col;
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const int j0 = (8 * ks + g) ^ (d & 15), j1 = (8 * ks + 4 + g) ^ (d & 15);
                const uint2 lo = *reinterpret_cast<const uint2*>(&Vt[d * KT + 4 * j0]);
                const uint2 hi = *reinterpret_cast<const uint2*>(&Vt[d * KT + 4 * j1]);
                const half8v a = __builtin_bit_cast(half8v, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
                    o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pop[ks][rt], o[rt][dt], 0, 0, 0);
            }
        }
    }
    // out[query][head][dims 16 dt + 4 g .. +3] = O / l, f32 or (out16) f16 in the operand order
    // of the GEMM that reads the [n, hq D] rows
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        if (qi[rt] >= n) continue;
        const float rl = 1.0f / lrow[rt];
        if (out16) {
            // o / l rounded to f32 and then to f16 for every element: the product is pinned in a
            // register first -- left alone, the compiler fuses some of these conversions into
            // one-rounding mixed FMAs (v_fma_mix) and not others, depending on the instantiation.
            // The lane's four dims 4 g .. 4 g + 3 (a 4-aligned run) fill slots s .. s + 3 of one
            // operand word in either order (Q4: in order; Q8: as e0 e2 e1 e3): one 8-byte store.
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++) {
                _Float16 h[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float v = o[rt][dt][i] * rl;
                    asm volatile("" : "+v"(v));
                    h[i] = (_Float16)v;
                }
                const int64_t at = f16q_index(qi[rt], (int64_t)hh[rt] * D + 16 * dt + 4 * g, (int64_t)hq * D, order);
                typedef _Float16 half4v __attribute__((ext_vector_type(4)));
                *reinterpret_cast<half4v*>(out16 + at) =
                    order == F16Q_Q8 ? half4v{h[0], h[2], h[1], h[3]} : half4v{h[0], h[1], h[2], h[3]};
            }
        } else {
            float* op = out + ((int64_t)qi[rt] * hq + hh[rt]) * D;
#pragma unroll
            for (int dt = 0; dt < D / 16; dt++)
                *reinterpret_cast<float4*>(op + 16 * dt + 4 * g) =
                    make_float4(o[rt][dt][0] * rl, o[rt][dt][1] * rl, o[rt][dt][2] * rl, o[rt][dt][3] * rl);
        }
    }
}

bool attention_prefill_supported(int kv_dtype, int hq, int hkv, int D) {
    const int G = hkv > 0 ? hq / hkv : 0;
    return kv_dtype == TL_HIP_F16 && (D == 64 || D == 128) && (G == 4 || G == 8) && hq == G * hkv;
}

int launch_attention_prefill(const float* q, const void* k, const void* v, float* out, int n, int hq, int hkv,
                             int D, int64_t lmax, const int32_t* pos_dev, int64_t pos_host, float scale,
                             hipStream_t s, _Float16* out16, int order) {
    const int G = hq / hkv;
    if (n < 1) return TL_HIP_OK;
    constexpr int HS = 2;  // head halves per KV head: one 16-row tile per wavefront
    if (hkv > 65535 / HS) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: prefill attention takes at most %d KV heads", 65535 / HS);
        return TL_HIP_ERR_ARG;
    }
    dim3 grid((unsigned)cdiv(n, 128 / G), hkv * HS);
    const __half* kh = static_cast<const __half*>(k);
    const __half* vh = static_cast<const __half*>(v);
    if (D == 64 && G == 8) k_attn_prefill<64, 8, HS><<<grid, 256, 0, s>>>(q, kh, vh, out, n, hkv, lmax, pos_dev, pos_host, scale, out16, order);
    else if (D == 64 && G == 4) k_attn_prefill<64, 4, HS><<<grid, 256, 0, s>>>(q, kh, vh, out, n, hkv, lmax, pos_dev, pos_host, scale, out16, order);
    else if (D == 128 && G == 8) k_attn_prefill<128, 8, HS><<<grid, 256, 0, s>>>(q, kh, vh, out, n, hkv, lmax, pos_dev, pos_host, scale, out16, order);
    else if (D == 128 && G == 4) k_attn_prefill<128, 4, HS><<<grid, 256, 0, s>>>(q, kh, vh, out, n, hkv, lmax, pos_dev, pos_host, scale, out16, order);
    else {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: prefill attention covers f16 caches, head_dim 64 / 128, 4 or 8 query "
                  "heads per KV head");
        return TL_HIP_ERR_ARG;
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "prefill attention launch");
}

bool attention_qh_supported(int kv_dtype, int D, int64_t lmax) {
    return ((kv_dtype == TL_HIP_F16 && (D == 64 || D == 128)) || (kv_dtype == TL_HIP_F32 && D == 64)) &&
           lmax * D < (int64_t(1) << 31);
}

// Short-cache form; returns TL_HIP_ERR_ARG (no launch) for shapes it does not cover.
int launch_attention_qh(const float* q, const void* k, const void* v, int kv_dtype, float* out,
                        int B, int hq, int hkv, int D, int64_t lmax, int64_t kv_bstride, int64_t L,
                        const int32_t* len_dev, int len_add, int len_step, float scale, hipStream_t s,
                        float* part, int nsplit) {
    if (nsplit < 1 || nsplit > 8 || (nsplit > 1 && !part)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: %d position shares per head (1..8, >1 with a record buffer)", nsplit);
        return TL_HIP_ERR_ARG;
    }
    AttnArgs a{q, k, v, out, part, hkv, lmax, kv_bstride, AttnLen{L, len_dev, len_add, len_step}, 64, nsplit,
               scale};
    const int G = hq / hkv;
    if (hkv < 1 || hkv > 0xffff || G < 1 || G > 0xff || lmax > INT32_MAX) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: short-cache attention: %d KV heads, %d query heads each, %lld cached "
                  "positions", hkv, G, (long long)lmax);
        return TL_HIP_ERR_ARG;
    }
    dim3 grid(hq, B, nsplit);
    // a workgroup with a share of the positions has fewer rounds for its wavefronts: 4 of them
    const bool w4 = nsplit > 1;
    const uint32_t hkv_g = (uint32_t)hkv | (uint32_t)G << 16 | (uint32_t)nsplit << 24;
#define TLH_QH(DD, T, WW)                                                                                     \
    k_attn_qh<DD, T, WW><<<grid, 64 * WW, 0, s>>>(q, k, v, len_dev, kv_bstride, (int)lmax, hkv_g, len_add, len_step, a)
    if (D == 64 && kv_dtype == TL_HIP_F16) {
        if (w4) TLH_QH(64, __half, 4);
        else TLH_QH(64, __half, 8);
    } else if (D == 128 && kv_dtype == TL_HIP_F16) {
        if (w4) TLH_QH(128, __half, 4);
        else TLH_QH(128, __half, 8);
    } else if (D == 64 && kv_dtype == TL_HIP_F32) {
        if (w4) TLH_QH(64, float, 4);
        else TLH_QH(64, float, 8);
    } else {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: short-cache attention covers head_dim 64 / 128 (f16 cache) and 64 (f32)");
        return TL_HIP_ERR_ARG;
    }
#undef TLH_QH
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "attention launch");
}

// Split plan: about 1024 workgroups over (B x Hkv x splits); chunks a multiple of 32 and at
// most ATT_MAX_CHUNK positions.
void attn_plan(int B, int hkv, int64_t L, int* chunk, int* nsplit) {
    int64_t pairs = (int64_t)B * hkv;
    int64_t want = (1024 + pairs - 1) / pairs;
    int64_t c = (L + want - 1) / want;
    if (c < 64) c = 64;
    c = (c + 31) / 32 * 32;
    if (c > ATT_MAX_CHUNK) c = ATT_MAX_CHUNK;
    *chunk = (int)c;
    *nsplit = (int)((L + c - 1) / c);
    while (*nsplit > ATT_MAX_SPLITS) {  // very long caches: widen the chunk
        c += 32;
        *nsplit = (int)((L + c - 1) / c);
    }
}

size_t attn_workspace_floats(int B, int hkv, int G, int D, int nsplit) {
    return (size_t)B * hkv * nsplit * G * (D + 2);
}

template <typename KVT>
static int attn_dispatch(const AttnArgs& a, int B, int hq, int D, hipStream_t s) {
    const int G = hq / a.hkv;
    dim3 grid(a.nsplit, a.hkv, B);
#define TLH_ATT(DD, GG)                                                          \
    if (D == DD && G == GG) {                                                    \
        k_attn<DD, GG, KVT><<<grid, 256, 0, s>>>(a);                             \
        if (a.nsplit > 1) k_attn_merge<DD, GG><<<dim3(a.hkv, B), 256, 0, s>>>(a); \
        hipError_t e = hipGetLastError();                                        \
        return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "attention launch");    \
    }
    TLH_ATT(128, 1) TLH_ATT(128, 2) TLH_ATT(128, 4) TLH_ATT(128, 8)
    TLH_ATT(64, 1) TLH_ATT(64, 2) TLH_ATT(64, 4) TLH_ATT(64, 8)
#undef TLH_ATT
    set_error(TL_HIP_ERR_ARG, "ArgumentError: attention supports head_dim 64/128 and 1, 2, 4 or 8 "
              "query heads per KV head (got D=%d, group %d)", D, G);
    return TL_HIP_ERR_ARG;
}

// Merge of the split records of one (batch, kv head, query head): 256 threads = D/4 float4
// columns x (1024 / D) split groups.  Every thread requests the o, max and sum entries of its
// splits at once (one memory round trip), the global max and the sums over split groups go
// through LDS.  out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M).
template <int D, int G>
__global__ __launch_bounds__(256) void k_attn_merge_gq(AttnArgs a) {
    attn_args_prefetch(a);
    constexpr int NC = D / 4, NG = 256 / NC;  // float4 columns, split groups
    constexpr int U = 8;                       // splits per thread held in registers
    __shared__ float4 acc[NG][NC];
    __shared__ float smax[NG], sden[NG];
    const int h = blockIdx.x, b = blockIdx.y, g = blockIdx.z, tid = threadIdx.x;
    const int col = tid % NC, grp = tid / NC;
    int64_t L = a.len.of(b);
    if (L > a.lmax) L = a.lmax;
    const int nact = (int)((L + a.chunk - 1) / a.chunk);
    if (nact <= 1) return;  // written by its only split
    const int64_t stride = (int64_t)G * (D + 2);
    const float* base = a.ws + (((int64_t)b * a.hkv + h) * a.nsplit) * stride + g * (D + 2);
    float M = -INFINITY;
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    float den = 0.f;
    // this thread's splits: grp, grp + NG, ... in passes of U (one pass up to U * NG splits)
    for (int s0 = grp; s0 < nact; s0 += U * NG) {
        float4 ov[U];
        float mv[U], lv[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int sp = s0 + u * NG;
            if (sp < nact) {
                ov[u] = *reinterpret_cast<const float4*>(base + sp * stride + 4 * col);
                mv[u] = base[sp * stride + D];
                lv[u] = base[sp * stride + D + 1];
            } else {
                ov[u] = make_float4(0.f, 0.f, 0.f, 0.f);
                mv[u] = -INFINITY;
                lv[u] = 0.f;
            }
        }
        float mp = M;
#pragma unroll
        for (int u = 0; u < U; u++) mp = fmaxf(mp, mv[u]);
        const float r = M == -INFINITY ? 0.f : expf(M - mp);  // rescale the earlier passes
        num.x *= r;
        num.y *= r;
        num.z *= r;
        num.w *= r;
        den *= r;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float w = mv[u] == -INFINITY ? 0.f : expf(mv[u] - mp);
            num.x = fmaf(ov[u].x, w, num.x);
            num.y = fmaf(ov[u].y, w, num.y);
            num.z = fmaf(ov[u].z, w, num.z);
            num.w = fmaf(ov[u].w, w, num.w);
            den = fmaf(lv[u], w, den);
        }
        M = mp;
    }
    if (col == 0) smax[grp] = M;
    __syncthreads();
    float Mall = -INFINITY;
#pragma unroll
    for (int q = 0; q < NG; q++) Mall = fmaxf(Mall, smax[q]);
    const float r = M == -INFINITY ? 0.f : expf(M - Mall);  // groups without splits add nothing
    acc[grp][col] = make_float4(num.x * r, num.y * r, num.z * r, num.w * r);
    if (col == 0) sden[grp] = den * r;
    __syncthreads();
    if (grp == 0) {
        float4 t = acc[0][col];
        float dd = sden[0];
#pragma unroll
        for (int q = 1; q < NG; q++) {
            const float4 v = acc[q][col];
            t.x += v.x;
            t.y += v.y;
            t.z += v.z;
            t.w += v.w;
            dd += sden[q];
        }
        const float rd = 1.0f / dd;
        const int hq = a.hkv * G;
        float4* o = reinterpret_cast<float4*>(a.out + ((int64_t)b * hq + h * G + g) * D) + col;
        *o = make_float4(t.x * rd, t.y * rd, t.z * rd, t.w * rd);
    }
}

// Grouped-query split form + merge; shapes as attention_gq_supported.  nsplit = splits of
// 128 positions the grid covers (attention_gq_splits of the longest length); ws holds
// 2 * nsplit records, since the launch halves the split size when the grid would be small.
int launch_attention_gq(const float* q, const void* k, const void* v, float* out, float* ws, int B, int hq,
                        int hkv, int D, int64_t lmax, int64_t kv_bstride, int64_t L, const int32_t* len_dev,
                        int len_add, int len_step, int nsplit, float scale, hipStream_t s) {
    const int G = hq / hkv;
    if (nsplit < 1 || nsplit > ATT_MAX_SPLITS) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: %d attention splits outside 1..%d", nsplit, ATT_MAX_SPLITS);
        return TL_HIP_ERR_ARG;
    }
    // 32 positions per wavefront, or 16 when that leaves fewer than ~2 workgroups per CU
    const int pw = (int64_t)B * hkv * nsplit >= 512 ? 32 : 16;
    if (pw == 16) nsplit *= 2;
    if (nsplit > ATT_MAX_SPLITS) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: %d attention splits exceed %d", nsplit, ATT_MAX_SPLITS);
        return TL_HIP_ERR_ARG;
    }
    AttnArgs a{q, k, v, out, ws, hkv, lmax, kv_bstride, AttnLen{L, len_dev, len_add, len_step}, 4 * pw, nsplit,
               scale};
    dim3 grid(nsplit, hkv, B);
    // one launch (the last-arriving split merges) when the records fit one workgroup's merge and
    // no other stream can run a call that shares the arrival counters
    const bool fuse = nsplit > 1 && nsplit <= ATT_FUSE_MAX && (int64_t)B * hkv <= ATT_ARRIVE_MAX &&
                      single_stream() && one_launch_merge();
#define TLH_GQ(DD, GG)                                                                              \
    if (D == DD && G == GG) {                                                                       \
        if (fuse) {                                                                                 \
            if (pw == 32) k_attn_gq<DD, GG, 32, true><<<grid, 256, 0, s>>>(a);                      \
            else k_attn_gq<DD, GG, 16, true><<<grid, 256, 0, s>>>(a);                               \
        } else {                                                                                    \
            if (pw == 32) k_attn_gq<DD, GG, 32, false><<<grid, 256, 0, s>>>(a);                     \
            else k_attn_gq<DD, GG, 16, false><<<grid, 256, 0, s>>>(a);                              \
            if (nsplit > 1) k_attn_merge_gq<DD, GG><<<dim3(hkv, B, GG), 256, 0, s>>>(a);            \
        }                                                                                           \
        hipError_t e = hipGetLastError();                                                           \
        return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "attention launch");                       \
    }
    TLH_GQ(64, 4) TLH_GQ(64, 8) TLH_GQ(128, 4) TLH_GQ(128, 8)
#undef TLH_GQ
    set_error(TL_HIP_ERR_ARG, "ArgumentError: grouped-query attention covers head_dim 64 / 128 with 4 or 8 "
              "query heads per KV head (got D=%d, group %d)", D, G);
    return TL_HIP_ERR_ARG;
}

// Splits of 128 positions covering L; the launch may halve the split size (the workspace
// must then hold twice as many records: attn_workspace_floats(..., 2 * nsplit)).
int attention_gq_splits(int64_t L) { return (int)cdiv(L, 128); }

bool attention_gq_supported(int kv_dtype, int hq, int hkv, int D) {
    const int G = hkv > 0 ? hq / hkv : 0;
    return kv_dtype == TL_HIP_F16 && (D == 64 || D == 128) && (G == 4 || G == 8) && hq == G * hkv;
}

int launch_attention(const float* q, const void* k, const void* v, int kv_dtype, float* out,
                     float* ws, int B, int hq, int hkv, int D, int64_t lmax,
                     int64_t kv_bstride, int64_t L, const int32_t* len_dev, int len_add,
                     int len_step, int chunk, int nsplit, float scale, hipStream_t s) {
    if (chunk > ATT_MAX_CHUNK || chunk % 32) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: attention chunk %d", chunk);
        return TL_HIP_ERR_ARG;
    }
    if (nsplit > ATT_MAX_SPLITS) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: %d attention splits exceed %d", nsplit, ATT_MAX_SPLITS);
        return TL_HIP_ERR_ARG;
    }
    AttnArgs a{q, k, v, out, ws, hkv, lmax, kv_bstride, AttnLen{L, len_dev, len_add, len_step},
               chunk, nsplit, scale};
    if (kv_dtype == TL_HIP_F16) return attn_dispatch<__half>(a, B, hq, D, s);
    return attn_dispatch<float>(a, B, hq, D, s);
}

}  // namespace tlhip

using namespace tlhip;

extern "C" tl_hip_tensor* tl_hip_attention_decode(const tl_hip_tensor* qh, const tl_hip_tensor* kh,
                                                  const tl_hip_tensor* vh, int64_t L, float scale) {
    if (!qh || !kh || !vh) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: q, k or v");
        return nullptr;
    }
    if (!state()) return nullptr;
    const Tensor* q = reinterpret_cast<const Tensor*>(qh);
    const Tensor* k = reinterpret_cast<const Tensor*>(kh);
    const Tensor* v = reinterpret_cast<const Tensor*>(vh);
    if (q->dtype != TL_HIP_F32 || k->dtype != v->dtype) {
        set_error(TL_HIP_ERR_TYPE, "TypeMismatch: q must be f32 and k, v of one dtype");
        return nullptr;
    }
    if (q->rank != 3 || k->rank != 4 || v->rank != 4) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: q [B,Hq,D], k/v [B,Hkv,Lmax,D] expected");
        return nullptr;
    }
    const int64_t B = q->shape[0], hq = q->shape[1], D = q->shape[2];
    const int64_t hkv = k->shape[1], lmax = k->shape[2];
    for (int i = 0; i < 4; i++)
        if (k->shape[i] != v->shape[i]) {
            set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: k and v shapes differ");
            return nullptr;
        }
    if (k->shape[0] != B || k->shape[3] != D || hkv <= 0 || hq % hkv != 0) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: q [%lld,%lld,%lld] vs kv [%lld,%lld,%lld,%lld]",
                  (long long)B, (long long)hq, (long long)D, (long long)k->shape[0], (long long)hkv,
                  (long long)lmax, (long long)k->shape[3]);
        return nullptr;
    }
    if (L < 1 || L > lmax) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: cached length %lld outside 1..%lld", (long long)L,
                  (long long)lmax);
        return nullptr;
    }
    if (B > 65535 || hkv > 65535) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: batch or head count too large");
        return nullptr;
    }
    const bool dec = attention_gq_supported(k->dtype, (int)hq, (int)hkv, (int)D);
    int chunk, nsplit;
    attn_plan((int)B, (int)hkv, L, &chunk, &nsplit);
    if (dec) {
        chunk = 128;
        nsplit = attention_gq_splits(L);
    }
    int64_t oshape[3] = {B, hq, D};
    Tensor* o = tensor_alloc(oshape, 3);
    if (!o) return nullptr;
    hipStream_t s = cur_stream();
    float* ws = (float*)dev_alloc(attn_workspace_floats((int)B, (int)hkv, (int)(hq / hkv), (int)D, 2 * nsplit) * 4);
    int rc = ws ? TL_HIP_OK : TL_HIP_ERR_ALLOC;
    if (rc == TL_HIP_OK && !dec && attention_qh_supported(k->dtype, (int)D, lmax))
        rc = launch_attention_qh(q->f32(), k->data, v->data, k->dtype, o->f32(), (int)B, (int)hq, (int)hkv, (int)D,
                                 lmax, hkv * lmax * D, L, nullptr, 0, 0, scale, s);
    else if (rc == TL_HIP_OK && dec)
        rc = launch_attention_gq(q->f32(), k->data, v->data, o->f32(), ws, (int)B, (int)hq, (int)hkv, (int)D, lmax,
                                 hkv * lmax * D, L, nullptr, 0, 0, nsplit, scale, s);
    else if (rc == TL_HIP_OK)
        rc = launch_attention(q->f32(), k->data, v->data, k->dtype, o->f32(), ws, (int)B, (int)hq, (int)hkv,
                              (int)D, lmax, hkv * lmax * D, L, nullptr, 0, 0, chunk, nsplit, scale, s);
    dev_free(ws);  // stream-ordered: reused only by later work on the same stream
    if (rc != TL_HIP_OK) {
        tensor_drop(o);
        return nullptr;
    }
    return H(o);
}

extern "C" tl_hip_tensor* tl_hip_attention_prefill(const tl_hip_tensor* qh, const tl_hip_tensor* kh,
                                                   const tl_hip_tensor* vh, int64_t pos0, float scale) {
    if (!qh || !kh || !vh) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: q, k or v");
        return nullptr;
    }
    if (!state()) return nullptr;
    const Tensor* q = reinterpret_cast<const Tensor*>(qh);
    const Tensor* k = reinterpret_cast<const Tensor*>(kh);
    const Tensor* v = reinterpret_cast<const Tensor*>(vh);
    if (q->dtype != TL_HIP_F32 || k->dtype != TL_HIP_F16 || v->dtype != TL_HIP_F16) {
        set_error(TL_HIP_ERR_TYPE, "TypeMismatch: q must be f32, k and v f16");
        return nullptr;
    }
    if (q->rank != 3 || k->rank != 3 || v->rank != 3) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: q [n,Hq,D], k/v [Hkv,Lmax,D] expected");
        return nullptr;
    }
    const int64_t n = q->shape[0], hq = q->shape[1], D = q->shape[2];
    const int64_t hkv = k->shape[0], lmax = k->shape[1];
    for (int i = 0; i < 3; i++)
        if (k->shape[i] != v->shape[i]) {
            set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: k and v shapes differ");
            return nullptr;
        }
    if (k->shape[2] != D || hkv <= 0 || hq % hkv != 0) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: q [%lld,%lld,%lld] vs kv [%lld,%lld,%lld]", (long long)n,
                  (long long)hq, (long long)D, (long long)hkv, (long long)lmax, (long long)k->shape[2]);
        return nullptr;
    }
    if (!attention_prefill_supported(TL_HIP_F16, (int)hq, (int)hkv, (int)D) || hkv > 32767) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: prefill attention covers head_dim 64 / 128 with 4 or 8 query heads "
                  "per KV head");
        return nullptr;
    }
    if (n < 1 || pos0 < 0 || pos0 > lmax - n || n > INT32_MAX) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: %lld queries from position %lld exceed the cache of %lld rows",
                  (long long)n, (long long)pos0, (long long)lmax);
        return nullptr;
    }
    int64_t oshape[3] = {n, hq, D};
    Tensor* o = tensor_alloc(oshape, 3);
    if (!o) return nullptr;
    int rc = launch_attention_prefill(q->f32(), k->data, v->data, o->f32(), (int)n, (int)hq, (int)hkv, (int)D, lmax,
                                      nullptr, pos0, scale, cur_stream());
    if (rc != TL_HIP_OK) {
        tensor_drop(o);
        return nullptr;
    }
    return H(o);
}

// ------------------------------------------------- scaled dot-product attention op ----
// IDevice::tensor_scaled_dot_product_attention with the tl_cpu semantics
// (crates/tl_cpu/src/device_impl.rs:775-872): per (slice, query row), scores
// s_j = (q . k_j) * (1 / sqrt(d_k)); where a mask is given, s_j = -1e9 when the mask's flat
// element i * seq_k + j exists and equals 0 (the same [seq_q, seq_k] mask for every slice);
// softmax over j (max, exp, sum, divide); out = sum_j p_j v_j.  One workgroup per query row:
// the q row sits in LDS, one wavefront forms each score (lanes over d, DPP reduction) into the
// row's slice of a score workspace, the workgroup reduces max and sum, normalises in place,
// and each thread accumulates output columns over the keys in key order.
__global__ __launch_bounds__(256) void k_sdpa(const float* __restrict__ q, const float* __restrict__ k,
                                              const float* __restrict__ v, const float* __restrict__ mask,
                                              int64_t mask_len, float* __restrict__ out, float* __restrict__ sc,
                                              int64_t sq, int64_t sk, int dk, int dv, float scale) {
    extern __shared__ float qs[];  // [dk]
    __shared__ float red[4];
    const int64_t row = blockIdx.x;  // slice * sq + i
    const int64_t slice = row / sq, i = row - slice * sq;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR
    const float* kb = k + slice * sk * dk;
    const float* vb = v + slice * sk * dv;
    float* s = sc + row * sk;
    for (int d = tid; d < dk; d += 256) qs[d] = q[row * dk + d];
    __syncthreads();
    for (int64_t j = wave; j < sk; j += 4) {
        const float* kr = kb + j * dk;
        float p = 0.f;
        for (int d = lane; d < dk; d += 64) p = fmaf(qs[d], kr[d], p);
        p = wave_allsum(p);
        if (lane == 0) {
            float x = p * scale;
            const int64_t mi = i * sk + j;
            if (mask && mi < mask_len && mask[mi] == 0.0f) x = -1e9f;
            s[j] = x;
        }
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int64_t j = tid; j < sk; j += 256) mx = fmaxf(mx, s[j]);
    mx = wave_allmax(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.f;
    for (int64_t j = tid; j < sk; j += 256) {
        const float e = expf(s[j] - mx);
        s[j] = e;
        sum += e;
    }
    sum = wave_allsum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = (red[0] + red[1]) + (red[2] + red[3]);
    for (int64_t j = tid; j < sk; j += 256) s[j] = s[j] / sum;
    __syncthreads();
    for (int d = tid; d < dv; d += 256) {
        float acc = 0.f;
        for (int64_t j = 0; j < sk; j++) acc = fmaf(s[j], vb[j * dv + d], acc);
        out[row * dv + d] = acc;
    }
}

extern "C" tl_hip_tensor* tl_hip_tensor_scaled_dot_product_attention(const tl_hip_tensor* qh, const tl_hip_tensor* kh,
                                                                     const tl_hip_tensor* vh,
                                                                     const tl_hip_tensor* maskh) {
    if (!qh || !kh || !vh) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: q, k or v");
        return nullptr;
    }
    if (!state()) return nullptr;
    const Tensor* q = reinterpret_cast<const Tensor*>(qh);
    const Tensor* k = reinterpret_cast<const Tensor*>(kh);
    const Tensor* v = reinterpret_cast<const Tensor*>(vh);
    const Tensor* mk = reinterpret_cast<const Tensor*>(maskh);
    if (q->dtype != TL_HIP_F32 || k->dtype != TL_HIP_F32 || v->dtype != TL_HIP_F32 ||
        (mk && mk->dtype != TL_HIP_F32)) {
        set_error(TL_HIP_ERR_TYPE, "TypeMismatch: q, k, v and mask must be f32");
        return nullptr;
    }
    const int r = q->rank;
    if (r < 2 || r > 4 || k->rank != r || v->rank != r) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: q, k, v must share a rank of 2, 3 or 4 ([batch, heads,] seq, dim)");
        return nullptr;
    }
    int64_t slices = 1;
    for (int d = 0; d < r - 2; d++) {
        if (k->shape[d] != q->shape[d] || v->shape[d] != q->shape[d]) {
            set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: q, k, v differ in batch / head dimensions");
            return nullptr;
        }
        slices *= q->shape[d];
    }
    const int64_t sq = q->shape[r - 2], dk = q->shape[r - 1], sk = k->shape[r - 2], dv = v->shape[r - 1];
    if (k->shape[r - 1] != dk || v->shape[r - 2] != sk) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: k [.., %lld, %lld] and v [.., %lld, %lld] for q [.., %lld, %lld]",
                  (long long)sk, (long long)k->shape[r - 1], (long long)v->shape[r - 2], (long long)dv,
                  (long long)sq, (long long)dk);
        return nullptr;
    }
    if (dk > 16384 || dv > 65536 || slices * sq > INT32_MAX) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: head dimension or row count too large");
        return nullptr;
    }
    int64_t oshape[4];
    for (int d = 0; d < r - 2; d++) oshape[d] = q->shape[d];
    oshape[r - 2] = sq;
    oshape[r - 1] = dv;
    Tensor* o = tensor_alloc(oshape, r);
    if (!o) return nullptr;
    hipStream_t s = cur_stream();
    if (o->numel == 0) return H(o);
    if (sk == 0) {  // no keys: every output sum is empty
        hipError_t e = hipMemsetAsync(o->data, 0, o->numel * 4, s);
        if (e != hipSuccess) {
            hip_fail(e, "hipMemsetAsync");
            tensor_drop(o);
            return nullptr;
        }
        return H(o);
    }
    float* ws = (float*)dev_alloc((size_t)(slices * sq) * sk * 4);
    if (!ws) {
        tensor_drop(o);
        return nullptr;
    }
    // 1 / sqrt(d_k) as tl_cpu computes it in f32 (device_impl.rs:800)
    const float scale = 1.0f / sqrtf((float)dk);
    k_sdpa<<<(unsigned)(slices * sq), 256, (size_t)(dk > 0 ? dk : 1) * 4, s>>>(
        q->f32(), k->f32(), v->f32(), mk ? mk->f32() : nullptr, mk ? mk->numel : 0, o->f32(), ws, sq, sk, (int)dk,
        (int)dv, scale);
    hipError_t e = hipGetLastError();
    dev_free(ws);
    if (e != hipSuccess) {
        hip_fail(e, "sdpa launch");
        tensor_drop(o);
        return nullptr;
    }
    return H(o);
}
