// Internal declarations shared by the tl_hip translation units (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>
#include <atomic>
#include <string>

#include "../../include/tl_hip.h"

namespace tlhip {

// ---- errors: thread-local last error, mirroring the reference's TLS LAST_ERROR
// (crates/tl_runtime/src/device_ffi.rs:22-80) ---------------------------------------
void set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
int hip_fail(hipError_t e, const char* what);  // records a DeviceError, returns status

#define TLH_CHECK_HIP(expr)                                  \
    do {                                                     \
        hipError_t _e = (expr);                              \
        if (_e != hipSuccess) return ::tlhip::hip_fail(_e, #expr); \
    } while (0)

// ---- kernel outputs that the next launch reads ----------------------------------------
// Written through the L2 at agent scope (global_store ... sc1): the dirty lines then leave
// during the kernel, not in the end-of-kernel cache write-back that the next dependent launch
// waits for (a 100-launch dependent chain of 512-workgroup kernels: 1.84 -> 1.70 us per
// launch on MI355X).  Ordinary stores as far as the memory model goes (relaxed atomics).
__device__ __forceinline__ void st_wt(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_wt(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_wt(uint8_t* p, uint8_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_wt(__half* p, __half v) {
    __hip_atomic_store(reinterpret_cast<uint16_t*>(p), __half_as_ushort(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Weight-stream loads: read once per pass and not reused by the launch, loaded non-temporal
// (global_load ... nt)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Raw (stride 0) buffer resource over [p, p + bytes): buffer loads past the range read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// Cache policy of a buffer access that is coherent at agent scope (the sc1 bit): the policy of
// agent-scope atomic loads and stores on this target.
constexpr int CPOL_SC1 = 16;
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return uint4{t.x, t.y, t.z, t.w};
}

// ---- device state -----------------------------------------------------------------
struct DeviceState {
    int device = -1;
    hipStream_t stream = nullptr;
    int num_cus = 0;
    int num_xcds = 8;
};
DeviceState* state();      // initialises device 0 on first use; nullptr on failure
hipStream_t cur_stream();  // library stream (or the override set by tl_hip_set_stream)

// ---- stream-ordered caching allocator --------------------------------------------
// A block is freed on the stream of its last use; a request on that stream reuses it with
// no synchronisation, a request on another stream only after the free's event completed.
void* dev_alloc(size_t bytes);  // on cur_stream(); nullptr + AllocationError on failure
void dev_free(void* p);         // on cur_stream()
void* dev_alloc_on(size_t bytes, hipStream_t s);
void dev_free_on(void* p, hipStream_t s);
// Marks that work runs on stream s; the first stream other than the library stream switches
// the allocator to event-tagged frees.
void note_stream(hipStream_t s);
// True when note_stream(s) would synchronise the library stream (the first caller stream).
bool note_stream_syncs(hipStream_t s);
bool single_stream();  // no stream but the library's has run library work (calls cannot overlap)
bool one_launch_merge();  // split kernels may merge their partials in the same launch
// Looks up the device address of the allocation-free GEMM's scratch array on `device` (the
// current device during library initialisation); status code.
int noalloc_scratch_init(int device);

// ---- tensors ---------------------------------------------------------------------
struct Tensor {
    void* data = nullptr;  // device memory
    int64_t shape[TL_HIP_MAX_RANK] = {0};
    int rank = 0;
    int64_t numel = 0;
    int dtype = TL_HIP_F32;
    bool owns = true;
    std::atomic<int> refs{1};
    float* f32() const { return static_cast<float*>(data); }
};
Tensor* tensor_alloc(const int64_t* shape, int rank, int dtype = TL_HIP_F32);
inline Tensor* T(tl_hip_tensor* h) { return reinterpret_cast<Tensor*>(h); }
inline tl_hip_tensor* H(Tensor* t) { return reinterpret_cast<tl_hip_tensor*>(t); }
void tensor_drop(Tensor* t);
size_t dtype_size(int dtype);

// ---- quantized weights (device residency of a GGUF tensor) -------------------------
// Struct-of-arrays repack of the GGUF blocks, organised in 32-weight units (nb units per
// row) so that every type offers one 16-byte quant load per unit:
//   Q4_0  qs [n][nb][16]  GGUF nibble order (byte j: weight j | weight j + 16 << 4)
//         d  [n][nb]      f16 scale
//   Q8_0  qs [n][nb][32]  int8, d [n][nb] f16
//   Q4_K  qs [n][nb][16]  the unit's 32 nibbles in Q4_0 order (unit = one sub-block)
//         hdr[n][nb/8][16] the super-block header: f16 d, f16 dmin, then the 16 6-bit
//                          fields re-laid (q4k_hdr_sm): scale j at bit 6j of words 1-2,
//                          min j at bit 16 + 6j of words 2-3
//   Q6_K  qs [n][nb][16]  low 4 bits in Q4_0 order
//         qh [n][nb][8]   high 2 bits: word 0 byte b bits 2t..2t+1 = weight b + 4t,
//                         word 1 the same for weights 16 + b + 4t
//         sc [n][nb][2]   the int8 scales of the unit's two 16-weight sub-blocks
//         d  [n][nb/8]    f16 super-block scale
// Byte counts equal the GGUF stream's (18 / 34 / 144 / 210 bytes per 32 / 32 / 256 / 256).
// Q4_K sub-block j's 6-bit scale and min from a resident super-block header (words: f16 d |
// f16 dmin, then the 96 bits of 16 fields -- scales at bits 6j, mins at bits 48 + 6j): one
// 64-bit shift and a mask each, with no branch on j.  GGUF packs them in 12 bytes two ways
// (QTensor::get_scale_min_k4, quantized.rs:405-415: sub-blocks 0-3 in the low 6 bits of
// bytes j and j + 4, sub-blocks 4-7 split over nibbles of bytes j + 4 and the top 2 bits of
// bytes j - 4 and j), which cost a lane-divergent branch per unit to unpack.
__host__ __device__ inline void q4k_hdr_sm(const uint4& hd, int j, uint32_t* sc, uint32_t* mn) {
    const uint64_t a = ((uint64_t)hd.z << 32) | hd.y, b = ((uint64_t)hd.w << 32) | hd.z;
    *sc = (uint32_t)(a >> (6 * j)) & 63u;
    *mn = (uint32_t)(b >> (16 + 6 * j)) & 63u;
}

struct QWeight {
    int ggml_type = 0;
    int64_t n = 0, k = 0, nb = 0;  // rows, cols, 32-weight units per row
    uint8_t* qs = nullptr;
    __half* d = nullptr;
    uint8_t* hdr = nullptr;  // Q4_K
    uint8_t* qh = nullptr;   // Q6_K
    int8_t* sc = nullptr;    // Q6_K
    uint32_t* us = nullptr;  // Q4_K: per-unit f16 pair (d sc, -dmin m) for the f16 GEMM, built on request
    int64_t shape[TL_HIP_MAX_RANK] = {0};
    int rank = 0;
    std::atomic<int> refs{1};
};
inline QWeight* Q(tl_hip_qtensor* h) { return reinterpret_cast<QWeight*>(h); }

// ---- fused decode matvec (matvec.hip) ---------------------------------------------
enum { EPI_PLAIN = 0, EPI_RES = 1, EPI_GLU = 2, EPI_ROPE_KV = 3, EPI_ARGMAX = 4 };

struct MvArgs {
    const uint8_t* qs;
    const __half* d;
    const uint8_t* hdr;
    const uint8_t* qh;
    const int8_t* sc;
    int64_t n, k, nb;
    const float* x;           // [m, k]; with EMBED the embedding table [vocab, k]
    const int32_t* embed_id;  // EMBED: token id (device)
    float* x_out;             // EMBED: gathered row written here (workgroup 0)
    const float* norm_w;      // NORM weight [k]
    float eps;
    float* y;                 // output
    const float* res;         // EPI_RES residual (may alias y)
    // EPI_ROPE_KV
    const int32_t* pos;
    const float* cos_t;
    const float* sin_t;
    float* q_out;
    void* kc;
    void* vc;
    int q_rows, kv_rows, hd, kv_f16;
    int64_t max_seq;
    int64_t row_off;  // rows of this weight start at row_off of the q | k | v projection
    // x formed from ATTN_SHARES attention records per head (launch_attention_qh with that
    // nsplit): x[h * attn_hd + d] = merge of records (h, 0 ..); M = 1, EPI_RES, no prologue
    const float* attn_rec;
    int attn_hd;
    // EPI_ARGMAX
    float* plogits;       // penalised logits
    const uint8_t* seen;  // repetition-penalty mask (nullptr = no penalty)
    uint8_t* seen_out;    // mask updated with the chosen token
    float penalty;
    float* part_v;        // per-workgroup best value
    int32_t* part_i;      // per-workgroup best index
    int32_t* part_nan;    // per-workgroup NaN flag
    int32_t* tok_out;
    int32_t* out_ids;
    int32_t* step;
    int32_t* pos_inc;     // position advanced by one (decode step end)
    int max_out;
    // top-p sampling instead of the greedy finish when smp_temp > 0 (decode steps)
    float smp_temp, smp_top_p;
    const float* smp_draws;  // one uniform draw per step
    uint32_t* smp_key;       // key scratch for vocabularies past 32768
};
struct QWeight;
// One fused matvec launch over weight w (m = 1 or 2 activation rows); weight fields of `a`
// are filled from w.
int launch_mv(const QWeight* w, MvArgs a, int m, int epi, bool norm, bool embed, hipStream_t s);
// workgroups (= argmax partial slots) of a matvec over n rows
int mv_partials(int64_t n);
bool matvec_fits(const QWeight* w, int64_t m);  // the LDS-staged matvec takes this product
// One launch for the two weights of a q | k | v projection (RMSNorm prologue, RoPE + KV
// epilogue): returns -1 without launching when the pair is not covered.
int launch_mv_pair(const QWeight* w1, const QWeight* w2, MvArgs a, int64_t row_off2, bool embed, hipStream_t s);
int launch_read_floor(const QWeight* w, hipStream_t s);  // read of w's arrays, matvec launch shape

// kernel entry points shared across translation units (all on the given stream)
int launch_quant_matvec(const QWeight* w, const float* x, float* y, int64_t m, hipStream_t s,
                        const float* residual);
int launch_quant_gemm(const QWeight* w, const float* x, float* y, int64_t m, hipStream_t s,
                      int mode);
// The f16 MFMA GEMM on an input already in f16 operand order (x16 [m, k]: every 32-element
// block stored as four 8-half words, the k slots of the MFMA operands).  Two orders: F16Q_Q4
// (word t = elements 4t..4t+3, 16+4t..16+4t+3; Q4_0 and the f16-dequantized K-quants) and
// F16Q_Q8 (word t = 8t, 8t+2, 8t+1, 8t+3, 8t+4, 8t+6, 8t+5, 8t+7; Q8_0).
typedef _Float16 half8 __attribute__((ext_vector_type(8)));  // one operand word
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ---- lane exchanges across 16 / 32 lanes without LDS (gfx950) ----------------------------
// v_permlane32_swap(a, b) (v_permlane16_swap) exchanges the upper 32 lanes (the odd 16-lane
// rows) of a with the lower 32 lanes (the even rows) of b: a lane l with bit OFF clear ends
// with (a_l, a_{l+OFF}), a lane with it set with (b_{l-OFF}, b_l).  VALU instructions: no LDS
// round trip as with ds_bpermute (__shfl_xor).
template <int OFF>
__device__ __forceinline__ void lane_swap(uint32_t& a, uint32_t& b) {
    static_assert(OFF == 16 || OFF == 32, "row-crossing swaps only");
    if constexpr (OFF == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
        a = r[0];
        b = r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        a = r[0];
        b = r[1];
    }
}
// a_l + a_{l^OFF}: the sum of a lane's value and its partner's (every lane gets it)
template <int OFF>
__device__ __forceinline__ float lane_pair_sum(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    lane_swap<OFF>(a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
template <int OFF>
__device__ __forceinline__ float lane_pair_max(float v) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    lane_swap<OFF>(a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
// the value of lane l ^ OFF
template <int OFF>
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t v) {
    uint32_t a = v, b = v;
    lane_swap<OFF>(a, b);
    return (__lane_id() & OFF) ? a : b;
}
template <int OFF>
__device__ __forceinline__ float lane_xor_f32(float v) {
    return __builtin_bit_cast(float, lane_xor_u32<OFF>(__builtin_bit_cast(uint32_t, v)));
}
// The same within 16 lanes by DPP, for all-reduce steps (any involution that pairs the two
// halves of each group of 2 OFF lanes): quad_perm [1,0,3,2] (OFF 1), [2,3,0,1] (2), half-row
// mirror (4), row mirror (8).
template <int OFF>
__device__ __forceinline__ uint32_t lane_pair_dpp(uint32_t v) {
    constexpr int CTRL = OFF == 1 ? 0xB1 : OFF == 2 ? 0x4E : OFF == 4 ? 0x141 : 0x140;
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
// DPP move within 16-lane rows (all rows and banks, bound_ctrl): quad_perm [1,0,3,2] 0xB1,
// [2,3,0,1] 0x4E, half-row mirror 0x141, row mirror 0x140, row_ror:k 0x120 + k (lane i reads
// lane (i + k) mod 16 of its row).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// sum over aligned groups of 8 lanes in the order xor 1, xor 2, xor 4: after the first two
// steps a lane's value equals its quad's, so the half-row mirror (lane 7 - i) reads the value
// of lane i ^ 4
__device__ __forceinline__ float sum8_dpp(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v;
}
// Wavefront all-reduce over the xor butterfly 32, 16, 8, 4, 2, 1 -- the pairing and order of
// `for (off = 32; off >= 1; off >>= 1) v = op(v, __shfl_xor(v, off))`, hence bitwise equal
// results.  32 and 16 are permlane swaps.  After the steps above bit k every lane holds the
// value of each lane that differs from it only in bits above k, so row_ror:k (lane
// (i + k) mod 16, which differs from i ^ k only in those bits) reads the xor partner's value.
__device__ __forceinline__ float wave_allsum(float v) {
    v = lane_pair_sum<32>(v);
    v = lane_pair_sum<16>(v);
    v += dpp_f<0x128>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x122>(v);
    v += dpp_f<0x121>(v);
    return v;
}
__device__ __forceinline__ float wave_allmax(float v) {
    v = lane_pair_max<32>(v);
    v = lane_pair_max<16>(v);
    v = fmaxf(v, dpp_f<0x128>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x122>(v));
    v = fmaxf(v, dpp_f<0x121>(v));
    return v;
}

// (greater value, then larger index) over the 64 lanes, empty lanes bi < 0, NaN flags or-ed:
// every lane ends with the wavefront's best.  The steps pair lanes by DPP within 16 lanes and
// by the permlane swaps across rows; the order of the steps does not matter for this
// commutative, associative selection (with a NaN the caller replays a sequential fold).
__device__ __forceinline__ void argmax_step(float& bv, int& bi, int& nan, float ov, int oi, int on) {
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
        bv = ov;
        bi = oi;
    }
    nan |= on;
}
template <int OFF>
__device__ __forceinline__ void argmax_round(float& bv, int& bi, int& nan) {
    uint32_t v, i, f;
    if constexpr (OFF >= 16) {
        v = lane_xor_u32<OFF>(__builtin_bit_cast(uint32_t, bv));
        i = lane_xor_u32<OFF>((uint32_t)bi);
        f = lane_xor_u32<OFF>((uint32_t)nan);
    } else {
        v = lane_pair_dpp<OFF>(__builtin_bit_cast(uint32_t, bv));
        i = lane_pair_dpp<OFF>((uint32_t)bi);
        f = lane_pair_dpp<OFF>((uint32_t)nan);
    }
    argmax_step(bv, bi, nan, __builtin_bit_cast(float, v), (int)i, (int)f);
}
__device__ __forceinline__ void argmax_allreduce(float& bv, int& bi, int& nan) {
    argmax_round<1>(bv, bi, nan);
    argmax_round<2>(bv, bi, nan);
    argmax_round<4>(bv, bi, nan);
    argmax_round<8>(bv, bi, nan);
    argmax_round<16>(bv, bi, nan);
    argmax_round<32>(bv, bi, nan);
}

enum { F16Q_Q4 = 0, F16Q_Q8 = 1 };
enum { GEMM_PLAIN = 0, GEMM_RES = 1, GEMM_GLU16 = 2, GEMM_ROPE_KV = 3 };
// RoPE of one interleaved pair (x0, x1) by (c, s): (x0 c - x1 s, x0 s + x1 c) with the
// contraction spelled out, so the prefill's RoPE kernel and the GEMM epilogue round alike.
__host__ __device__ inline void rope_pair(float x0, float x1, float c, float s, float* r0, float* r1) {
    *r0 = fmaf(x0, c, -(x1 * s));
    *r1 = fmaf(x0, s, x1 * c);
}
// Operands of the ROPE_KV epilogue: the GEMM's rows are tokens pos .. pos + m - 1 and its
// columns are columns col_off .. of [q | k | v] (H + 2 KV heads of hd; col_off a multiple of
// hd: a weight holding some of the heads); q is rotated into q [m, H hd], k rotated and v
// copied into the caches [KV][max_seq][hd] (f16 when kv_f16, else f32) at slot pos + row.
// Table row pos + row (per_token) or pos of ct / st [*, hd] (entries 2i, 2i + 1 alike).
struct RopeKvEpi {
    float* q = nullptr;
    void* kc = nullptr;
    void* vc = nullptr;
    const float* ct = nullptr;
    const float* st = nullptr;
    const int32_t* pos = nullptr;
    int H = 0, KV = 0, hd = 0, per_token = 0, kv_f16 = 0, col_off = 0;
    int hd_shift = 0;  // log2(hd): the head size is a power of two
    int64_t max_seq = 0;
};
// Epilogue: PLAIN y = v; RES y = res + v (res may be y); GLU16 columns (2i, 2i + 1) are
// (gate_i, up_i) and silu(gate_i) * up_i goes to out16 [m, n / 2] in operand order `order`;
// ROPE_KV: RoPE and the KV-cache append of a [q | k | v] projection (rk), y not written.
struct GemmEpi {
    int mode;
    const float* res;
    _Float16* out16;
    int order;
    RopeKvEpi rk{};
};
// The ROPE_KV epilogue, split into what depends on the GEMM's column c only (RopeCol: column
// col_off + c of [q | k | v]: q, k or v, its head and index within the head) and the store of
// one token row r (pair values (x0, x1) of the column's interleaved pair, v the column's own
// value; cs / sn the table entries of the pair, rope_tab).  Column indices are 32-bit
// (n < 2^31).
struct RopeCol {
    uint32_t kind;  // 0 q, 1 k, 2 v
    uint32_t c;     // column of [q | k | v]
    uint32_t head;  // KV head (k, v)
    uint32_t i;     // index within the head vector
};
__device__ inline RopeCol rope_col(const RopeKvEpi& rk, int64_t c64) {
    const uint32_t c = (uint32_t)c64 + (uint32_t)rk.col_off, hd = (uint32_t)rk.hd, sh = (uint32_t)rk.hd_shift;
    const uint32_t qw = (uint32_t)rk.H * hd, kw = (uint32_t)rk.KV * hd;
    const uint32_t kind = c < qw ? 0u : c < qw + kw ? 1u : 2u;
    const uint32_t rel = kind == 0 ? c : kind == 1 ? c - qw : c - qw - kw;
    return RopeCol{kind, c, rel >> sh, rel & (hd - 1)};
}
// the table row of token row r: pos + r (per_token) or pos
__device__ inline int64_t rope_tab(const RopeKvEpi& rk, const RopeCol& cl, int64_t r, int64_t pos) {
    return (rk.per_token ? pos + r : pos) * rk.hd + (cl.i & ~1u);
}
__device__ inline void rope_kv_put(const RopeKvEpi& rk, const RopeCol& cl, int64_t r, int64_t pos, float x0, float x1,
                                   float v, float cs, float sn) {
    if (cl.kind == 2) {
        const int64_t at = ((int64_t)cl.head * rk.max_seq + pos + r) * rk.hd + cl.i;
        if (rk.kv_f16) static_cast<__half*>(rk.vc)[at] = __float2half(v);
        else static_cast<float*>(rk.vc)[at] = v;
        return;
    }
    float r0, r1;
    rope_pair(x0, x1, cs, sn, &r0, &r1);
    const float o = (cl.i & 1) ? r1 : r0;
    if (cl.kind == 0) {
        rk.q[r * ((int64_t)rk.H * rk.hd) + cl.c] = o;
    } else {
        const int64_t at = ((int64_t)cl.head * rk.max_seq + pos + r) * rk.hd + cl.i;
        if (rk.kv_f16) static_cast<__half*>(rk.kc)[at] = __float2half(o);
        else static_cast<float*>(rk.kc)[at] = o;
    }
}
// a 4-column unit (columns c .. c + 3, c a multiple of 4: two whole pairs of one head) of
// token row r: its place and each pair's table entries once, and one 16-byte (f32) or 8-byte
// (f16) store of the four values
__device__ inline void rope_kv_store4(const RopeKvEpi& rk, int64_t r, int64_t c, int64_t pos, float4 v) {
    const RopeCol cl = rope_col(rk, c);
    float o[4] = {v.x, v.y, v.z, v.w};
    if (cl.kind != 2) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            RopeCol ch = cl;
            ch.i += 2 * h;
            const int64_t ti = rope_tab(rk, ch, r, pos);
            rope_pair(o[2 * h], o[2 * h + 1], rk.ct[ti], rk.st[ti], &o[2 * h], &o[2 * h + 1]);
        }
    }
    if (cl.kind == 0) {
        *reinterpret_cast<float4*>(rk.q + r * ((int64_t)rk.H * rk.hd) + cl.c) = make_float4(o[0], o[1], o[2], o[3]);
        return;
    }
    void* base = cl.kind == 1 ? rk.kc : rk.vc;
    const int64_t at = ((int64_t)cl.head * rk.max_seq + pos + r) * rk.hd + cl.i;
    if (rk.kv_f16) {
        typedef _Float16 half4v __attribute__((ext_vector_type(4)));
        // (float -> f16 by round to nearest even, as __float2half in rope_kv_put)
        *reinterpret_cast<half4v*>(static_cast<__half*>(base) + at) =
            half4v{(_Float16)o[0], (_Float16)o[1], (_Float16)o[2], (_Float16)o[3]};
    } else {
        *reinterpret_cast<float4*>(static_cast<float*>(base) + at) = make_float4(o[0], o[1], o[2], o[3]);
    }
}
__host__ __device__ inline int64_t f16q_index(int64_t r, int64_t e, int64_t k, int order) {
    const int64_t b = e >> 5;
    const int e32 = (int)(e & 31);
    int t, slot;
    if (order == F16Q_Q8) {
        const int e8 = e32 & 7;
        t = e32 >> 3;
        slot = (e8 & 4) | ((e8 & 1) << 1) | ((e8 >> 1) & 1);
    } else {
        t = (e32 & 15) >> 2;
        slot = (e32 & 3) + (e32 & 16 ? 4 : 0);
    }
    return ((r * (k >> 5) + b) * 4 + t) * 8 + slot;
}
int f16q_order(int ggml_type);  // the operand order the f16 GEMM of this weight type reads
int launch_x_to_f16q(const float* x, _Float16* x16, int64_t m, int64_t k, int order, hipStream_t s);
// K a multiple of 128 (TL_HIP_ERR_ARG otherwise); GLU16 also needs N a multiple of 64.
// noalloc: split-K partials in part_ws (sized by the caller), nothing allocated.
// defer_part: a split-K launch hands its partial slices to the caller instead of summing
// them (see gemm.hip); launch_splitk_sum or launch_rmsnorm_f16q's summing form adds them.
int launch_gemm_f16q(const QWeight* w, const _Float16* x16, float* y, int64_t m, const GemmEpi& ep,
                     hipStream_t s, bool noalloc = false, float* part_ws = nullptr, float** defer_part = nullptr,
                     int* defer_nsp = nullptr);
int launch_splitk_sum(const float* part, float* y, const float* res, int64_t mn, int nsp, hipStream_t s);
// Q4_K weights: builds w->us (4 bytes per 32 weights) on stream s, after which the f16 GEMM
// dequantizes them in registers like Q4_0 instead of through an f16 copy per call.
int q4k_build_unit_scales(QWeight* w, hipStream_t s);
int launch_matmul_f32(const float* a, const float* b, float* c, int64_t batch, int64_t m,
                      int64_t k, int64_t n, int64_t a_bstride, int64_t b_bstride,
                      hipStream_t s);

int launch_rmsnorm(const float* x, const float* r, const float* w, float* out, int64_t rows,
                   int64_t n, float eps, int mode, hipStream_t s);
// mode-0 RMSNorm of [rows, n] written as f16 in GEMM operand order `order` (n % 32 == 0,
// n <= 8192): the value launch_rmsnorm produces, rounded once.  With part (nsp slices of
// rows * n floats from a deferred split-K GEMM), x first becomes x + the slices in order --
// written back, as launch_splitk_sum would -- and that row is normalised.
int launch_rmsnorm_f16q(float* x, const float* w, _Float16* out16, int64_t rows, int64_t n, float eps, int order,
                        hipStream_t s, const float* part = nullptr, int nsp = 0);
int launch_swiglu(const float* g, const float* u, float* o, int64_t n, int mode, hipStream_t s);
int launch_softmax(const float* x, float* out, int64_t outer, int64_t as, int64_t inner,
                   hipStream_t s);
int launch_argmax(const float* x, int64_t n, int32_t* out_idx, hipStream_t s);
// Top-p sampling (sample_impl's temp > 0 branch) of x [n] with the uniform draw u.  fin ==
// nullptr: the index goes to out[0] as a float.  fin: the decode step's form -- u is
// fin->draws[*fin->step] and the choice is recorded as the greedy finish records it.
// Inputs of more than 32768 logits need a key scratch of sample_key_words(n) words.
struct SmpFin {
    const float* draws;
    int32_t* tok_out;
    int32_t* out_ids;
    int32_t* step;
    uint8_t* seen_out;
    int32_t* pos_inc;
    int max_out;
};
int launch_sample_top_p(const float* x, int64_t n, float temp, float top_p, float u, uint32_t* key, float* out,
                        const SmpFin* fin, hipStream_t s);
int sample_key_words(int64_t n);
double sample_draw();            // the calling thread's next uniform draw in [0, 1)
void sample_seed(uint64_t seed);
int launch_rep_penalty(const float* x, const uint8_t* seen, float* o, int64_t rows,
                       int64_t vocab, float p, hipStream_t s);
int launch_embedding(const float* table, const int32_t* ids, float* o, int64_t n, int64_t dim,
                     hipStream_t s);
int launch_apply_rope(const float* x, const float* ct, const float* st, float* out,
                      int64_t total, int64_t hd, int64_t cos_len, int64_t sin_len, int64_t row0,
                      int64_t vpt, hipStream_t s);
int launch_rope_table(float* out, int64_t seq_len, int64_t dim, float base, int is_sin,
                      hipStream_t s);
// Attention over a [B?, Hkv, lmax, D] cache (kv_bstride elements between batch items, 0 =
// shared).  Cached length of item b = (len_dev ? *len_dev + len_add : L) + b * len_step.
int launch_attention(const float* q, const void* k, const void* v, int kv_dtype, float* out,
                     float* ws, int B, int hq, int hkv, int D, int64_t lmax,
                     int64_t kv_bstride, int64_t L, const int32_t* len_dev, int len_add,
                     int len_step, int chunk, int nsplit, float scale, hipStream_t s);
// Shapes of the grouped-query split form: f16 cache, D 64 / 128, 4 or 8 query heads per KV head.
bool attention_gq_supported(int kv_dtype, int hq, int hkv, int D);
// Grouped-query split form (shapes of attention_gq_supported): one workgroup per split of
// 128 (or 64) positions, KV head and batch item, then the split merge; nsplit =
// attention_gq_splits of the longest length, ws sized for 2 * nsplit records.
int launch_attention_gq(const float* q, const void* k, const void* v, float* out, float* ws, int B, int hq,
                        int hkv, int D, int64_t lmax, int64_t kv_bstride, int64_t L, const int32_t* len_dev,
                        int len_add, int len_step, int nsplit, float scale, hipStream_t s);
int attention_gq_splits(int64_t L);
// Causal prefill with f16 MFMA (shapes of attention_prefill_supported): q [n, hq, D] f32 of
// queries at positions pos0 + i over the cache [hkv, lmax, D] f16; out [n, hq, D].  pos0 is
// *pos_dev when pos_dev is given, else pos_host; pos0 + n <= lmax.  With out16 the rows go
// to f16 [n, hq D] in GEMM operand order `order` instead (hq D a multiple of 32).
bool attention_prefill_supported(int kv_dtype, int hq, int hkv, int D);
int launch_attention_prefill(const float* q, const void* k, const void* v, float* out, int n, int hq, int hkv,
                             int D, int64_t lmax, const int32_t* pos_dev, int64_t pos_host, float scale,
                             hipStream_t s, _Float16* out16 = nullptr, int order = 0);
// Short-cache form: one workgroup per (query head, batch item); shapes: attention_qh_supported.
bool attention_qh_supported(int kv_dtype, int D, int64_t lmax);
// position shares per query head in the decoder's attention (records merged by the o-projection)
constexpr int ATTN_SHARES = 4;  // 2 shares: 1810-1820 tok/s, 4: 1840-1843, 8: 1787 (merge cost)
// nsplit > 1: each head's positions in nsplit shares of whole 64-position rounds, one
// workgroup each, leaving unnormalised records [o (D) | max | sum | 0 | 0] (D + 4 floats) at
// part[((b * hq + head) * nsplit + share)] instead of writing out; the decode o-projection
// merges ATTN_SHARES shares in its activation staging (MvArgs::attn_rec).
int launch_attention_qh(const float* q, const void* k, const void* v, int kv_dtype, float* out,
                        int B, int hq, int hkv, int D, int64_t lmax, int64_t kv_bstride, int64_t L,
                        const int32_t* len_dev, int len_add, int len_step, float scale, hipStream_t s,
                        float* part = nullptr, int nsplit = 1);
void attn_plan(int B, int hkv, int64_t L, int* chunk, int* nsplit);
size_t attn_workspace_floats(int B, int hkv, int G, int D, int nsplit);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// GGUF block geometry of the quantized types: weights and bytes per block (0 = unsupported).
inline int ggml_block_elems(int t) {
    return t == TL_HIP_GGML_Q4_0 || t == TL_HIP_GGML_Q8_0 ? 32 : t == TL_HIP_GGML_Q4_K || t == TL_HIP_GGML_Q6_K ? 256 : 0;
}
inline int ggml_block_bytes(int t) {
    return t == TL_HIP_GGML_Q4_0 ? 18 : t == TL_HIP_GGML_Q8_0 ? 34 : t == TL_HIP_GGML_Q4_K ? 144 : t == TL_HIP_GGML_Q6_K ? 210 : 0;
}
inline const char* ggml_type_name(int t) {
    return t == TL_HIP_GGML_Q4_0 ? "Q4_0" : t == TL_HIP_GGML_Q8_0 ? "Q8_0" : t == TL_HIP_GGML_Q4_K ? "Q4_K" : t == TL_HIP_GGML_Q6_K ? "Q6_K" : "?";
}
// bytes of one row of k weights in the GGUF stream
inline size_t ggml_row_bytes(int t, int64_t k) { return (size_t)(k / ggml_block_elems(t)) * ggml_block_bytes(t); }

}  // namespace tlhip
