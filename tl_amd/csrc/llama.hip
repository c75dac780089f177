// Llama decoder driver: the model composition of examples/apps/tinyllama/chatbot.tl
// (Linear / RMSNorm / MLP / Attention / Block, lines 1-112, and the decode loop, 174-222)
// executed on the device.
//
// Differences in form (not in arithmetic) from the chatbot's op-by-op execution:
//  * q/k/v and gate/up weights are concatenated row-wise at load, so each projection pair /
//    triple is one matvec (every output row is the same dot product).  Parts stored in
//    different GGUF types (llama.cpp's Q4_K_M files keep some attn_v / ffn_down tensors in
//    Q6_K) form one segment per run of equal type: the q|k|v segments share the RoPE + KV
//    epilogue through their row offset, separate gate / up run as two matvecs + SwiGLU;
//  * the residual adds x + o-proj(x) and x + down(x) are fused into the matvec epilogue;
//  * RoPE, the KV-cache append and the q transpose are one kernel writing into a persistent
//    per-layer cache [Hkv, max_seq, head_dim] (instead of cat_4d + KVCache.update,
//    chatbot.tl:63-69), and attention reads the cache in place with GQA (no
//    repeat_interleave copy);
//  * the LM head runs on the last row only (the chatbot narrows to it, chatbot.tl:189);
//  * the cache position lives in device memory, so a decode step has no host
//    dependency: it is captured as hipGraphs of one and of eight consecutive steps and
//    replayed.
#include "internal.h"

#include <algorithm>
#include <cstring>
#include <vector>

namespace tlhip {

// token embedding of one or more ids (tensor.rs:1094-1112); ids were range-checked on the
// host or produced by argmax (< vocab).
__global__ void k_embed(const float* __restrict__ emb, const int32_t* __restrict__ ids,
                        float* __restrict__ x, int n, int64_t dim) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * dim) return;
    int64_t i = t / dim, j = t % dim;
    x[t] = emb[(int64_t)ids[i] * dim + j];
}

// RoPE (interleaved pairs, ffi.rs:2655-2681) on q and k of n tokens, q re-laid out as
// [n, H, hd] (already its layout) and k, v appended to the cache at position pos + t.
// Rotation row: pos (tl_cpu: the narrowed table's first row) or pos + t (per-token).
template <typename KVT>
__global__ void k_rope_kv(const float* __restrict__ qkv, float* __restrict__ qout,
                          KVT* __restrict__ kc, KVT* __restrict__ vc,
                          const float* __restrict__ ct, const float* __restrict__ st,
                          const int32_t* __restrict__ pos_dev, int n, int H, int KV, int hd,
                          int64_t max_seq, int per_token) {
    // arguments in one round of scalar loads (left to the compiler: three dependent rounds)
    asm volatile("" : : "s"(qkv), "s"(qout), "s"(kc), "s"(vc), "s"(ct), "s"(st), "s"(pos_dev), "s"(n), "s"(H),
                 "s"(KV), "s"(hd), "s"(max_seq), "s"(per_token));
    const int row = H * hd + 2 * KV * hd;
    const int pairs = (H + KV) * hd / 2;  // rotated pairs per token
    const int vals = KV * hd;             // copied v values per token
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_tok = pairs + vals;
    if (t >= (int64_t)n * per_tok) return;
    const int tok = (int)(t / per_tok);
    const int e = (int)(t % per_tok);
    const int64_t pos = (int64_t)(*pos_dev);
    const int64_t cpos = pos + tok;  // cache slot
    const float* src = qkv + (int64_t)tok * row;
    if (e < pairs) {
        const int64_t trow = per_token ? pos + tok : pos;
        const int idx = 2 * e;  // element index within q|k
        const int i = idx % hd;  // pair start within the head vector
        float c = ct[trow * hd + i], s = st[trow * hd + i];
        float x0 = src[idx], x1 = src[idx + 1];
        float r0, r1;
        rope_pair(x0, x1, c, s, &r0, &r1);
        if (idx < H * hd) {
            qout[(int64_t)tok * H * hd + idx] = r0;
            qout[(int64_t)tok * H * hd + idx + 1] = r1;
        } else {
            int kidx = idx - H * hd;
            int kh = kidx / hd;
            KVT* dst = kc + ((int64_t)kh * max_seq + cpos) * hd + i;
            dst[0] = (KVT)r0;
            dst[1] = (KVT)r1;
        }
    } else {
        int vidx = e - pairs;
        int vh = vidx / hd, d = vidx % hd;
        vc[((int64_t)vh * max_seq + cpos) * hd + d] = (KVT)src[H * hd + KV * hd + vidx];
    }
}

// SwiGLU on the interleaved gate/up rows: a[r, j] = silu(gu[r, 2j]) * gu[r, 2j + 1]
// (silu of ffi.rs:2097-2113 then mul, chatbot.tl:33-38)
__global__ void k_swiglu_rows(const float* __restrict__ gu, float* __restrict__ a, int n,
                              int64_t F) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * F) return;
    float2 p = reinterpret_cast<const float2*>(gu)[t];
    a[t] = (p.x * (1.0f / (1.0f + expf(-p.x)))) * p.y;
}

__global__ void k_add_inplace(float* __restrict__ x, const float* __restrict__ t, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + t[i];
}

__global__ void k_advance(int32_t* pos, int n) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *pos += n;
}

// A run of q|k|v rows stored in one type: rows [row_off, row_off + w->n) of the projection.
struct Seg {
    QWeight* w;
    int64_t row_off;
};

struct Llama {
    int nl, D, H, KV, hd, F, V, max_seq;
    float eps, theta;
    int kv_f16 = 0, rope_per_token = 0;
    std::vector<std::vector<Seg>> qkv_segs;
    std::vector<QWeight*> wo, wgu, wdown;
    std::vector<QWeight*> wg, wu;  // gate / up when their types differ (wgu is then null)
    QWeight* lm = nullptr;
    // host staging of q/k/v and gate/up until all parts of a layer are present
    std::vector<std::vector<uint8_t>> stage;  // [nl * 5]: q k v gate up
    std::vector<int> stage_type;
    std::vector<float*> attn_norm, ffn_norm;
    float* out_norm = nullptr;
    float* emb = nullptr;
    float *cos_t = nullptr, *sin_t = nullptr;
    std::vector<void*> kc, vc;
    // activations for up to max_tok tokens per call
    int64_t max_tok = 0;
    float *x = nullptr, *h = nullptr, *qkv = nullptr, *q = nullptr, *ao = nullptr, *t = nullptr,
          *gu = nullptr, *act = nullptr, *logits = nullptr, *plogits = nullptr, *ws = nullptr;
    size_t ws_floats = 0;
    // f16 GEMM inputs in operand order (fused prefill): [n, D] and [n, F]
    _Float16 *xa16 = nullptr, *xb16 = nullptr;
    int32_t *ids = nullptr, *pos = nullptr, *tok = nullptr, *step = nullptr, *out_ids = nullptr;
    uint8_t* seen = nullptr;
    // greedy-argmax candidates of the LM-head matvec (one per workgroup)
    float* am_v = nullptr;
    int32_t *am_i = nullptr, *am_nan = nullptr;
    int max_out = 0;
    // top-p sampling in generate (temp <= 0: greedy): one uniform draw per step, uploaded
    // before the steps run; a key scratch for vocabularies past what the kernel holds in
    // registers
    float smp_temp = 0.0f, smp_top_p = 1.0f;
    float* draws = nullptr;
    uint32_t* smp_key = nullptr;
    int64_t host_pos = 0;
    // the decode step captured as hipGraphs: graph[0] holds one step, graph[1] GRAPH_STEPS
    // consecutive steps (one graph launch per GRAPH_STEPS tokens); both built on the first
    // graph-mode call for a key
    hipGraphExec_t graph[2] = {nullptr, nullptr};
    // what the captured steps were built for: penalty bits (the value is a kernel argument),
    // kv_f16, rope_per_token, sampling temp and top_p bits
    uint32_t graph_key[5] = {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};
    int64_t graph_builds = 0;
};

static Llama* L_(tl_hip_llama* h) { return reinterpret_cast<Llama*>(h); }

static void free_graph(Llama* m) {
    for (hipGraphExec_t& g : m->graph) {
        if (g) {
            (void)hipGraphExecDestroy(g);
            g = nullptr;
        }
    }
}

// Steps per multi-step decode graph.  Every step reads its position, input token and output
// slot from device memory, so consecutive copies of the step replay correctly; one graph
// launch then carries the launch overhead of GRAPH_STEPS tokens.
constexpr int GRAPH_STEPS = 8;

static int alloc_kv(Llama* m) {
    for (void* p : m->kc) dev_free(p);
    for (void* p : m->vc) dev_free(p);
    m->kc.assign(m->nl, nullptr);
    m->vc.assign(m->nl, nullptr);
    size_t bytes = (size_t)m->KV * m->max_seq * m->hd * (m->kv_f16 ? 2 : 4);
    for (int l = 0; l < m->nl; l++) {
        m->kc[l] = dev_alloc(bytes);
        m->vc[l] = dev_alloc(bytes);
        if (!m->kc[l] || !m->vc[l]) return TL_HIP_ERR_ALLOC;
        TLH_CHECK_HIP(hipMemsetAsync(m->kc[l], 0, bytes, cur_stream()));
        TLH_CHECK_HIP(hipMemsetAsync(m->vc[l], 0, bytes, cur_stream()));
    }
    return TL_HIP_OK;
}

// Activation buffers for n tokens per call.  A failed grow leaves no buffer at all and
// max_tok 0, so the next call of any size allocates again instead of running on freed memory;
// the captured decode step (which holds the old pointers) is dropped first.
static int ensure_tokens(Llama* m, int64_t n) {
    if (n <= m->max_tok) return TL_HIP_OK;
    free_graph(m);
    m->max_tok = 0;
    float** bufs[] = {&m->x, &m->h, &m->qkv, &m->q, &m->ao, &m->t, &m->gu, &m->act};
    for (float** b : bufs) {
        dev_free(*b);
        *b = nullptr;
    }
    dev_free(m->ids);
    dev_free(m->ws);
    dev_free(m->xa16);
    dev_free(m->xb16);
    m->ids = nullptr;
    m->ws = nullptr;
    m->xa16 = m->xb16 = nullptr;
    m->ws_floats = 0;
    const int64_t qkv_w = m->D + 2 * (int64_t)m->KV * m->hd;
    m->x = (float*)dev_alloc(n * m->D * 4);
    m->h = (float*)dev_alloc(n * m->D * 4);
    m->qkv = (float*)dev_alloc(n * qkv_w * 4);
    m->q = (float*)dev_alloc(n * m->D * 4);
    m->ao = (float*)dev_alloc(n * m->D * 4);
    m->t = (float*)dev_alloc(n * m->D * 4);
    m->gu = (float*)dev_alloc(n * std::max(2 * (int64_t)m->F, qkv_w) * 4);  // also the q|k|v segment staging
    m->act = (float*)dev_alloc(n * (int64_t)m->F * 4);
    m->ids = (int32_t*)dev_alloc(n * 4);
    m->xa16 = (_Float16*)dev_alloc(n * m->D * 2);
    m->xb16 = (_Float16*)dev_alloc(n * (int64_t)m->F * 2);
    // attention workspace: B = n queries, splits of 64 positions over max_seq (the grouped-query
    // kernel's smallest split; 128-position splits use half of it)
    int nsplit = 2 * (int)cdiv(m->max_seq, 128);
    m->ws_floats = attn_workspace_floats((int)n, m->KV, m->H / m->KV, m->hd, nsplit);
    m->ws = (float*)dev_alloc(m->ws_floats * 4);
    bool ok = m->ids && m->ws && m->xa16 && m->xb16;
    for (float** b : bufs) ok = ok && *b;
    if (!ok) {
        for (float** b : bufs) {
            dev_free(*b);
            *b = nullptr;
        }
        void** rest[] = {(void**)&m->ids, (void**)&m->ws, (void**)&m->xa16, (void**)&m->xb16};
        for (void** b : rest) {
            dev_free(*b);
            *b = nullptr;
        }
        m->ws_floats = 0;
        return TL_HIP_ERR_ALLOC;
    }
    m->max_tok = n;
    return TL_HIP_OK;
}

static void release_w(QWeight* w) {
    if (w) tl_hip_qtensor_release(reinterpret_cast<tl_hip_qtensor*>(w));
}

static int try_merge(Llama* m, int layer) {
    auto& S = m->stage;
    const int base = layer * 5;
    if (!S[base].empty() && !S[base + 1].empty() && !S[base + 2].empty()) {
        // q | k | v in runs of equal type, each run one row-concatenated weight
        const int64_t rows[3] = {m->D, (int64_t)m->KV * m->hd, (int64_t)m->KV * m->hd};
        std::vector<Seg> segs;
        int64_t off = 0;
        for (int i = 0; i < 3;) {
            const int ty = m->stage_type[base + i];
            int j = i;
            std::vector<uint8_t> cat;
            int64_t nrows = 0;
            while (j < 3 && m->stage_type[base + j] == ty) {
                cat.insert(cat.end(), S[base + j].begin(), S[base + j].end());
                nrows += rows[j];
                j++;
            }
            int64_t shape[2] = {nrows, m->D};
            tl_hip_qtensor* q = tl_hip_qtensor_new(ty, cat.data(), cat.size(), shape, 2);
            if (!q) {
                for (auto& sg : segs) release_w(sg.w);
                return tl_hip_last_status();
            }
            segs.push_back(Seg{Q(q), off});
            off += nrows;
            i = j;
        }
        for (auto& sg : m->qkv_segs[layer]) release_w(sg.w);
        m->qkv_segs[layer] = segs;
        for (int i = 0; i < 3; i++) std::vector<uint8_t>().swap(S[base + i]);
    }
    if (!S[base + 3].empty() && !S[base + 4].empty()) {
        const int ty = m->stage_type[base + 3], tu = m->stage_type[base + 4];
        release_w(m->wgu[layer]);
        release_w(m->wg[layer]);
        release_w(m->wu[layer]);
        m->wgu[layer] = m->wg[layer] = m->wu[layer] = nullptr;
        if (ty == tu) {
            // rows interleaved (gate_0, up_0, gate_1, up_1, ...): the SwiGLU epilogue of the
            // matvec then sees both halves of an output in one workgroup
            const size_t row_bytes = ggml_row_bytes(ty, m->D);
            std::vector<uint8_t> cat(S[base + 3].size() * 2);
            for (int64_t i = 0; i < m->F; i++) {
                std::memcpy(cat.data() + (2 * i) * row_bytes, S[base + 3].data() + i * row_bytes, row_bytes);
                std::memcpy(cat.data() + (2 * i + 1) * row_bytes, S[base + 4].data() + i * row_bytes, row_bytes);
            }
            int64_t shape[2] = {2 * (int64_t)m->F, m->D};
            tl_hip_qtensor* q = tl_hip_qtensor_new(ty, cat.data(), cat.size(), shape, 2);
            if (!q) return tl_hip_last_status();
            m->wgu[layer] = Q(q);
        } else {
            int64_t shape[2] = {(int64_t)m->F, m->D};
            tl_hip_qtensor* g = tl_hip_qtensor_new(ty, S[base + 3].data(), S[base + 3].size(), shape, 2);
            if (!g) return tl_hip_last_status();
            tl_hip_qtensor* u = tl_hip_qtensor_new(tu, S[base + 4].data(), S[base + 4].size(), shape, 2);
            if (!u) {
                tl_hip_qtensor_release(g);
                return tl_hip_last_status();
            }
            m->wg[layer] = Q(g);
            m->wu[layer] = Q(u);
        }
        for (int i = 3; i < 5; i++) std::vector<uint8_t>().swap(S[base + i]);
    }
    return TL_HIP_OK;
}

// y[n, N] = x[n, K] . W^T (+ residual); matvec for n <= 4, GEMM otherwise
static int linear(const QWeight* w, const float* x, float* y, int64_t n, const float* res,
                  float* tmp, int f16, hipStream_t s) {
    if (n <= 4) return launch_quant_matvec(w, x, y, n, s, res);
    if (!res) return launch_quant_gemm(w, x, y, n, s, f16);
    int rc = launch_quant_gemm(w, x, tmp, n, s, f16);
    if (rc) return rc;
    k_add_inplace<<<cdiv(n * w->n, 256), 256, 0, s>>>(y, tmp, n * w->n);
    return TL_HIP_OK;
}

static int check_ready(Llama* m) {
    for (int l = 0; l < m->nl; l++)
        if (m->qkv_segs[l].empty() || !m->wo[l] || !(m->wgu[l] || (m->wg[l] && m->wu[l])) || !m->wdown[l] ||
            !m->attn_norm[l] || !m->ffn_norm[l]) {
            set_error(TL_HIP_ERR_ARG, "ArgumentError: layer %d is missing weights", l);
            return TL_HIP_ERR_ARG;
        }
    if (!m->lm || !m->out_norm || !m->emb) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: LM head, output norm or embedding missing");
        return TL_HIP_ERR_ARG;
    }
    return TL_HIP_OK;
}

// Whether the f16 prefill applies RoPE and the KV append in the epilogues of its [q | k | v]
// GEMMs rather than in k_rope_kv after plain GEMMs: the same values either way.
static std::atomic<bool> g_rope_epilogue{true};

// RoPE on the q|k rows of n tokens and the k / v append at the device position (prefill).
static void prefill_rope_kv(Llama* m, int l, int n, hipStream_t s) {
    const int64_t hd = m->hd;
    int64_t work = (int64_t)n * ((m->H + m->KV) * hd / 2 + m->KV * hd);
    if (m->kv_f16)
        k_rope_kv<__half><<<cdiv(work, 256), 256, 0, s>>>(m->qkv, m->q, (__half*)m->kc[l], (__half*)m->vc[l],
                                                         m->cos_t, m->sin_t, m->pos, n, m->H, m->KV, (int)hd,
                                                         m->max_seq, m->rope_per_token);
    else
        k_rope_kv<float><<<cdiv(work, 256), 256, 0, s>>>(m->qkv, m->q, (float*)m->kc[l], (float*)m->vc[l],
                                                        m->cos_t, m->sin_t, m->pos, n, m->H, m->KV, (int)hd,
                                                        m->max_seq, m->rope_per_token);
}

// Causal attention of n prompt rows: query i (absolute position pos + i) attends cache
// positions 0 .. pos + i.  The f16 prefill uses the MFMA form, the f32 path the grouped-query
// split form.  Output to m->ao (f32) or, with out16, to f16 in GEMM operand order.
static int prefill_attention(Llama* m, int l, int n, int f16, _Float16* out16, int order, hipStream_t s) {
    const int64_t hd = m->hd;
    const int kvt = m->kv_f16 ? TL_HIP_F16 : TL_HIP_F32;
    if (f16 && attention_prefill_supported(kvt, m->H, m->KV, (int)hd))
        return launch_attention_prefill(m->q, m->kc[l], m->vc[l], m->ao, n, m->H, m->KV, (int)hd, m->max_seq,
                                        m->pos, 0, 1.0f / sqrtf((float)hd), s, out16, order);
    int rc;
    if (attention_gq_supported(kvt, m->H, m->KV, (int)hd))
        rc = launch_attention_gq(m->q, m->kc[l], m->vc[l], m->ao, m->ws, n, m->H, m->KV, (int)hd, m->max_seq, 0, 0,
                                 m->pos, 1, 1, attention_gq_splits(m->host_pos + n), 1.0f / sqrtf((float)hd), s);
    else
        rc = launch_attention(m->q, m->kc[l], m->vc[l], kvt, m->ao, m->ws, n, m->H, m->KV, (int)hd, m->max_seq, 0,
                              0, m->pos, 1, 1, 64, (int)cdiv(m->host_pos + n, 64), 1.0f / sqrtf((float)hd), s);
    if (rc == TL_HIP_OK && out16) rc = launch_x_to_f16q(m->ao, out16, n, m->D, order, s);
    return rc;
}

// The f16 prefill of a layer with its activations handed between the GEMMs as f16 operand
// words: RMSNorm -> f16 (qkv GEMM input), attention -> f16 (o-proj input), o-proj + residual
// in the GEMM epilogue, RMSNorm -> f16, gate/up GEMM with SwiGLU in the epilogue -> f16
// (down input), down + residual.  Same values as the unfused path, where each GEMM input is
// converted from the f32 producer output.
static bool fused_layer_ok(const Llama* m, int l) {
    const QWeight* wgu = m->wgu[l];
    if (!wgu || wgu->n % 64 || m->D % 32 || m->D > 8192) return false;
    const int oq = f16q_order(m->qkv_segs[l][0].w->ggml_type);
    for (const Seg& sg : m->qkv_segs[l])  // one operand order for the shared input, K in steps of 128
        if (sg.w->nb % 4 || f16q_order(sg.w->ggml_type) != oq) return false;
    return m->wo[l]->nb % 4 == 0 && wgu->nb % 4 == 0 && m->wdown[l]->nb % 4 == 0;
}

// the f16 GEMM of a prefill; a Q4_K weight gets its unit scales on first use.  With pend, a
// split-K launch leaves its partial slices there instead of summing them into y.
struct Pending {
    float* part = nullptr;  // nsp slices of [n, D] still to be added (with the residual) into x
    int nsp = 0;
};
static int gemm16(QWeight* w, const _Float16* x16, float* y, int n, const GemmEpi& ep, hipStream_t s,
                  Pending* pend = nullptr) {
    const int rc = q4k_build_unit_scales(w, s);
    if (rc) return rc;
    return pend ? launch_gemm_f16q(w, x16, y, n, ep, s, false, nullptr, &pend->part, &pend->nsp)
                : launch_gemm_f16q(w, x16, y, n, ep, s);
}

// x += pending partial slices (the residual GEMM's deferred split-K sum), then free them
static int flush_pending(Pending& p, float* x, int64_t mn, hipStream_t s) {
    if (!p.part) return TL_HIP_OK;
    const int rc = launch_splitk_sum(p.part, x, x, mn, p.nsp, s);
    dev_free_on(p.part, s);
    p = Pending{};
    return rc;
}

// A residual GEMM that splits K (the o-projection and down projection at short prompts, and
// at 512 tokens, where they have one tile per CU) leaves its partial slices to the RMSNorm
// that reads the residual next: that kernel adds them into x in slice order -- the split-K
// sum's own additions -- and normalises the row, one launch instead of two.  The down
// projection's slices are carried to the next layer's first RMSNorm (pend).
static int prefill_layer_fused(Llama* m, int l, int n, hipStream_t s, Pending& pend) {
    const int64_t D = m->D, qkv_w = D + 2 * (int64_t)m->KV * m->hd;
    const GemmEpi plain{GEMM_PLAIN, nullptr, nullptr, 0}, res{GEMM_RES, m->x, nullptr, 0};
    int rc;
    const int oq = f16q_order(m->qkv_segs[l][0].w->ggml_type);
    rc = launch_rmsnorm_f16q(m->x, m->attn_norm[l], m->xa16, n, D, m->eps, oq, s, pend.part, pend.nsp);
    if (pend.part) dev_free_on(pend.part, s);
    pend = Pending{};
    if (rc) return rc;
    if (g_rope_epilogue.load(std::memory_order_relaxed) && m->hd >= 4 && (m->hd & (m->hd - 1)) == 0) {
        // RoPE and the KV append ride in the epilogue of each [q | k | v] weight's GEMM
        GemmEpi rope{GEMM_ROPE_KV, nullptr, nullptr, 0};
        rope.rk.q = m->q;
        rope.rk.kc = m->kc[l];
        rope.rk.vc = m->vc[l];
        rope.rk.ct = m->cos_t;
        rope.rk.st = m->sin_t;
        rope.rk.pos = m->pos;
        rope.rk.H = m->H;
        rope.rk.KV = m->KV;
        rope.rk.hd = (int)m->hd;
        rope.rk.per_token = m->rope_per_token;
        rope.rk.kv_f16 = m->kv_f16 ? 1 : 0;
        rope.rk.max_seq = m->max_seq;
        while ((1 << rope.rk.hd_shift) < m->hd) rope.rk.hd_shift++;
        for (const Seg& sg : m->qkv_segs[l]) {  // y (m->qkv) is not written in this mode
            rope.rk.col_off = (int)sg.row_off;
            if ((rc = gemm16(sg.w, m->xa16, m->qkv, n, rope, s))) return rc;
        }
    } else if (m->qkv_segs[l].size() == 1) {
        if ((rc = gemm16(m->qkv_segs[l][0].w, m->xa16, m->qkv, n, plain, s))) return rc;
        prefill_rope_kv(m, l, n, s);
    } else {
        for (const Seg& sg : m->qkv_segs[l]) {  // each segment's columns of the [n, qkv_w] rows
            if ((rc = gemm16(sg.w, m->xa16, m->gu, n, plain, s))) return rc;
            TLH_CHECK_HIP(hipMemcpy2DAsync(m->qkv + sg.row_off, qkv_w * 4, m->gu, sg.w->n * 4, sg.w->n * 4, n,
                                           hipMemcpyDeviceToDevice, s));
        }
        prefill_rope_kv(m, l, n, s);
    }
    if ((rc = prefill_attention(m, l, n, 1, m->xa16, f16q_order(m->wo[l]->ggml_type), s))) return rc;
    Pending op;
    if ((rc = gemm16(m->wo[l], m->xa16, m->x, n, res, s, &op))) return rc;
    rc = launch_rmsnorm_f16q(m->x, m->ffn_norm[l], m->xa16, n, D, m->eps, f16q_order(m->wgu[l]->ggml_type), s, op.part,
                             op.nsp);
    if (op.part) dev_free_on(op.part, s);
    if (rc) return rc;
    const GemmEpi glu{GEMM_GLU16, nullptr, m->xb16, f16q_order(m->wdown[l]->ggml_type)};
    if ((rc = gemm16(m->wgu[l], m->xa16, nullptr, n, glu, s))) return rc;
    return gemm16(m->wdown[l], m->xb16, m->x, n, res, s, &pend);
}

// Enqueues one forward over n tokens whose ids are already in m->ids (device); leaves the
// last row's logits in m->logits and advances the device position by n.
static int enqueue_forward(Llama* m, int n, int f16, hipStream_t s) {
    const int64_t D = m->D;
    const int64_t qkv_w = D + 2 * (int64_t)m->KV * m->hd;
    int rc;
    k_embed<<<cdiv(n * D, 256), 256, 0, s>>>(m->emb, m->ids, m->x, n, D);
    Pending pend;  // a fused layer's deferred down-projection sum
    struct Guard {  // frees undelivered partial slices on an error return
        Pending& p;
        hipStream_t s;
        ~Guard() { if (p.part) dev_free_on(p.part, s); }
    } guard{pend, s};
    for (int l = 0; l < m->nl; l++) {
        if (f16 && n > 4 && fused_layer_ok(m, l)) {
            if ((rc = prefill_layer_fused(m, l, n, s, pend))) return rc;
            continue;
        }
        if ((rc = flush_pending(pend, m->x, (int64_t)n * D, s))) return rc;
        if ((rc = launch_rmsnorm(m->x, nullptr, m->attn_norm[l], m->h, n, D, m->eps, 0, s))) return rc;
        if (m->qkv_segs[l].size() == 1) {
            if ((rc = linear(m->qkv_segs[l][0].w, m->h, m->qkv, n, nullptr, nullptr, f16, s))) return rc;
        } else {
            for (const Seg& sg : m->qkv_segs[l]) {  // each segment's columns of the [n, qkv_w] rows
                if ((rc = linear(sg.w, m->h, m->gu, n, nullptr, nullptr, f16, s))) return rc;
                TLH_CHECK_HIP(hipMemcpy2DAsync(m->qkv + sg.row_off, qkv_w * 4, m->gu, sg.w->n * 4, sg.w->n * 4, n,
                                               hipMemcpyDeviceToDevice, s));
            }
        }
        prefill_rope_kv(m, l, n, s);
        rc = prefill_attention(m, l, n, f16, nullptr, 0, s);
        if (rc) return rc;
        if ((rc = linear(m->wo[l], m->ao, m->x, n, m->x, m->t, f16, s))) return rc;
        if ((rc = launch_rmsnorm(m->x, nullptr, m->ffn_norm[l], m->h, n, D, m->eps, 0, s))) return rc;
        if (m->wgu[l]) {
            if ((rc = linear(m->wgu[l], m->h, m->gu, n, nullptr, nullptr, f16, s))) return rc;
            k_swiglu_rows<<<cdiv(n * (int64_t)m->F, 256), 256, 0, s>>>(m->gu, m->act, n, m->F);
        } else {
            float* up = m->gu + (int64_t)n * m->F;
            if ((rc = linear(m->wg[l], m->h, m->gu, n, nullptr, nullptr, f16, s))) return rc;
            if ((rc = linear(m->wu[l], m->h, up, n, nullptr, nullptr, f16, s))) return rc;
            if ((rc = launch_swiglu(m->gu, up, m->act, (int64_t)n * m->F, 0, s))) return rc;
        }
        if ((rc = linear(m->wdown[l], m->act, m->x, n, m->x, m->t, f16, s))) return rc;
    }
    if ((rc = flush_pending(pend, m->x, (int64_t)n * D, s))) return rc;
    k_advance<<<1, 64, 0, s>>>(m->pos, n);
    if ((rc = launch_rmsnorm(m->x + (int64_t)(n - 1) * D, nullptr, m->out_norm, m->h, 1, D, m->eps, 0, s))) return rc;
    if ((rc = launch_quant_matvec(m->lm, m->h, m->logits, 1, s, nullptr))) return rc;
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TL_HIP_OK : hip_fail(e, "forward launch");
}

// One greedy decode step from the token in m->tok (device), five kernels per layer:
//   [embed (layer 0) +] RMSNorm + q|k|v matvec + RoPE + KV append   (EPI_ROPE_KV)
//   attention over the cache (one workgroup per query head; the split form beyond 4096)
//   o-proj matvec + residual                                         (EPI_RES)
//   RMSNorm + gate/up matvec + SwiGLU                                (EPI_GLU)
//   down matvec + residual                                           (EPI_RES)
// and one more for the output RMSNorm + LM head + penalty + argmax + step bookkeeping.
static int enqueue_step(Llama* m, float penalty, hipStream_t s) {
    const int64_t hd = m->hd;
    const int nsplit = (int)cdiv(m->max_seq, 64);
    int rc;
    for (int l = 0; l < m->nl; l++) {
        MvArgs a = {};
        a.eps = m->eps;
        if (l == 0) {  // the token's embedding row, also stored as the residual stream
            a.x = m->emb;
            a.embed_id = m->tok;
            a.x_out = m->x;
        } else {
            a.x = m->x;
        }
        a.norm_w = m->attn_norm[l];
        a.pos = m->pos;
        a.cos_t = m->cos_t;
        a.sin_t = m->sin_t;
        a.q_out = m->q;
        a.kc = m->kc[l];
        a.vc = m->vc[l];
        a.q_rows = m->D;
        a.kv_rows = m->KV * (int)hd;
        a.hd = (int)hd;
        a.kv_f16 = m->kv_f16;
        a.max_seq = m->max_seq;
        // a projection in two weight types (Q4_K q | k with Q6_K v, llama.cpp's Q4_K_M) in one launch
        rc = -1;
        if (m->qkv_segs[l].size() == 2) {
            a.row_off = m->qkv_segs[l][0].row_off;
            rc = launch_mv_pair(m->qkv_segs[l][0].w, m->qkv_segs[l][1].w, a, m->qkv_segs[l][1].row_off, l == 0, s);
            if (rc > 0) return rc;
        }
        if (rc == -1)
            for (const Seg& sg : m->qkv_segs[l]) {
                a.row_off = sg.row_off;
                if ((rc = launch_mv(sg.w, a, 1, EPI_ROPE_KV, true, l == 0, s))) return rc;
            }
        // caches up to 4096 positions: ATTN_SHARES workgroups per query head (each a share of
        // the positions) in a single launch, their records merged by the o-projection as it
        // stages its input (the split form's merge launch costs more than it saves here)
        const bool qh = m->max_seq <= 4096 &&
                        attention_qh_supported(m->kv_f16 ? TL_HIP_F16 : TL_HIP_F32, (int)hd, m->max_seq);
        const bool shares = qh && hd % 4 == 0 && m->ws_floats >= (size_t)m->H * ATTN_SHARES * (hd + 4);
        if (qh)
            rc = launch_attention_qh(m->q, m->kc[l], m->vc[l], m->kv_f16 ? TL_HIP_F16 : TL_HIP_F32, m->ao, 1, m->H,
                                     m->KV, (int)hd, m->max_seq, 0, 0, m->pos, 1, 0, 1.0f / sqrtf((float)hd), s,
                                     shares ? m->ws : nullptr, shares ? ATTN_SHARES : 1);
        else if (attention_gq_supported(m->kv_f16 ? TL_HIP_F16 : TL_HIP_F32, m->H, m->KV, (int)hd))
            rc = launch_attention_gq(m->q, m->kc[l], m->vc[l], m->ao, m->ws, 1, m->H, m->KV, (int)hd, m->max_seq, 0,
                                     0, m->pos, 1, 0, attention_gq_splits(m->max_seq), 1.0f / sqrtf((float)hd), s);
        else
            rc = launch_attention(m->q, m->kc[l], m->vc[l], m->kv_f16 ? TL_HIP_F16 : TL_HIP_F32, m->ao, m->ws, 1,
                                  m->H, m->KV, (int)hd, m->max_seq, 0, 0, m->pos, 1, 0, 64, nsplit,
                                  1.0f / sqrtf((float)hd), s);
        if (rc) return rc;
        MvArgs o = {};
        o.x = shares ? nullptr : m->ao;
        o.attn_rec = shares ? m->ws : nullptr;
        o.attn_hd = (int)hd;
        o.y = m->x;
        o.res = m->x;
        if ((rc = launch_mv(m->wo[l], o, 1, EPI_RES, false, false, s))) return rc;
        MvArgs g = {};
        g.x = m->x;
        g.norm_w = m->ffn_norm[l];
        g.eps = m->eps;
        if (m->wgu[l]) {
            g.y = m->act;
            if ((rc = launch_mv(m->wgu[l], g, 1, EPI_GLU, true, false, s))) return rc;
        } else {
            g.y = m->gu;
            if ((rc = launch_mv(m->wg[l], g, 1, EPI_PLAIN, true, false, s))) return rc;
            g.y = m->gu + m->F;
            if ((rc = launch_mv(m->wu[l], g, 1, EPI_PLAIN, true, false, s))) return rc;
            if ((rc = launch_swiglu(m->gu, m->gu + m->F, m->act, m->F, 0, s))) return rc;
        }
        MvArgs d = {};
        d.x = m->act;
        d.y = m->x;
        d.res = m->x;
        if ((rc = launch_mv(m->wdown[l], d, 1, EPI_RES, false, false, s))) return rc;
    }
    MvArgs h = {};
    h.x = m->x;
    h.norm_w = m->out_norm;
    h.eps = m->eps;
    h.y = m->logits;
    h.plogits = m->plogits;
    h.seen = penalty != 1.0f ? m->seen : nullptr;
    h.seen_out = penalty != 1.0f ? m->seen : nullptr;
    h.penalty = penalty;
    h.part_v = m->am_v;
    h.part_i = m->am_i;
    h.part_nan = m->am_nan;
    h.tok_out = m->tok;
    h.out_ids = m->out_ids;
    h.step = m->step;
    h.pos_inc = m->pos;
    h.max_out = m->max_out;
    h.smp_temp = m->smp_temp;
    h.smp_top_p = m->smp_top_p;
    h.smp_draws = m->draws;
    h.smp_key = m->smp_key;
    return launch_mv(m->lm, h, 1, EPI_ARGMAX, true, false, s);
}

}  // namespace tlhip

using namespace tlhip;

extern "C" {

tl_hip_llama* tl_hip_llama_new(int n_layers, int d_model, int n_heads, int n_kv_heads, int ffn_dim,
                               int vocab, float eps, float rope_theta, int max_seq) {
    if (!state()) return nullptr;
    if (n_layers <= 0 || d_model <= 0 || n_heads <= 0 || n_kv_heads <= 0 || ffn_dim <= 0 || vocab <= 0 ||
        max_seq <= 0 || d_model % n_heads || n_heads % n_kv_heads || (d_model / n_heads) % 2 ||
        d_model % 32 || ffn_dim % 32) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: invalid decoder configuration");
        return nullptr;
    }
    Llama* m = new Llama();
    m->nl = n_layers;
    m->D = d_model;
    m->H = n_heads;
    m->KV = n_kv_heads;
    m->hd = d_model / n_heads;
    m->F = ffn_dim;
    m->V = vocab;
    m->max_seq = max_seq;
    m->eps = eps;
    m->theta = rope_theta;
    m->qkv_segs.assign(n_layers, {});
    m->wo.assign(n_layers, nullptr);
    m->wgu.assign(n_layers, nullptr);
    m->wg.assign(n_layers, nullptr);
    m->wu.assign(n_layers, nullptr);
    m->wdown.assign(n_layers, nullptr);
    m->stage.assign((size_t)n_layers * 5, {});
    m->stage_type.assign((size_t)n_layers * 5, -1);
    m->attn_norm.assign(n_layers, nullptr);
    m->ffn_norm.assign(n_layers, nullptr);
    hipStream_t s = cur_stream();
    // chatbot.tl:151-152: rope_new_cos(head_dim, table_len, theta) -> [table_len, head_dim]
    m->cos_t = (float*)dev_alloc((size_t)max_seq * m->hd * 4);
    m->sin_t = (float*)dev_alloc((size_t)max_seq * m->hd * 4);
    m->logits = (float*)dev_alloc((size_t)vocab * 4);
    m->plogits = (float*)dev_alloc((size_t)vocab * 4);
    m->pos = (int32_t*)dev_alloc(4);
    m->tok = (int32_t*)dev_alloc(4);
    m->step = (int32_t*)dev_alloc(4);
    m->seen = (uint8_t*)dev_alloc(vocab);
    const int parts = mv_partials(vocab);
    m->am_v = (float*)dev_alloc((size_t)parts * 4);
    m->am_i = (int32_t*)dev_alloc((size_t)parts * 4);
    m->am_nan = (int32_t*)dev_alloc((size_t)parts * 4);
    // generated ids of one generate call: at most max_seq (the cache bounds the steps), so the
    // captured step never has to be rebuilt for a longer call
    m->out_ids = (int32_t*)dev_alloc((size_t)max_seq * 4);
    m->max_out = max_seq;
    m->draws = (float*)dev_alloc((size_t)max_seq * 4);
    const int kw = sample_key_words(vocab);
    if (kw) m->smp_key = (uint32_t*)dev_alloc((size_t)kw * 4);
    int rc = (m->cos_t && m->sin_t && m->logits && m->plogits && m->pos && m->tok && m->step && m->seen &&
              m->am_v && m->am_i && m->am_nan && m->out_ids && m->draws && (!kw || m->smp_key))
                 ? TL_HIP_OK : TL_HIP_ERR_ALLOC;
    if (rc == TL_HIP_OK) rc = launch_rope_table(m->cos_t, max_seq, m->hd, rope_theta, 0, s);
    if (rc == TL_HIP_OK) rc = launch_rope_table(m->sin_t, max_seq, m->hd, rope_theta, 1, s);
    if (rc == TL_HIP_OK) rc = alloc_kv(m);
    if (rc == TL_HIP_OK) rc = ensure_tokens(m, 1);
    if (rc == TL_HIP_OK) rc = tl_hip_llama_reset(reinterpret_cast<tl_hip_llama*>(m));
    if (rc != TL_HIP_OK) {
        tl_hip_llama_free(reinterpret_cast<tl_hip_llama*>(m));
        return nullptr;
    }
    return reinterpret_cast<tl_hip_llama*>(m);
}

int tl_hip_llama_free(tl_hip_llama* h) {
    if (!h) return TL_HIP_OK;
    Llama* m = L_(h);
    (void)hipStreamSynchronize(cur_stream());
    free_graph(m);
    auto rel = [](QWeight* w) {
        if (w) tl_hip_qtensor_release(reinterpret_cast<tl_hip_qtensor*>(w));
    };
    for (int l = 0; l < m->nl; l++) {
        for (auto& sg : m->qkv_segs[l]) rel(sg.w);
        rel(m->wo[l]);
        rel(m->wgu[l]);
        rel(m->wg[l]);
        rel(m->wu[l]);
        rel(m->wdown[l]);
        dev_free(m->attn_norm[l]);
        dev_free(m->ffn_norm[l]);
    }
    rel(m->lm);
    for (void* p : m->kc) dev_free(p);
    for (void* p : m->vc) dev_free(p);
    void* bufs[] = {m->out_norm, m->emb, m->cos_t, m->sin_t, m->x, m->h, m->qkv, m->q, m->ao, m->t, m->gu,
                    m->act, m->logits, m->plogits, m->ws, m->ids, m->pos, m->tok, m->step, m->out_ids, m->seen,
                    m->am_v, m->am_i, m->am_nan, m->xa16, m->xb16, m->draws, m->smp_key};
    for (void* p : bufs) dev_free(p);
    delete m;
    return TL_HIP_OK;
}

int tl_hip_llama_set_linear(tl_hip_llama* h, int layer, int which, int ggml_type, const uint8_t* data,
                            size_t nbytes) {
    if (!h || !data) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model or data");
        return TL_HIP_ERR_NULL;
    }
    Llama* m = L_(h);
    if (layer < -1 || layer >= m->nl || (layer >= 0 && (which < 0 || which > 6))) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: weight slot (%d, %d)", layer, which);
        return TL_HIP_ERR_ARG;
    }
    free_graph(m);
    const int64_t D = m->D, KVd = (int64_t)m->KV * m->hd, F = m->F;
    if (layer == -1 || which == 3 || which == 6) {
        int64_t shape[2];
        if (layer == -1) { shape[0] = m->V; shape[1] = D; }
        else if (which == 3) { shape[0] = D; shape[1] = D; }
        else { shape[0] = D; shape[1] = F; }
        tl_hip_qtensor* q = tl_hip_qtensor_new(ggml_type, data, nbytes, shape, 2);
        if (!q) return tl_hip_last_status();
        QWeight** slot = layer == -1 ? &m->lm : (which == 3 ? &m->wo[layer] : &m->wdown[layer]);
        if (*slot) tl_hip_qtensor_release(reinterpret_cast<tl_hip_qtensor*>(*slot));
        *slot = Q(q);
        return TL_HIP_OK;
    }
    // q k v gate up: validate the part, stage it, and merge once a group is complete
    int part = which <= 2 ? which : which - 1;  // 0 q, 1 k, 2 v, 3 gate, 4 up
    int64_t rows = which == 0 ? D : (which <= 2 ? KVd : F);
    int64_t numel = rows * D;
    if (!ggml_block_elems(ggml_type)) {
        set_error(TL_HIP_ERR_TYPE, "TypeMismatch: ggml type %d has no device residency", ggml_type);
        return TL_HIP_ERR_TYPE;
    }
    if (D % ggml_block_elems(ggml_type)) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: rows of %lld do not hold whole %s blocks", (long long)D,
                  ggml_type_name(ggml_type));
        return TL_HIP_ERR_SHAPE;
    }
    const size_t want = (size_t)rows * ggml_row_bytes(ggml_type, D);
    (void)numel;
    if (nbytes != want) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: Data size mismatch: expected %zu, got %zu", want, nbytes);
        return TL_HIP_ERR_ARG;
    }
    m->stage[layer * 5 + part].assign(data, data + nbytes);
    m->stage_type[layer * 5 + part] = ggml_type;
    return try_merge(m, layer);
}

int tl_hip_llama_set_norm(tl_hip_llama* h, int layer, int which, const float* w) {
    if (!h || !w) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model or weight");
        return TL_HIP_ERR_NULL;
    }
    Llama* m = L_(h);
    if (layer < -1 || layer >= m->nl || (layer >= 0 && which != 0 && which != 1)) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: norm slot (%d, %d)", layer, which);
        return TL_HIP_ERR_ARG;
    }
    float** slot = layer == -1 ? &m->out_norm : (which == 0 ? &m->attn_norm[layer] : &m->ffn_norm[layer]);
    if (!*slot) {
        *slot = (float*)dev_alloc((size_t)m->D * 4);
        if (!*slot) return TL_HIP_ERR_ALLOC;
        free_graph(m);
    }
    TLH_CHECK_HIP(hipMemcpyAsync(*slot, w, (size_t)m->D * 4, hipMemcpyHostToDevice, cur_stream()));
    TLH_CHECK_HIP(hipStreamSynchronize(cur_stream()));
    return TL_HIP_OK;
}

int tl_hip_llama_set_embedding(tl_hip_llama* h, const float* table) {
    if (!h || !table) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model or table");
        return TL_HIP_ERR_NULL;
    }
    Llama* m = L_(h);
    size_t bytes = (size_t)m->V * m->D * 4;
    if (!m->emb) {
        m->emb = (float*)dev_alloc(bytes);
        if (!m->emb) return TL_HIP_ERR_ALLOC;
        free_graph(m);
    }
    TLH_CHECK_HIP(hipMemcpyAsync(m->emb, table, bytes, hipMemcpyHostToDevice, cur_stream()));
    TLH_CHECK_HIP(hipStreamSynchronize(cur_stream()));
    return TL_HIP_OK;
}

// One GGUF tensor as a host f32 vector of the expected shape (norms are tiny).
static int gguf_f32(tl_hip_gguf* g, const char* name, int64_t n, std::vector<float>* out) {
    tl_hip_tensor* t = tl_hip_gguf_get(g, name);
    if (!t) return tl_hip_last_status();
    int rc = TL_HIP_OK;
    if (tl_hip_tensor_numel(t) != n) {
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: '%s' has %lld elements, expected %lld", name,
                  (long long)tl_hip_tensor_numel(t), (long long)n);
        rc = TL_HIP_ERR_SHAPE;
    } else {
        out->resize((size_t)n);
        rc = tl_hip_tensor_to_host(t, out->data(), n);
    }
    tl_hip_tensor_release(t);
    return rc;
}

int tl_hip_llama_load_gguf(tl_hip_llama* h, tl_hip_gguf* g) {
    if (!h || !g) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model or gguf");
        return TL_HIP_ERR_NULL;
    }
    Llama* m = L_(h);
    static const char* kLin[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    const int64_t D = m->D, KVd = (int64_t)m->KV * m->hd, F = m->F;
    const int64_t want[7][2] = {{D, D}, {KVd, D}, {KVd, D}, {D, D}, {F, D}, {F, D}, {D, F}};
    char name[160];
    auto linear = [&](int layer, int which, const char* nm, int64_t n, int64_t k) -> int {
        int type = 0, rank = 0;
        int64_t shape[TL_HIP_MAX_RANK];
        uint64_t nbytes = 0;
        if (tl_hip_gguf_tensor_info(g, nm, &type, shape, &rank, &nbytes)) return tl_hip_last_status();
        if (rank != 2 || shape[0] != n || shape[1] != k) {
            set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: '%s' is not [%lld, %lld]", nm, (long long)n, (long long)k);
            return TL_HIP_ERR_SHAPE;
        }
        const uint8_t* data = tl_hip_gguf_tensor_data(g, nm, &nbytes);
        if (!data) return tl_hip_last_status();
        return tl_hip_llama_set_linear(h, layer, which, type, data, (size_t)nbytes);
    };
    std::vector<float> v;
    int rc;
    for (int l = 0; l < m->nl; l++) {
        for (int w = 0; w < 7; w++) {
            snprintf(name, sizeof(name), "blk.%d.%s.weight", l, kLin[w]);
            if ((rc = linear(l, w, name, want[w][0], want[w][1]))) return rc;
        }
        for (int w = 0; w < 2; w++) {
            snprintf(name, sizeof(name), "blk.%d.%s_norm.weight", l, w == 0 ? "attn" : "ffn");
            if ((rc = gguf_f32(g, name, D, &v))) return rc;
            if ((rc = tl_hip_llama_set_norm(h, l, w, v.data()))) return rc;
        }
    }
    if ((rc = gguf_f32(g, "output_norm.weight", D, &v))) return rc;
    if ((rc = tl_hip_llama_set_norm(h, -1, 0, v.data()))) return rc;
    if ((rc = linear(-1, 0, "output.weight", m->V, D))) return rc;
    // token_embd.weight: the f32 table (dequantized on the device when stored quantized)
    tl_hip_tensor* e = tl_hip_gguf_get(g, "token_embd.weight");
    if (!e) return tl_hip_last_status();
    const Tensor* et = reinterpret_cast<const Tensor*>(e);
    if (et->rank != 2 || et->shape[0] != m->V || et->shape[1] != D) {
        tl_hip_tensor_release(e);
        set_error(TL_HIP_ERR_SHAPE, "ShapeMismatch: token_embd.weight is not [%d, %lld]", m->V, (long long)D);
        return TL_HIP_ERR_SHAPE;
    }
    const size_t bytes = (size_t)m->V * D * 4;
    if (!m->emb) {
        m->emb = (float*)dev_alloc(bytes);
        if (!m->emb) {
            tl_hip_tensor_release(e);
            return TL_HIP_ERR_ALLOC;
        }
        free_graph(m);
    }
    hipError_t err = hipMemcpyAsync(m->emb, et->data, bytes, hipMemcpyDeviceToDevice, cur_stream());
    if (err == hipSuccess) err = hipStreamSynchronize(cur_stream());
    tl_hip_tensor_release(e);
    if (err != hipSuccess) return hip_fail(err, "embedding copy");
    return TL_HIP_OK;
}

int tl_hip_debug_prefill_rope_epilogue(int on) {
    if (on < 0) return g_rope_epilogue.load() ? 1 : 0;
    return g_rope_epilogue.exchange(on != 0) ? 1 : 0;
}

int tl_hip_llama_configure(tl_hip_llama* h, int kv_f16, int rope_per_token) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model");
        return TL_HIP_ERR_NULL;
    }
    Llama* m = L_(h);
    free_graph(m);
    m->rope_per_token = rope_per_token ? 1 : 0;
    if ((kv_f16 ? 1 : 0) != m->kv_f16) {
        m->kv_f16 = kv_f16 ? 1 : 0;
        int rc = alloc_kv(m);
        if (rc) return rc;
    }
    return tl_hip_llama_reset(h);
}

int tl_hip_llama_reset(tl_hip_llama* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model");
        return TL_HIP_ERR_NULL;
    }
    Llama* m = L_(h);
    TLH_CHECK_HIP(hipMemsetAsync(m->pos, 0, 4, cur_stream()));
    TLH_CHECK_HIP(hipStreamSynchronize(cur_stream()));
    m->host_pos = 0;
    return TL_HIP_OK;
}

int64_t tl_hip_llama_graph_builds(const tl_hip_llama* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model");
        return -1;
    }
    return reinterpret_cast<const Llama*>(h)->graph_builds;
}

int64_t tl_hip_llama_position(const tl_hip_llama* h) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model");
        return -1;
    }
    return reinterpret_cast<const Llama*>(h)->host_pos;
}

int tl_hip_llama_forward(tl_hip_llama* h, const int32_t* ids, int n, float* logits_out, int prefill_f16) {
    if (!h || !ids) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model or ids");
        return TL_HIP_ERR_NULL;
    }
    Llama* m = L_(h);
    int rc = check_ready(m);
    if (rc) return rc;
    if (n <= 0 || m->host_pos + n > m->max_seq) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: %d tokens at position %lld exceed max_seq %d", n,
                  (long long)m->host_pos, m->max_seq);
        return TL_HIP_ERR_ARG;
    }
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= m->V) {
            set_error(TL_HIP_ERR_INDEX, "IndexOutOfBounds: Embedding index %d out of range for vocab size %d",
                      ids[i], m->V);
            return TL_HIP_ERR_INDEX;
        }
    if ((rc = ensure_tokens(m, n))) return rc;
    hipStream_t s = cur_stream();
    TLH_CHECK_HIP(hipMemcpyAsync(m->ids, ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
    if ((rc = enqueue_forward(m, n, prefill_f16, s))) return rc;
    m->host_pos += n;
    if (logits_out)
        TLH_CHECK_HIP(hipMemcpyAsync(logits_out, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost, s));
    TLH_CHECK_HIP(hipStreamSynchronize(s));
    return TL_HIP_OK;
}

int32_t tl_hip_llama_sample_greedy(tl_hip_llama* h, double repetition_penalty, const int32_t* history,
                                   int n_history) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model");
        return -1;
    }
    Llama* m = L_(h);
    if (repetition_penalty <= 0.0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: repetition penalty must be positive");
        return -1;
    }
    hipStream_t s = cur_stream();
    const float pen = (float)repetition_penalty;
    const float* lg = m->logits;
    if (pen != 1.0f) {
        std::vector<uint8_t> seen(m->V, 0);
        for (int i = 0; i < n_history; i++)
            if (history && history[i] >= 0 && history[i] < m->V) seen[history[i]] = 1;
        if (hipMemcpyAsync(m->seen, seen.data(), m->V, hipMemcpyHostToDevice, s) != hipSuccess ||
            launch_rep_penalty(m->logits, m->seen, m->plogits, 1, m->V, pen, s) != TL_HIP_OK) {
            hip_fail(hipGetLastError(), "repetition penalty");
            return -1;
        }
        lg = m->plogits;
    }
    if (launch_argmax(lg, m->V, m->tok, s) != TL_HIP_OK) return -1;
    int32_t id = -1;
    hipError_t e = hipMemcpyAsync(&id, m->tok, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        hip_fail(e, "sample readback");
        return -1;
    }
    return id;
}

int32_t tl_hip_llama_sample(tl_hip_llama* h, float temp, float top_p, double repetition_penalty,
                            const int32_t* history, int n_history) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model");
        return -1;
    }
    if (temp <= 0.0f) return tl_hip_llama_sample_greedy(h, repetition_penalty, history, n_history);
    Llama* m = L_(h);
    if (repetition_penalty <= 0.0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: repetition penalty must be positive");
        return -1;
    }
    hipStream_t s = cur_stream();
    const float pen = (float)repetition_penalty;
    const float* lg = m->logits;
    if (pen != 1.0f) {
        std::vector<uint8_t> seen(m->V, 0);
        for (int i = 0; i < n_history; i++)
            if (history && history[i] >= 0 && history[i] < m->V) seen[history[i]] = 1;
        if (hipMemcpyAsync(m->seen, seen.data(), m->V, hipMemcpyHostToDevice, s) != hipSuccess ||
            launch_rep_penalty(m->logits, m->seen, m->plogits, 1, m->V, pen, s) != TL_HIP_OK) {
            hip_fail(hipGetLastError(), "repetition penalty");
            return -1;
        }
        lg = m->plogits;
    }
    // the chosen index as a float in am_v[0] (a free word between decode steps)
    if (launch_sample_top_p(lg, m->V, temp, top_p, (float)sample_draw(), m->smp_key, m->am_v, nullptr, s) != TL_HIP_OK)
        return -1;
    float id = -1.0f;
    hipError_t e = hipMemcpyAsync(&id, m->am_v, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        hip_fail(e, "sample readback");
        return -1;
    }
    return (int32_t)id;
}

int tl_hip_llama_set_sampling(tl_hip_llama* h, float temp, float top_p) {
    if (!h) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model");
        return TL_HIP_ERR_NULL;
    }
    if (temp != temp || top_p != top_p) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: sampling temp and top_p must not be NaN");
        return TL_HIP_ERR_ARG;
    }
    Llama* m = L_(h);
    m->smp_temp = temp > 0.0f ? temp : 0.0f;
    m->smp_top_p = top_p;
    return TL_HIP_OK;
}

int tl_hip_llama_generate(tl_hip_llama* h, int32_t first, int n_steps, int32_t* out_ids,
                          double repetition_penalty, const int32_t* history, int n_history, int use_graph) {
    if (!h || !out_ids) {
        set_error(TL_HIP_ERR_NULL, "NullPointerError: model or output");
        return TL_HIP_ERR_NULL;
    }
    Llama* m = L_(h);
    int rc = check_ready(m);
    if (rc) return rc;
    if (n_steps <= 0) return TL_HIP_OK;
    if (m->host_pos + n_steps > m->max_seq) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: %d steps at position %lld exceed max_seq %d", n_steps,
                  (long long)m->host_pos, m->max_seq);
        return TL_HIP_ERR_ARG;
    }
    if (first < 0 || first >= m->V) {
        set_error(TL_HIP_ERR_INDEX, "IndexOutOfBounds: token %d out of range for vocab size %d", first, m->V);
        return TL_HIP_ERR_INDEX;
    }
    if (repetition_penalty <= 0.0) {
        set_error(TL_HIP_ERR_ARG, "ArgumentError: repetition penalty must be positive");
        return TL_HIP_ERR_ARG;
    }
    hipStream_t s = cur_stream();
    if ((rc = ensure_tokens(m, 1))) return rc;
    const float pen = (float)repetition_penalty;
    if (pen != 1.0f) {
        // the ids the penalty sees: history plus the token being fed (chatbot.tl:188, 221)
        std::vector<uint8_t> seen(m->V, 0);
        for (int i = 0; i < n_history; i++)
            if (history && history[i] >= 0 && history[i] < m->V) seen[history[i]] = 1;
        seen[first] = 1;
        TLH_CHECK_HIP(hipMemcpyAsync(m->seen, seen.data(), m->V, hipMemcpyHostToDevice, s));
        TLH_CHECK_HIP(hipStreamSynchronize(s));
    }
    int32_t zero = 0;
    std::vector<float> draws;
    if (m->smp_temp > 0.0f) {  // one draw per step, in step order (T::from_f64(u): rounded to f32)
        draws.resize(n_steps);
        for (float& d : draws) d = (float)sample_draw();
        TLH_CHECK_HIP(hipMemcpyAsync(m->draws, draws.data(), (size_t)n_steps * 4, hipMemcpyHostToDevice, s));
    }
    TLH_CHECK_HIP(hipMemcpyAsync(m->tok, &first, 4, hipMemcpyHostToDevice, s));
    TLH_CHECK_HIP(hipMemcpyAsync(m->step, &zero, 4, hipMemcpyHostToDevice, s));
    TLH_CHECK_HIP(hipStreamSynchronize(s));
    if (use_graph) {
        uint32_t key[5] = {0, (uint32_t)m->kv_f16, (uint32_t)m->rope_per_token, 0, 0};
        std::memcpy(&key[0], &pen, 4);
        if (m->smp_temp > 0.0f) {
            std::memcpy(&key[3], &m->smp_temp, 4);
            std::memcpy(&key[4], &m->smp_top_p, 4);
        }
        if (std::memcmp(key, m->graph_key, sizeof(key)) != 0) {
            free_graph(m);
            std::memcpy(m->graph_key, key, sizeof(key));
        }
        // both graph shapes are captured on the first graph-mode call for a key, whatever its
        // n_steps: a later call of any length then only replays (a capture is ~10 ms of host
        // work, which must not land inside a caller's timed or latency-bound call)
        const int n_multi = n_steps / GRAPH_STEPS, n_single = n_steps % GRAPH_STEPS;
        for (int gi = 0; gi < 2; gi++) {
            if (m->graph[gi]) continue;
            hipGraph_t g;
            TLH_CHECK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            for (int i = 0; i < (gi == 0 ? 1 : GRAPH_STEPS) && rc == 0; i++) rc = enqueue_step(m, pen, s);
            hipError_t e = hipStreamEndCapture(s, &g);
            if (rc) {
                if (e == hipSuccess) (void)hipGraphDestroy(g);
                return rc;
            }
            if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
            e = hipGraphInstantiate(&m->graph[gi], g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (e != hipSuccess) {
                m->graph[gi] = nullptr;
                return hip_fail(e, "hipGraphInstantiate");
            }
            m->graph_builds++;
        }
        for (int i = 0; i < n_multi; i++) TLH_CHECK_HIP(hipGraphLaunch(m->graph[1], s));
        for (int i = 0; i < n_single; i++) TLH_CHECK_HIP(hipGraphLaunch(m->graph[0], s));
    } else {
        for (int i = 0; i < n_steps; i++)
            if ((rc = enqueue_step(m, pen, s))) return rc;
    }
    TLH_CHECK_HIP(hipMemcpyAsync(out_ids, m->out_ids, (size_t)n_steps * 4, hipMemcpyDeviceToHost, s));
    TLH_CHECK_HIP(hipStreamSynchronize(s));
    m->host_pos += n_steps;
    return TL_HIP_OK;
}

}  // extern "C"
