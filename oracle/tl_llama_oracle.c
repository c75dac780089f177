/*
 * tl_llama_oracle.c -- CPU restatement of the reference's Llama decoder composition
 * (examples/apps/tinyllama/chatbot.tl:1-226) over the tl_cpu ops restated in
 * tl_cpu_oracle.c.  TEST INFRASTRUCTURE ONLY (checker for the parity tests, the smoke
 * check and the benchmark's CPU-baseline leg); the product never links or loads it.
 *
 * Arithmetic per element follows the tl_cpu op sequence the chatbot issues, so the logits
 * are bit-identical to running those ops one after another:
 *   - quantized linear = dequantize -> transpose -> matmul_impl (system.rs:193-222), here
 *     with the cached transposed f32 weight and tlo_matmul_fast (bit-identical to
 *     tlo_matmul, each output a left-to-right sum from 0),
 *   - attention = transpose / cat_4d / repeat_interleave / matmul_4d / scale / +mask /
 *     softmax / matmul_4d (chatbot.tl:50-90) computed directly with the same per-element
 *     operation order (tlo_attention_compose checks this against the literal op chain).
 * Pinned by tests/test_oracle_model.py: logits and greedy ids bit-equal to a literal replay of
 * the chatbot's op chain (one oracle op per program line, each op pinned on its own) over a
 * 6-token prefill at position 0 plus three decode steps, Q4_0 / Q8_0 / Q4_K_M weights, with
 * and without the repetition penalty 1.1 (chatbot.tl:188).
 * Model hyper-parameters are arguments; the chatbot hard-codes TinyLlama's
 * (chatbot.tl:51-54, 73, 83, 151, 168, 181).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int tlo_dequantize_q4_0(const uint8_t* data, int64_t nbytes, int64_t numel, float* out);
int tlo_dequantize_q8_0(const uint8_t* data, int64_t nbytes, int64_t numel, float* out);
int tlo_dequantize_q4_k(const uint8_t* data, int64_t nbytes, int64_t numel, float* out);
int tlo_dequantize_q6_k(const uint8_t* data, int64_t nbytes, int64_t numel, float* out);
void tlo_transpose_2d(const float* a, int64_t rows, int64_t cols, float* out);
void tlo_matmul_fast(const float* A, const float* B, float* C, int64_t m, int64_t k, int64_t n);
void tlo_rms_norm(const float* x, int64_t rows, int64_t n, const float* w, float eps, float* out);
void tlo_rope_new_cos(int64_t seq_len, int64_t dim, float base, float* out);
void tlo_rope_new_sin(int64_t seq_len, int64_t dim, float base, float* out);
void tlo_apply_rope(const float* x, int64_t total, int64_t head_dim, const float* cos_t,
                    int64_t cos_len, const float* sin_t, int64_t sin_len, float* out);
void tlo_silu(const float* x, int64_t n, float* out);
int tlo_embedding(const float* table, int64_t vocab, int64_t dim, const float* ids, int64_t n,
                  float* out);

/* Direct form of the chatbot attention (chatbot.tl:63-87) for one layer.
 *   q     [sl, nh, hd]   (after RoPE, token-major as produced by the q projection)
 *   kc,vc [nkv, L, hd]   (k_tot / v_tot after cat_4d, i.e. the cache incl. the new tokens)
 *   out   [sl, nh*hd]    (ao.transpose(1,2).reshape([sl, nh*hd]))
 * score = sum_d q*k (matmul_4d, sum from 0 left to right), * scale (tensor_scale), + mask
 * (0 or -inf, only when sl > 1; add_4d), softmax over L (tensor.rs:1065-1092), then
 * out = sum_l p*v (matmul_4d).  KV head of query head h is h / (nh/nkv)
 * (repeat_interleave, tensor.rs:1178-1200).  When causal, L must equal sl (the chatbot only
 * masks at start position 0: a [sl,sl] mask broadcast against [.., sl, L]). */
int tlo_attention(const float* q, const float* kc, const float* vc, int64_t sl, int64_t nh,
                  int64_t nkv, int64_t hd, int64_t L, float scale, int causal, float* out) {
    if (causal && L != sl) return -2;
    int64_t rep = nh / nkv;
    float* p = (float*)malloc(sizeof(float) * (size_t)L);
    if (!p) return -1;
    for (int64_t h = 0; h < nh; h++) {
        const float* K = kc + (h / rep) * L * hd;
        const float* V = vc + (h / rep) * L * hd;
        for (int64_t i = 0; i < sl; i++) {
            const float* qi = q + (i * nh + h) * hd;
            for (int64_t l = 0; l < L; l++) {
                float s = 0.0f;
                for (int64_t d = 0; d < hd; d++) s += qi[d] * K[l * hd + d];
                s = s * scale;
                if (causal) s = s + (l > i ? -INFINITY : 0.0f);
                p[l] = s;
            }
            float mx = -INFINITY;
            for (int64_t l = 0; l < L; l++)
                if (p[l] > mx) mx = p[l];
            float sum = 0.0f;
            for (int64_t l = 0; l < L; l++) { p[l] = expf(p[l] - mx); sum += p[l]; }
            for (int64_t l = 0; l < L; l++) p[l] /= sum;
            float* oi = out + i * nh * hd + h * hd;
            for (int64_t d = 0; d < hd; d++) {
                float acc = 0.0f;
                for (int64_t l = 0; l < L; l++) acc += p[l] * V[l * hd + d];
                oi[d] = acc;
            }
        }
    }
    free(p);
    return 0;
}

typedef struct {
    float* wt;      /* transposed dequantized weight [k, n] (QTensor::cache_transposed) */
    int64_t n, k;
} tlo_linear;

typedef struct {
    int n_layers, d_model, n_heads, n_kv, head_dim, ffn, vocab, max_seq;
    float eps, theta;
    float* emb;       /* [vocab, d_model] */
    float* out_norm;  /* [d_model] */
    tlo_linear lm_head;
    float** attn_norm;
    float** ffn_norm;
    tlo_linear* lin;  /* [n_layers * 7]: q k v o gate up down */
    float** kcache;   /* per layer [n_kv, max_seq, head_dim] */
    float** vcache;
    float* cos_t;     /* rope_new_cos(head_dim, max_seq, theta) -> [max_seq, head_dim] */
    float* sin_t;
    int64_t cache_len;
} tlo_llama;

tlo_llama* tlo_llama_new(int n_layers, int d_model, int n_heads, int n_kv, int ffn, int vocab,
                         float eps, float theta, int max_seq) {
    tlo_llama* m = (tlo_llama*)calloc(1, sizeof(tlo_llama));
    if (!m) return NULL;
    m->n_layers = n_layers; m->d_model = d_model; m->n_heads = n_heads; m->n_kv = n_kv;
    m->head_dim = d_model / n_heads; m->ffn = ffn; m->vocab = vocab; m->max_seq = max_seq;
    m->eps = eps; m->theta = theta;
    m->attn_norm = (float**)calloc((size_t)n_layers, sizeof(float*));
    m->ffn_norm = (float**)calloc((size_t)n_layers, sizeof(float*));
    m->lin = (tlo_linear*)calloc((size_t)n_layers * 7, sizeof(tlo_linear));
    m->kcache = (float**)calloc((size_t)n_layers, sizeof(float*));
    m->vcache = (float**)calloc((size_t)n_layers, sizeof(float*));
    int64_t hd = m->head_dim;
    for (int l = 0; l < n_layers; l++) {
        m->kcache[l] = (float*)calloc((size_t)(n_kv * (int64_t)max_seq * hd), sizeof(float));
        m->vcache[l] = (float*)calloc((size_t)(n_kv * (int64_t)max_seq * hd), sizeof(float));
    }
    /* chatbot.tl:151-152: Tensor::rope_new_cos(64, 2048, 10000.0) -> [2048, 64] */
    m->cos_t = (float*)malloc(sizeof(float) * (size_t)(max_seq * hd));
    m->sin_t = (float*)malloc(sizeof(float) * (size_t)(max_seq * hd));
    tlo_rope_new_cos(max_seq, hd, theta, m->cos_t);
    tlo_rope_new_sin(max_seq, hd, theta, m->sin_t);
    return m;
}

static void lin_free(tlo_linear* l) { free(l->wt); l->wt = NULL; }

void tlo_llama_free(tlo_llama* m) {
    if (!m) return;
    for (int l = 0; l < m->n_layers; l++) {
        free(m->attn_norm[l]); free(m->ffn_norm[l]);
        free(m->kcache[l]); free(m->vcache[l]);
        for (int w = 0; w < 7; w++) lin_free(&m->lin[l * 7 + w]);
    }
    free(m->attn_norm); free(m->ffn_norm); free(m->lin); free(m->kcache); free(m->vcache);
    lin_free(&m->lm_head);
    free(m->emb); free(m->out_norm); free(m->cos_t); free(m->sin_t);
    free(m);
}

/* Linear::from_map + the CPU dequant/transposed caches (chatbot.tl:10-14; quantized.rs:
 * 117-141; system.rs:193-222).  layer -1 = the LM head ("output.weight"). */
int tlo_llama_set_linear(tlo_llama* m, int layer, int which, const uint8_t* data, int64_t nbytes,
                         int ggml_type, int64_t n, int64_t k) {
    tlo_linear* L = layer < 0 ? &m->lm_head : &m->lin[layer * 7 + which];
    float* w = (float*)malloc(sizeof(float) * (size_t)(n * k));
    if (!w) return -1;
    int rc = ggml_type == 2    ? tlo_dequantize_q4_0(data, nbytes, n * k, w)
             : ggml_type == 8  ? tlo_dequantize_q8_0(data, nbytes, n * k, w)
             : ggml_type == 12 ? tlo_dequantize_q4_k(data, nbytes, n * k, w)
             : ggml_type == 14 ? tlo_dequantize_q6_k(data, nbytes, n * k, w)
                               : -1;
    if (rc) { free(w); return rc; }
    lin_free(L);
    L->wt = (float*)malloc(sizeof(float) * (size_t)(n * k));
    tlo_transpose_2d(w, n, k, L->wt);
    L->n = n; L->k = k;
    free(w);
    return 0;
}

/* RMSNorm::new (chatbot.tl:17-18); layer -1 = output_norm.  which 0 = attn_norm, 1 = ffn_norm */
int tlo_llama_set_norm(tlo_llama* m, int layer, int which, const float* w) {
    float** slot = layer < 0 ? &m->out_norm : (which == 0 ? &m->attn_norm[layer] : &m->ffn_norm[layer]);
    free(*slot);
    *slot = (float*)malloc(sizeof(float) * (size_t)m->d_model);
    memcpy(*slot, w, sizeof(float) * (size_t)m->d_model);
    return 0;
}

int tlo_llama_set_embedding(tlo_llama* m, const float* emb) {
    free(m->emb);
    m->emb = (float*)malloc(sizeof(float) * (size_t)((int64_t)m->vocab * m->d_model));
    memcpy(m->emb, emb, sizeof(float) * (size_t)((int64_t)m->vocab * m->d_model));
    return 0;
}

void tlo_llama_reset(tlo_llama* m) { m->cache_len = 0; }

static void linear(const tlo_linear* L, const float* x, int64_t m, float* y) {
    tlo_matmul_fast(x, L->wt, y, m, L->k, L->n);
}

/* One pass of the chatbot decode loop body (chatbot.tl:174-187) over `sl` new tokens at
 * start position `sp` (= the KV-cache length): embedding -> n_layers x Block::forward ->
 * output norm -> LM head.  Writes the logits of the last row ([vocab]) to `logits`
 * (lo.narrow(0, sl-1, 1), chatbot.tl:189; the LM head rows are independent so only the
 * last one is computed). */
int tlo_llama_forward(tlo_llama* m, const float* ids, int64_t sl, float* logits) {
    const int64_t D = m->d_model, H = m->n_heads, KV = m->n_kv, hd = m->head_dim, F = m->ffn;
    const int64_t sp = m->cache_len, L = sp + sl;
    if (L > m->max_seq) return -3;
    float* x = (float*)malloc(sizeof(float) * (size_t)(sl * D));
    float* h = (float*)malloc(sizeof(float) * (size_t)(sl * D));
    float* q = (float*)malloc(sizeof(float) * (size_t)(sl * D));
    float* qr = (float*)malloc(sizeof(float) * (size_t)(sl * D));
    float* k = (float*)malloc(sizeof(float) * (size_t)(sl * KV * hd));
    float* kr = (float*)malloc(sizeof(float) * (size_t)(sl * KV * hd));
    float* v = (float*)malloc(sizeof(float) * (size_t)(sl * KV * hd));
    float* ao = (float*)malloc(sizeof(float) * (size_t)(sl * D));
    float* t = (float*)malloc(sizeof(float) * (size_t)(sl * D));
    float* g = (float*)malloc(sizeof(float) * (size_t)(sl * F));
    float* u = (float*)malloc(sizeof(float) * (size_t)(sl * F));
    float* kt = (float*)malloc(sizeof(float) * (size_t)(KV * L * hd));
    float* vt = (float*)malloc(sizeof(float) * (size_t)(KV * L * hd));
    int rc = tlo_embedding(m->emb, m->vocab, D, ids, sl, x);          /* chatbot.tl:178 */
    if (rc) goto done;
    /* cs = cos.narrow(0, sp, sl): apply_rope reads its first hd entries = row sp
     * (chatbot.tl:56-61; ffi.rs:2655-2681). */
    const float* cs = m->cos_t + sp * hd;
    const float* ss = m->sin_t + sp * hd;
    for (int l = 0; l < m->n_layers; l++) {
        tlo_linear* W = &m->lin[l * 7];
        tlo_rms_norm(x, sl, D, m->attn_norm[l], m->eps, h);          /* chatbot.tl:108 */
        linear(&W[0], h, sl, q);                                       /* chatbot.tl:52-54 */
        linear(&W[1], h, sl, k);
        linear(&W[2], h, sl, v);
        tlo_apply_rope(q, sl * D, hd, cs, sl * hd, ss, sl * hd, qr);   /* chatbot.tl:60-61 */
        tlo_apply_rope(k, sl * KV * hd, hd, cs, sl * hd, ss, sl * hd, kr);
        /* kt = kr.transpose(1,2) appended to the cache (chatbot.tl:63-69) */
        float* Kc = m->kcache[l];
        float* Vc = m->vcache[l];
        for (int64_t j = 0; j < KV; j++)
            for (int64_t i = 0; i < sl; i++) {
                memcpy(Kc + (j * m->max_seq + sp + i) * hd, kr + (i * KV + j) * hd, sizeof(float) * (size_t)hd);
                memcpy(Vc + (j * m->max_seq + sp + i) * hd, v + (i * KV + j) * hd, sizeof(float) * (size_t)hd);
            }
        for (int64_t j = 0; j < KV; j++) {
            memcpy(kt + j * L * hd, Kc + j * m->max_seq * hd, sizeof(float) * (size_t)(L * hd));
            memcpy(vt + j * L * hd, Vc + j * m->max_seq * hd, sizeof(float) * (size_t)(L * hd));
        }
        rc = tlo_attention(qr, kt, vt, sl, H, KV, hd, L, 0.125f, sl > 1, ao);  /* 71-87 */
        if (rc) goto done;
        linear(&W[3], ao, sl, t);                                      /* chatbot.tl:89 */
        for (int64_t i = 0; i < sl * D; i++) x[i] = x[i] + t[i];       /* chatbot.tl:109 */
        tlo_rms_norm(x, sl, D, m->ffn_norm[l], m->eps, h);            /* chatbot.tl:110 */
        linear(&W[4], h, sl, g);                                       /* chatbot.tl:33-38 */
        tlo_silu(g, sl * F, g);
        linear(&W[5], h, sl, u);
        for (int64_t i = 0; i < sl * F; i++) g[i] = g[i] * u[i];
        linear(&W[6], g, sl, t);
        for (int64_t i = 0; i < sl * D; i++) x[i] = x[i] + t[i];       /* chatbot.tl:111 */
    }
    m->cache_len = L;
    tlo_rms_norm(x + (sl - 1) * D, 1, D, m->out_norm, m->eps, h);     /* chatbot.tl:186 */
    linear(&m->lm_head, h, 1, logits);
done:
    free(x); free(h); free(q); free(qr); free(k); free(kr); free(v); free(ao); free(t);
    free(g); free(u); free(kt); free(vt);
    return rc;
}
