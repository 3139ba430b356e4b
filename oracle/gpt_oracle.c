/*
 * gpt_oracle.c -- CPU restatement of IndexTTS2's GPT mel-code decoder (the
 * GPT-2 stack of UnifiedVoice: 1280 wide, 20 heads of 64, MLP 5120 with
 * gelu_new, learned mel position embeddings, ln_f + final_norm + mel_head)
 * as the reference's fp32 CPU path computes it (runtime/impl/gpt.cpp).
 *
 * TEST INFRASTRUCTURE ONLY (see cfm_oracle.h): the reference the GPU decode
 * is compared with, and the timed CPU baseline; the product never links it.
 *
 * Weights are set by their checkpoint names in the checkpoint's layouts:
 * the GPT-2 Conv1D matrices are [in][out] and are transposed to [out][in]
 * when set, as load_gpt_transformer_layer_weights does
 * (transpose_gpt_conv1d_weight, gpt.cpp:208-216).  The layer count is a
 * parameter (the checkpoint has 24; gpt.cpp:1800 loops over 24).
 *
 * Threads split output rows of a linear and heads of an attention; every
 * output element is still accumulated by one thread in the reference's
 * order, so results do not depend on the thread count.
 */
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cfm_oracle.h"

enum { W = 1280, QKV = 3840, MLP = 5120, HEADS = 20, HD = 64, VOCAB = 8194, POS = 1818 };
enum { START_TOKEN = 8192, STOP_TOKEN = 8193 };

typedef struct {
    float *ln1_w, *ln1_b, *c_attn_w, *c_attn_b, *proj_w, *proj_b;
    float *ln2_w, *ln2_b, *fc_w, *fc_b, *mp_w, *mp_b;
} gpt_layer;

struct orc_gpt {
    int layers;
    gpt_layer* L;
    float *lnf_w, *lnf_b, *fn_w, *fn_b, *head_w, *head_b, *mel_emb, *pos_emb;
};

static char g_err[256];
const char* orc_gpt_last_error(void) { return g_err; }

orc_gpt* orc_gpt_new(int layers) {
    if (layers < 1 || layers > 64) return NULL;
    orc_gpt* m = (orc_gpt*)calloc(1, sizeof(orc_gpt));
    m->layers = layers;
    m->L = (gpt_layer*)calloc((size_t)layers, sizeof(gpt_layer));
    return m;
}

void orc_gpt_free(orc_gpt* m) {
    if (!m) return;
    for (int l = 0; l < m->layers; ++l) {
        float** p = (float**)&m->L[l];
        for (size_t i = 0; i < sizeof(gpt_layer) / sizeof(float*); ++i) free(p[i]);
    }
    free(m->L);
    float* f[] = {m->lnf_w, m->lnf_b, m->fn_w, m->fn_b, m->head_w, m->head_b, m->mel_emb, m->pos_emb};
    for (size_t i = 0; i < sizeof(f) / sizeof(f[0]); ++i) free(f[i]);
    free(m);
}

/* transpose_gpt_conv1d_weight (gpt.cpp:208-216): [in][out] -> [out][in]. */
static float* transpose_conv1d(const float* w_in_out, uint32_t in, uint32_t out) {
    float* t = (float*)malloc((size_t)in * out * sizeof(float));
    for (uint32_t i = 0; i < in; ++i)
        for (uint32_t o = 0; o < out; ++o) t[(size_t)o * in + i] = w_in_out[(size_t)i * out + o];
    return t;
}

static float* copy_of(const float* d, uint64_t n) {
    float* p = (float*)malloc(n * sizeof(float));
    memcpy(p, d, n * sizeof(float));
    return p;
}

/* Sets one tensor; returns 0, or -1 (unknown name or wrong element count). */
int orc_gpt_set(orc_gpt* m, const char* name, const float* data, uint64_t count) {
    struct { const char* n; float** slot; uint64_t elems; } fin[] = {
        {"gpt.gpt.ln_f.weight", &m->lnf_w, W},          {"gpt.gpt.ln_f.bias", &m->lnf_b, W},
        {"gpt.final_norm.weight", &m->fn_w, W},         {"gpt.final_norm.bias", &m->fn_b, W},
        {"gpt.mel_head.weight", &m->head_w, (uint64_t)VOCAB * W},
        {"gpt.mel_head.bias", &m->head_b, VOCAB},
        {"gpt.mel_embedding.weight", &m->mel_emb, (uint64_t)VOCAB * W},
        {"gpt.mel_pos_embedding.emb.weight", &m->pos_emb, (uint64_t)POS * W},
    };
    for (size_t i = 0; i < sizeof(fin) / sizeof(fin[0]); ++i) {
        if (strcmp(name, fin[i].n) == 0) {
            if (count != fin[i].elems) goto bad_count;
            free(*fin[i].slot);
            *fin[i].slot = copy_of(data, count);
            return 0;
        }
    }
    int layer = -1, used = 0;
    if (sscanf(name, "gpt.gpt.h.%d.%n", &layer, &used) == 1 && used > 0 && layer >= 0 && layer < m->layers) {
        const char* s = name + used;
        gpt_layer* L = &m->L[layer];
        struct { const char* n; float** slot; uint64_t elems; uint32_t in, out; } t[] = {
            {"ln_1.weight", &L->ln1_w, W, 0, 0},          {"ln_1.bias", &L->ln1_b, W, 0, 0},
            {"attn.c_attn.weight", &L->c_attn_w, (uint64_t)W * QKV, W, QKV},
            {"attn.c_attn.bias", &L->c_attn_b, QKV, 0, 0},
            {"attn.c_proj.weight", &L->proj_w, (uint64_t)W * W, W, W},
            {"attn.c_proj.bias", &L->proj_b, W, 0, 0},
            {"ln_2.weight", &L->ln2_w, W, 0, 0},          {"ln_2.bias", &L->ln2_b, W, 0, 0},
            {"mlp.c_fc.weight", &L->fc_w, (uint64_t)W * MLP, W, MLP},
            {"mlp.c_fc.bias", &L->fc_b, MLP, 0, 0},
            {"mlp.c_proj.weight", &L->mp_w, (uint64_t)MLP * W, MLP, W},
            {"mlp.c_proj.bias", &L->mp_b, W, 0, 0},
        };
        for (size_t i = 0; i < sizeof(t) / sizeof(t[0]); ++i) {
            if (strcmp(s, t[i].n) == 0) {
                if (count != t[i].elems) goto bad_count;
                free(*t[i].slot);
                *t[i].slot = t[i].in ? transpose_conv1d(data, t[i].in, t[i].out) : copy_of(data, count);
                return 0;
            }
        }
    }
    snprintf(g_err, sizeof(g_err), "unknown GPT tensor %s", name);
    return -1;
bad_count:
    snprintf(g_err, sizeof(g_err), "GPT tensor %s: wrong element count %llu", name,
             (unsigned long long)count);
    return -1;
}

/* Number of tensors not yet set (0 = complete). */
int orc_gpt_missing(const orc_gpt* m) {
    int n = 0;
    for (int l = 0; l < m->layers; ++l) {
        float* const* p = (float* const*)&m->L[l];
        for (size_t i = 0; i < sizeof(gpt_layer) / sizeof(float*); ++i) n += p[i] == NULL;
    }
    const float* f[] = {m->lnf_w, m->lnf_b, m->fn_w, m->fn_b, m->head_w, m->head_b, m->mel_emb, m->pos_emb};
    for (size_t i = 0; i < sizeof(f) / sizeof(f[0]); ++i) n += f[i] == NULL;
    return n;
}

/* ---- primitives ----------------------------------------------------------- */

/* cpu_gelu_new (tokenizer_tests.cpp:3931-3945). */
void orc_gelu_new(const float* x, size_t n, float* out) {
    const float c = 0.7978845608028654f;
    for (size_t i = 0; i < n; ++i) {
        const float v = x[i];
        if (v > 10.0f) out[i] = v;
        else if (v < -10.0f) out[i] = 0.0f;
        else out[i] = 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
    }
}

/* cpu_attention_single_query (tokenizer_tests.cpp:4034-4060); scores is scratch. */
static void attention_one(const float* q, const float* k, const float* v, uint32_t key_tokens,
                          uint32_t head_dim, size_t stride, float* scores, float* out) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    float max_score = -INFINITY;
    for (uint32_t tk = 0; tk < key_tokens; ++tk) {
        float score = 0.0f;
        for (uint32_t d = 0; d < head_dim; ++d) score += q[d] * k[(size_t)tk * stride + d];
        score *= scale;
        scores[tk] = score;
        if (score > max_score) max_score = score;
    }
    float denom = 0.0f;
    for (uint32_t tk = 0; tk < key_tokens; ++tk) {
        scores[tk] = expf(scores[tk] - max_score);
        denom += scores[tk];
    }
    for (uint32_t d = 0; d < head_dim; ++d) {
        float acc = 0.0f;
        for (uint32_t tk = 0; tk < key_tokens; ++tk) acc += (scores[tk] / denom) * v[(size_t)tk * stride + d];
        out[d] = acc;
    }
}

void orc_attention_single_query(const float* q, const float* k, const float* v, uint32_t key_tokens,
                                uint32_t head_dim, float* out) {
    float* scores = (float*)malloc((size_t)(key_tokens ? key_tokens : 1) * sizeof(float));
    attention_one(q, k, v, key_tokens, head_dim, head_dim, scores, out);
    free(scores);
}

/* cpu_attention_single_head_causal (tokenizer_tests.cpp:4003-4032): query tq
 * attends to keys 0..tq, which is the single-query form over tq + 1 keys. */
void orc_attention_causal(const float* q, const float* k, const float* v, uint32_t tokens,
                          uint32_t head_dim, float* out) {
    float* scores = (float*)malloc((size_t)(tokens ? tokens : 1) * sizeof(float));
    for (uint32_t tq = 0; tq < tokens; ++tq)
        attention_one(q + (size_t)tq * head_dim, k, v, tq + 1, head_dim, head_dim, scores,
                      out + (size_t)tq * head_dim);
    free(scores);
}

/* cpu_linear (tokenizer_tests.cpp:3026-3036) with output rows split over threads. */
static void linear_par(const float* w, const float* b, const float* x, uint32_t rows, uint32_t cols,
                       float* out) {
    long r;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (r = 0; r < (long)rows; ++r) {
        float acc = b[r];
        const float* wr = w + (size_t)r * cols;
        for (uint32_t c = 0; c < cols; ++c) acc += wr[c] * x[c];
        out[r] = acc;
    }
}

/* ---- GPT stages ----------------------------------------------------------- */

/* run_gpt_layer_qkv_cpu (gpt.cpp:1060-1077): per row LN(ln_1) then c_attn. */
void orc_gpt_layer_qkv(const orc_gpt* m, const float* in, uint32_t tokens, uint32_t layer, float* qkv) {
    const gpt_layer* L = &m->L[layer];
    float normed[W];
    for (uint32_t t = 0; t < tokens; ++t) {
        orc_layernorm(in + (size_t)t * W, L->ln1_w, L->ln1_b, W, 1e-5f, normed);
        linear_par(L->c_attn_w, L->c_attn_b, normed, QKV, W, qkv + (size_t)t * QKV);
    }
}

/* run_gpt_layer0_attention_core_cpu (gpt.cpp:371-395): per head causal
 * attention over the [q | k | v] rows, heads concatenated. */
static void attention_core(const float* qkv, uint32_t tokens, float* concat) {
    long h;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (h = 0; h < HEADS; ++h) {
        float* qh = (float*)malloc((size_t)tokens * HD * 3 * sizeof(float));
        float* kh = qh + (size_t)tokens * HD;
        float* vh = kh + (size_t)tokens * HD;
        float* yh = (float*)malloc((size_t)tokens * HD * sizeof(float));
        for (uint32_t t = 0; t < tokens; ++t) {
            const size_t base = (size_t)t * QKV + (size_t)h * HD;
            memcpy(qh + (size_t)t * HD, qkv + base, HD * sizeof(float));
            memcpy(kh + (size_t)t * HD, qkv + base + W, HD * sizeof(float));
            memcpy(vh + (size_t)t * HD, qkv + base + 2 * W, HD * sizeof(float));
        }
        orc_attention_causal(qh, kh, vh, tokens, HD, yh);
        for (uint32_t t = 0; t < tokens; ++t)
            memcpy(concat + (size_t)t * W + (size_t)h * HD, yh + (size_t)t * HD, HD * sizeof(float));
        free(yh);
        free(qh);
    }
}

/* The MLP half shared by the full and the cached block: out = res +
 * c_proj(gelu_new(c_fc(LN(res; ln_2)))) (gpt.cpp:1201-1214). */
static void mlp_residual(const gpt_layer* L, const float* res, float* out) {
    float normed[W], projected[W];
    float* hidden = (float*)malloc((size_t)MLP * sizeof(float));
    orc_layernorm(res, L->ln2_w, L->ln2_b, W, 1e-5f, normed);
    linear_par(L->fc_w, L->fc_b, normed, MLP, W, hidden);
    orc_gelu_new(hidden, MLP, hidden);
    linear_par(L->mp_w, L->mp_b, hidden, W, MLP, projected);
    for (uint32_t i = 0; i < W; ++i) out[i] = res[i] + projected[i];
    free(hidden);
}

/* run_gpt_transformer_block_cpu_layer (gpt.cpp:658-712): the full causal block. */
void orc_gpt_block(const orc_gpt* m, const float* in, uint32_t tokens, uint32_t layer, float* out) {
    const gpt_layer* L = &m->L[layer];
    float* qkv = (float*)malloc((size_t)tokens * QKV * sizeof(float));
    float* att = (float*)malloc((size_t)tokens * W * sizeof(float));
    float projected[W], res[W];
    orc_gpt_layer_qkv(m, in, tokens, layer, qkv);
    attention_core(qkv, tokens, att);
    for (uint32_t t = 0; t < tokens; ++t) {
        linear_par(L->proj_w, L->proj_b, att + (size_t)t * W, W, W, projected);
        for (uint32_t c = 0; c < W; ++c) res[c] = in[(size_t)t * W + c] + projected[c];
        mlp_residual(L, res, out + (size_t)t * W);
    }
    free(att);
    free(qkv);
}

/* run_gpt_cached_attention_current_cpu (gpt.cpp:1147-1170): the current
 * query attends to the cache's keys followed by its own key. */
static void cached_attention_current(const float* cache_k, const float* cache_v, uint32_t cache_tokens,
                                     const float* cur_qkv, float* concat) {
    long h;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (h = 0; h < HEADS; ++h) {
        const uint32_t n = cache_tokens + 1;
        float* kh = (float*)malloc((size_t)n * HD * 2 * sizeof(float) + (size_t)n * sizeof(float));
        float* vh = kh + (size_t)n * HD;
        float* scores = vh + (size_t)n * HD;
        for (uint32_t t = 0; t < cache_tokens; ++t) {
            memcpy(kh + (size_t)t * HD, cache_k + (size_t)t * W + (size_t)h * HD, HD * sizeof(float));
            memcpy(vh + (size_t)t * HD, cache_v + (size_t)t * W + (size_t)h * HD, HD * sizeof(float));
        }
        memcpy(kh + (size_t)cache_tokens * HD, cur_qkv + W + (size_t)h * HD, HD * sizeof(float));
        memcpy(vh + (size_t)cache_tokens * HD, cur_qkv + 2 * W + (size_t)h * HD, HD * sizeof(float));
        attention_one(cur_qkv + (size_t)h * HD, kh, vh, n, HD, HD, scores, concat + (size_t)h * HD);
        free(kh);
    }
}

/* run_gpt_cached_block_current_cpu (gpt.cpp:1180-1214). */
void orc_gpt_cached_block_current(const orc_gpt* m, const float* cache_k, const float* cache_v,
                                  uint32_t cache_tokens, const float* current, const float* current_qkv,
                                  uint32_t layer, float* out) {
    const gpt_layer* L = &m->L[layer];
    float att[W], projected[W], res[W];
    cached_attention_current(cache_k, cache_v, cache_tokens, current_qkv, att);
    linear_par(L->proj_w, L->proj_b, att, W, W, projected);
    for (uint32_t i = 0; i < W; ++i) res[i] = current[i] + projected[i];
    mlp_residual(L, res, out);
}

/* argmax_row (gpt.cpp:1297-1308): the first index of the maximum. */
static uint32_t argmax_first(const float* v, uint32_t n) {
    uint32_t best = 0;
    float bv = v[0];
    for (uint32_t i = 1; i < n; ++i)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

/* ln_f, final_norm and mel_head of one row (gpt.cpp:1420-1423). */
static uint32_t head_row(const orc_gpt* m, const float* x, float* ln_f, float* final_norm, float* logits) {
    orc_layernorm(x, m->lnf_w, m->lnf_b, W, 1e-5f, ln_f);
    orc_layernorm(ln_f, m->fn_w, m->fn_b, W, 1e-5f, final_norm);
    linear_par(m->head_w, m->head_b, final_norm, VOCAB, W, logits);
    return argmax_first(logits, VOCAB);
}

/* run_gpt_logits_cpu (gpt.cpp:1310-1331) over run_gpt_transformer_stack_cpu
 * (gpt.cpp:833-849): every layer on all rows, then per row ln_f,
 * final_norm, mel_head.  final_norm [tokens][1280], logits [tokens][8194];
 * returns the argmax of the last row. */
uint32_t orc_gpt_logits(const orc_gpt* m, const float* in, uint32_t tokens, float* final_norm, float* logits) {
    float* a = (float*)malloc((size_t)tokens * W * sizeof(float));
    float* b = (float*)malloc((size_t)tokens * W * sizeof(float));
    float ln_f[W];
    memcpy(a, in, (size_t)tokens * W * sizeof(float));
    for (int l = 0; l < m->layers; ++l) {
        orc_gpt_block(m, a, tokens, (uint32_t)l, b);
        float* t = a; a = b; b = t;
    }
    uint32_t am = 0;
    for (uint32_t t = 0; t < tokens; ++t)
        am = head_row(m, a + (size_t)t * W, ln_f, final_norm + (size_t)t * W, logits + (size_t)t * VOCAB);
    free(a);
    free(b);
    return am;
}

/* run_gpt_cached_decode_cpu (gpt.cpp:1400-1425): rows 0..P-1 of `input` are
 * the prefix (full blocks, each layer's K/V taken from its QKV), row P the
 * current row (cached blocks).  Returns the argmax. */
uint32_t orc_gpt_cached_decode(const orc_gpt* m, const float* input, uint32_t prefix_tokens, float* ln_f,
                               float* final_norm, float* logits) {
    const uint32_t P = prefix_tokens;
    float* prefix = (float*)malloc(((size_t)P + 1) * W * sizeof(float));
    float* next = (float*)malloc(((size_t)P + 1) * W * sizeof(float));
    float* qkv = (float*)malloc(((size_t)P + 1) * QKV * sizeof(float));
    float* ck = (float*)malloc(((size_t)P + 1) * W * sizeof(float));
    float* cv = (float*)malloc(((size_t)P + 1) * W * sizeof(float));
    float cur[W], cur_qkv[QKV], nxt[W];
    memcpy(prefix, input, (size_t)P * W * sizeof(float));
    memcpy(cur, input + (size_t)P * W, W * sizeof(float));
    for (int l = 0; l < m->layers; ++l) {
        orc_gpt_layer_qkv(m, prefix, P, (uint32_t)l, qkv);
        for (uint32_t t = 0; t < P; ++t) {  /* extract_gpt_kv_cache (gpt.cpp:1121-1135) */
            memcpy(ck + (size_t)t * W, qkv + (size_t)t * QKV + W, W * sizeof(float));
            memcpy(cv + (size_t)t * W, qkv + (size_t)t * QKV + 2 * W, W * sizeof(float));
        }
        if (P) orc_gpt_block(m, prefix, P, (uint32_t)l, next);
        float* t = prefix; prefix = next; next = t;
        orc_gpt_layer_qkv(m, cur, 1, (uint32_t)l, cur_qkv);
        orc_gpt_cached_block_current(m, ck, cv, P, cur, cur_qkv, (uint32_t)l, nxt);
        memcpy(cur, nxt, sizeof(cur));
    }
    const uint32_t am = head_row(m, cur, ln_f, final_norm, logits);
    free(prefix); free(next); free(qkv); free(ck); free(cv);
    return am;
}

/* gpt_cached_generate_position (gpt.cpp:1873-1875). */
static uint32_t generate_position(uint32_t step, int hf) { return hf && step > 0 ? step + 1 : step; }

/* Greedy loops fill predicted [steps], input_tokens [steps + 1] and
 * last_logits [8194]; the counts and the first stop step go to *res. */
/* run_gpt_kv_greedy_cpu (gpt.cpp:1877-1911): prefill the K/V caches from the
 * prefix rows (run_gpt_kv_prefill_cpu, gpt.cpp:1796-1806), then per step
 * embed the last input token at its position, run the cached blocks
 * (appending each layer's K/V), take ln_f, final_norm, mel_head and the
 * argmax; stop at the first stop token.  Returns -1 for a position beyond
 * the position table (the reference throws there), else 0. */
int orc_gpt_kv_greedy(const orc_gpt* m, const float* prefix, uint32_t prefix_tokens, uint32_t steps, int hf,
                      uint32_t* predicted, uint32_t* input_tokens, float* last_logits,
                      orc_gpt_greedy_result* res) {
    const uint32_t P = prefix_tokens, cap = P + steps + 1;
    const int NL = m->layers;
    float* ck = (float*)malloc((size_t)NL * cap * W * sizeof(float));
    float* cv = (float*)malloc((size_t)NL * cap * W * sizeof(float));
    float* hid = (float*)malloc(((size_t)P + 1) * W * sizeof(float));
    float* nxt = (float*)malloc(((size_t)P + 1) * W * sizeof(float));
    float* qkv = (float*)malloc(((size_t)P + 1) * QKV * sizeof(float));
    float cur[W], cur_qkv[QKV], out[W], ln_f[W], fnorm[W];
    int rc = 0;
    res->n_predicted = 0;
    res->n_input = 1;
    res->first_stop_step = -1;
    input_tokens[0] = START_TOKEN;
    memcpy(hid, prefix, (size_t)P * W * sizeof(float));
    for (int l = 0; l < NL; ++l) {
        float* K = ck + (size_t)l * cap * W;
        float* V = cv + (size_t)l * cap * W;
        orc_gpt_layer_qkv(m, hid, P, (uint32_t)l, qkv);
        for (uint32_t t = 0; t < P; ++t) {
            memcpy(K + (size_t)t * W, qkv + (size_t)t * QKV + W, W * sizeof(float));
            memcpy(V + (size_t)t * W, qkv + (size_t)t * QKV + 2 * W, W * sizeof(float));
        }
        if (P) orc_gpt_block(m, hid, P, (uint32_t)l, nxt);
        float* t = hid; hid = nxt; nxt = t;
    }
    uint32_t kv = P;
    for (uint32_t step = 0; step < steps; ++step) {
        /* build_gpt_greedy_current_cpu (gpt.cpp:1545-1554) */
        const uint32_t tok = input_tokens[res->n_input - 1];
        const uint32_t pos = generate_position(step, hf);
        if (pos >= POS || tok >= VOCAB) { rc = -1; break; }
        for (uint32_t c = 0; c < W; ++c)
            cur[c] = m->mel_emb[(size_t)tok * W + c] + m->pos_emb[(size_t)pos * W + c];
        for (int l = 0; l < NL; ++l) {
            float* K = ck + (size_t)l * cap * W;
            float* V = cv + (size_t)l * cap * W;
            orc_gpt_layer_qkv(m, cur, 1, (uint32_t)l, cur_qkv);
            orc_gpt_cached_block_current(m, K, V, kv, cur, cur_qkv, (uint32_t)l, out);
            /* append_gpt_current_kv (gpt.cpp:1137-1144) */
            memcpy(K + (size_t)kv * W, cur_qkv + W, W * sizeof(float));
            memcpy(V + (size_t)kv * W, cur_qkv + 2 * W, W * sizeof(float));
            memcpy(cur, out, sizeof(cur));
        }
        ++kv;
        const uint32_t next = head_row(m, cur, ln_f, fnorm, last_logits);
        predicted[res->n_predicted++] = next;
        if (next == STOP_TOKEN) {
            res->first_stop_step = (int32_t)step;
            break;
        }
        input_tokens[res->n_input++] = next;
    }
    free(ck); free(cv); free(hid); free(nxt); free(qkv);
    return rc;
}

/* run_gpt_greedy_cpu (gpt.cpp:1833-1851): the uncached loop that reruns the
 * whole sequence (prefix, then the input tokens at positions 0..n-1) every
 * step and does not stop at the stop token. */
int orc_gpt_greedy_full(const orc_gpt* m, const float* prefix, uint32_t prefix_tokens, uint32_t steps,
                        uint32_t* predicted, uint32_t* input_tokens, float* last_logits,
                        orc_gpt_greedy_result* res) {
    const uint32_t P = prefix_tokens;
    float* seq = (float*)malloc(((size_t)P + steps + 1) * W * sizeof(float));
    float* fnorm = (float*)malloc(((size_t)P + steps + 1) * W * sizeof(float));
    float* logits = (float*)malloc(((size_t)P + steps + 1) * VOCAB * sizeof(float));
    int rc = 0;
    res->n_predicted = 0;
    res->n_input = 1;
    res->first_stop_step = -1;
    input_tokens[0] = START_TOKEN;
    memcpy(seq, prefix, (size_t)P * W * sizeof(float));
    for (uint32_t step = 0; step < steps; ++step) {
        const uint32_t n = res->n_input;
        if (n > POS) { rc = -1; break; }
        for (uint32_t t = 0; t < n; ++t)  /* build_gpt_greedy_sequence_cpu (gpt.cpp:1511-1525) */
            for (uint32_t c = 0; c < W; ++c)
                seq[((size_t)P + t) * W + c] =
                    m->mel_emb[(size_t)input_tokens[t] * W + c] + m->pos_emb[(size_t)t * W + c];
        const uint32_t next = orc_gpt_logits(m, seq, P + n, fnorm, logits);
        memcpy(last_logits, logits + ((size_t)P + n - 1) * VOCAB, VOCAB * sizeof(float));
        predicted[res->n_predicted++] = next;
        if (next == STOP_TOKEN && res->first_stop_step < 0) res->first_stop_step = (int32_t)step;
        input_tokens[res->n_input++] = next;
    }
    free(seq); free(fnorm); free(logits);
    return rc;
}

/* ---- sampling (the do_sample path) ---------------------------------------- */

/* SplitMix64 of the GPT sampler (gpt.cpp:1601-1616). */
static uint64_t sm64_next(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
static double sm64_unit(uint64_t* s) { return (double)(sm64_next(s) >> 11) * (1.0 / 9007199254740992.0); }

typedef struct { float v; uint32_t i; } score_idx;
static int cmp_desc(const void* a, const void* b) {
    const float x = ((const score_idx*)a)->v, y = ((const score_idx*)b)->v;
    return x > y ? -1 : (x < y ? 1 : 0);
}
static int cmp_asc_idx(const void* a, const void* b) {  /* the top-p order (gpt.cpp:1667-1672) */
    const score_idx* p = (const score_idx*)a;
    const score_idx* q = (const score_idx*)b;
    if (p->v == q->v) return p->i < q->i ? -1 : (p->i > q->i ? 1 : 0);
    return p->v < q->v ? -1 : 1;
}

/* apply_gpt_sampling_processors (gpt.cpp:1618-1718): repetition penalty over
 * the distinct history tokens, temperature, top-k (keep scores >= the k-th
 * largest), top-p (drop the low tail whose cumulative probability, in
 * ascending score order, stays <= 1 - top_p; the largest always stays).
 * Returns 0, or -1 for an invalid setting (the reference throws). */
int orc_gpt_sampling_processors(const float* logits, uint32_t n, const uint32_t* history, uint32_t n_history,
                                float temperature, uint32_t top_k, float top_p, float repetition_penalty,
                                float* scores) {
    memcpy(scores, logits, n * sizeof(float));
    if (repetition_penalty != 1.0f) {
        if (repetition_penalty <= 0.0f) return -1;
        uint8_t* seen = (uint8_t*)calloc(n, 1);
        for (uint32_t h = 0; h < n_history; ++h) {
            const uint32_t t = history[h];
            if (t >= n || seen[t]) continue;
            seen[t] = 1;
            if (scores[t] < 0.0f) scores[t] *= repetition_penalty;
            else scores[t] /= repetition_penalty;
        }
        free(seen);
    }
    if (temperature <= 0.0f) return -1;
    if (temperature != 1.0f)
        for (uint32_t i = 0; i < n; ++i) scores[i] /= temperature;
    score_idx* s = (score_idx*)malloc(n * sizeof(score_idx));
    if (top_k > 0 && top_k < n) {
        for (uint32_t i = 0; i < n; ++i) { s[i].v = scores[i]; s[i].i = i; }
        qsort(s, n, sizeof(score_idx), cmp_desc);  /* the k-th largest value, as nth_element */
        const float pivot = s[top_k - 1].v;
        for (uint32_t i = 0; i < n; ++i)
            if (scores[i] < pivot) scores[i] = -INFINITY;
    }
    if (top_p < 1.0f) {
        if (top_p <= 0.0f) { free(s); return -1; }
        for (uint32_t i = 0; i < n; ++i) { s[i].v = scores[i]; s[i].i = i; }
        qsort(s, n, sizeof(score_idx), cmp_asc_idx);
        float max_score = -INFINITY;
        for (uint32_t i = 0; i < n; ++i)
            if (isfinite(scores[i]) && scores[i] > max_score) max_score = scores[i];
        if (!isfinite(max_score)) { free(s); return -1; }
        double* probs = (double*)calloc(n, sizeof(double));
        uint8_t* rem = (uint8_t*)calloc(n, 1);
        double total = 0.0;
        for (uint32_t i = 0; i < n; ++i)
            if (isfinite(scores[i])) { probs[i] = exp((double)(scores[i] - max_score)); total += probs[i]; }
        if (total <= 0.0) { free(s); free(probs); free(rem); return -1; }
        double cumulative = 0.0;
        const double low_tail = 1.0 - (double)top_p;
        uint32_t finite_seen = 0;
        for (uint32_t o = 0; o < n; ++o) {
            const uint32_t idx = s[o].i;
            if (!isfinite(scores[idx])) { rem[idx] = 1; continue; }
            ++finite_seen;
            cumulative += probs[idx] / total;
            if (cumulative <= low_tail) rem[idx] = 1;
        }
        if (finite_seen > 0) rem[s[n - 1].i] = 0;
        for (uint32_t i = 0; i < n; ++i)
            if (rem[i]) scores[i] = -INFINITY;
        free(probs);
        free(rem);
    }
    free(s);
    return 0;
}

/* sample_gpt_token_from_logits (gpt.cpp:1720-1750): one draw of the
 * splitmix64 stream, scaled by the total exp mass, walked in index order. */
uint32_t orc_gpt_sample_token(const float* processed, uint32_t n, uint64_t* rng_state) {
    float max_score = -INFINITY;
    for (uint32_t i = 0; i < n; ++i)
        if (isfinite(processed[i]) && processed[i] > max_score) max_score = processed[i];
    double* probs = (double*)calloc(n, sizeof(double));
    double total = 0.0;
    for (uint32_t i = 0; i < n; ++i)
        if (isfinite(processed[i])) { probs[i] = exp((double)(processed[i] - max_score)); total += probs[i]; }
    const double target = sm64_unit(rng_state) * total;
    double cumulative = 0.0;
    uint32_t last_finite = 0, pick = UINT32_MAX;
    for (uint32_t i = 0; i < n && pick == UINT32_MAX; ++i) {
        if (probs[i] <= 0.0) continue;
        last_finite = i;
        cumulative += probs[i];
        if (target < cumulative) pick = i;
    }
    free(probs);
    return pick == UINT32_MAX ? last_finite : pick;
}

/* The sampled form of the cached loop (run_gpt_kv_greedy_metal with
 * do_sample, gpt.cpp:2221-2240): after each step's logits, the processors over
 * the history and one draw; the rng is seeded once per call.  The history is
 * repetition_history_prefix followed by the predictions so far whenever a
 * prefix is given (history_prefix non-NULL, even with n_history_prefix 0: the
 * reference inserts the vector it points to, however short), or with no
 * prefix (NULL) the start token followed by them (gpt.cpp:2224-2229).  last_processed receives the last step's processed
 * logits.  Returns 0, or -1 (a position past the table or an invalid
 * setting). */
int orc_gpt_kv_sample(const orc_gpt* m, const float* prefix, uint32_t prefix_tokens, uint32_t steps, int hf,
                      uint64_t seed, float temperature, uint32_t top_k, float top_p, float repetition_penalty,
                      const uint32_t* history_prefix, uint32_t n_history_prefix,
                      uint32_t* predicted, uint32_t* input_tokens, float* last_logits, float* last_processed,
                      orc_gpt_greedy_result* res) {
    const uint32_t P = prefix_tokens, cap = P + steps + 1;
    uint32_t* history = (uint32_t*)malloc(((size_t)n_history_prefix + steps + 1) * sizeof(uint32_t));
    if (n_history_prefix) memcpy(history, history_prefix, (size_t)n_history_prefix * sizeof(uint32_t));
    const int NL = m->layers;
    float* ck = (float*)malloc((size_t)NL * cap * W * sizeof(float));
    float* cv = (float*)malloc((size_t)NL * cap * W * sizeof(float));
    float* hid = (float*)malloc(((size_t)P + 1) * W * sizeof(float));
    float* nxt = (float*)malloc(((size_t)P + 1) * W * sizeof(float));
    float* qkv = (float*)malloc(((size_t)P + 1) * QKV * sizeof(float));
    float cur[W], cur_qkv[QKV], out[W], ln_f[W], fnorm[W];
    uint64_t rng = seed;
    int rc = 0;
    res->n_predicted = 0;
    res->n_input = 1;
    res->first_stop_step = -1;
    input_tokens[0] = START_TOKEN;
    memcpy(hid, prefix, (size_t)P * W * sizeof(float));
    for (int l = 0; l < NL; ++l) {
        float* K = ck + (size_t)l * cap * W;
        float* V = cv + (size_t)l * cap * W;
        orc_gpt_layer_qkv(m, hid, P, (uint32_t)l, qkv);
        for (uint32_t t = 0; t < P; ++t) {
            memcpy(K + (size_t)t * W, qkv + (size_t)t * QKV + W, W * sizeof(float));
            memcpy(V + (size_t)t * W, qkv + (size_t)t * QKV + 2 * W, W * sizeof(float));
        }
        if (P) orc_gpt_block(m, hid, P, (uint32_t)l, nxt);
        float* t = hid; hid = nxt; nxt = t;
    }
    uint32_t kv = P;
    for (uint32_t step = 0; step < steps; ++step) {
        const uint32_t tok = input_tokens[res->n_input - 1];
        const uint32_t pos = generate_position(step, hf);
        if (pos >= POS || tok >= VOCAB) { rc = -1; break; }
        for (uint32_t c = 0; c < W; ++c)
            cur[c] = m->mel_emb[(size_t)tok * W + c] + m->pos_emb[(size_t)pos * W + c];
        for (int l = 0; l < NL; ++l) {
            float* K = ck + (size_t)l * cap * W;
            float* V = cv + (size_t)l * cap * W;
            orc_gpt_layer_qkv(m, cur, 1, (uint32_t)l, cur_qkv);
            orc_gpt_cached_block_current(m, K, V, kv, cur, cur_qkv, (uint32_t)l, out);
            memcpy(K + (size_t)kv * W, cur_qkv + W, W * sizeof(float));
            memcpy(V + (size_t)kv * W, cur_qkv + 2 * W, W * sizeof(float));
            memcpy(cur, out, sizeof(cur));
        }
        ++kv;
        head_row(m, cur, ln_f, fnorm, last_logits);
        /* the history: the caller's prefix, or else the start token; then
         * every prediction so far (the loop stops at the first stop token, so
         * these are input tokens 1..) */
        const uint32_t* hist = input_tokens;
        uint32_t n_hist = res->n_input;
        if (history_prefix) {
            for (uint32_t i = 1; i < res->n_input; ++i) history[n_history_prefix + i - 1] = input_tokens[i];
            hist = history;
            n_hist = n_history_prefix + res->n_input - 1;
        }
        if (orc_gpt_sampling_processors(last_logits, VOCAB, hist, n_hist, temperature, top_k, top_p,
                                        repetition_penalty, last_processed) != 0) { rc = -1; break; }
        const uint32_t next = orc_gpt_sample_token(last_processed, VOCAB, &rng);
        predicted[res->n_predicted++] = next;
        if (next == STOP_TOKEN) {
            res->first_stop_step = (int32_t)step;
            break;
        }
        input_tokens[res->n_input++] = next;
    }
    free(ck); free(cv); free(hid); free(nxt); free(qkv); free(history);
    return rc;
}
