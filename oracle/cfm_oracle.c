/*
 * cfm_oracle.c -- CPU restatement of the reference's fp32 DiT-CFM path.
 *
 * TEST INFRASTRUCTURE ONLY (see cfm_oracle.h): the reference the HIP path is
 * compared with, and the timed CPU baseline.  Nothing in the product library calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp, no fast-math).
 * -ffp-contract=off keeps every multiply and add a separately rounded IEEE
 * operation, so the result does not depend on whether the host has FMA.
 *
 * Reference files cited below are relative to the reference repository root.
 */
#include "cfm_oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;
static char g_err[512];

static void set_err(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

const char* orc_last_error(void) { return g_err; }

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int orc_get_threads(void) { return g_threads; }

static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "cfm_oracle: out of memory (%zu bytes)\n", n);
        abort();
    }
    return p;
}

static float* fbuf(size_t n) { return (float*)xmalloc(n * sizeof(float)); }

static float* fzeros(size_t n) {
    float* p = fbuf(n);
    memset(p, 0, n * sizeof(float));
    return p;
}

/* ------------------------------------------------------------------------ */
/* f16 -> f32, tokenizer_tests.cpp:4284-4309                                  */
/* ------------------------------------------------------------------------ */
float orc_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x03ffu;
    uint32_t bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: shift the mantissa up until the implicit bit appears */
            int e = 1;
            while ((mant & 0x0400u) == 0) {
                mant <<= 1;
                --e;
            }
            mant &= 0x03ffu;
            bits = sign | ((uint32_t)(e + 127 - 15) << 23) | (mant << 13);
        }
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((ex + 127 - 15) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

void orc_halves_to_floats(const uint16_t* h, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_half_to_float(h[i]);
}

/* ------------------------------------------------------------------------ */
/* splitmix64 + Box-Muller, tokenizer_tests.cpp:2102-2140                     */
/* ------------------------------------------------------------------------ */
uint64_t orc_splitmix64_next(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

float orc_uniform_open01(uint64_t* state) {
    const double scale = 1.0 / (double)(1ull << 53);
    const uint64_t bits = orc_splitmix64_next(state) >> 11;
    double value = ((double)bits + 0.5) * scale;
    if (value <= 0.0) {
        value = scale;
    } else if (value >= 1.0) {
        value = 1.0 - scale;
    }
    return (float)value;
}

void orc_normal_noise(uint32_t tokens, uint32_t channels, uint64_t seed, float temperature,
                      float* out) {
    const float two_pi = 6.2831853071795864769f;
    const size_t n = (size_t)tokens * channels;
    uint64_t state = seed;
    size_t i = 0;
    while (i < n) {
        const float u1 = orc_uniform_open01(&state);
        const float u2 = orc_uniform_open01(&state);
        const float radius = sqrtf(-2.0f * logf(u1));
        const float angle = two_pi * u2;
        out[i++] = radius * cosf(angle) * temperature;
        if (i < n) out[i++] = radius * sinf(angle) * temperature;
    }
}

/* ------------------------------------------------------------------------ */
/* norms and linear, tokenizer_tests.cpp:2992-3036                            */
/* ------------------------------------------------------------------------ */
void orc_layernorm(const float* x, const float* gamma, const float* beta, uint32_t n, float eps,
                   float* out) {
    float mean = 0.0f;
    for (uint32_t i = 0; i < n; ++i) mean += x[i];
    mean /= (float)n;
    float var = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        const float d = x[i] - mean;
        var += d * d;
    }
    var /= (float)n;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (uint32_t i = 0; i < n; ++i) out[i] = (x[i] - mean) * inv_std * gamma[i] + beta[i];
}

void orc_rmsnorm(const float* x, const float* gamma, uint32_t n, float eps, float* out) {
    float mean_sq = 0.0f;
    for (uint32_t i = 0; i < n; ++i) mean_sq += x[i] * x[i];
    mean_sq /= (float)n;
    const float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    for (uint32_t i = 0; i < n; ++i) out[i] = x[i] * inv_rms * gamma[i];
}

/* cpu_linear: out[row] = bias[row] + sum_col w[row,col]*x[col], the sum taken
 * left to right.  Eight output rows are walked together only to give the CPU
 * independent dependency chains; each row's own chain is unchanged. */
void orc_linear(const float* w, const float* b, const float* x, uint32_t rows, uint32_t cols,
                float* out) {
    uint32_t row = 0;
    for (; row + 8 <= rows; row += 8) {
        float acc[8];
        for (int j = 0; j < 8; ++j) acc[j] = b[row + j];
        const float* wr = w + (size_t)row * cols;
        for (uint32_t col = 0; col < cols; ++col) {
            const float xv = x[col];
            for (int j = 0; j < 8; ++j) acc[j] += wr[(size_t)j * cols + col] * xv;
        }
        for (int j = 0; j < 8; ++j) out[row + j] = acc[j];
    }
    for (; row < rows; ++row) {
        float acc = b[row];
        const float* wr = w + (size_t)row * cols;
        for (uint32_t col = 0; col < cols; ++col) acc += wr[col] * x[col];
        out[row] = acc;
    }
}

void orc_linear_rows(const float* w, const float* b, const float* x, uint32_t tokens,
                     uint32_t rows, uint32_t cols, float* out) {
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)tokens; ++t) {
        orc_linear(w, b, x + (size_t)t * cols, rows, cols, out + (size_t)t * rows);
    }
}

/* ------------------------------------------------------------------------ */
/* length regulator pieces                                                    */
/* ------------------------------------------------------------------------ */
/* cpu_nearest_interpolate (tokenizer_tests.cpp:3127-3140): in_t =
 * floor(out_t * (in/out)) with the scale and the product in float, clamped. */
void orc_nearest_interpolate(const float* x, uint32_t in_tokens, uint32_t out_tokens,
                             uint32_t width, float* out) {
    const float scale = (float)in_tokens / (float)out_tokens;
    for (uint32_t t = 0; t < out_tokens; ++t) {
        uint32_t src = (uint32_t)floorf((float)t * scale);
        if (src >= in_tokens) src = in_tokens - 1;
        memcpy(out + (size_t)t * width, x + (size_t)src * width, width * sizeof(float));
    }
}

/* cpu_groupnorm1 (tokenizer_tests.cpp:3874-3896): one group over all
 * tokens x channels; mean and variance are single fp32 accumulators walked in
 * memory order, as the reference does. */
void orc_groupnorm1(const float* x, const float* gamma, const float* beta, uint32_t tokens,
                    uint32_t channels, float eps, float* out) {
    const size_t count = (size_t)tokens * channels;
    float mean = 0.0f;
    for (size_t i = 0; i < count; ++i) mean += x[i];
    mean /= (float)count;
    float var = 0.0f;
    for (size_t i = 0; i < count; ++i) {
        const float d = x[i] - mean;
        var += d * d;
    }
    var /= (float)count;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (uint32_t t = 0; t < tokens; ++t)
        for (uint32_t c = 0; c < channels; ++c) {
            const size_t i = (size_t)t * channels + c;
            out[i] = (x[i] - mean) * inv_std * gamma[c] + beta[c];
        }
}

/* cpu_mish (tokenizer_tests.cpp:3898-3904): x * tanh(log1p(exp(x))). */
void orc_mish(const float* x, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * tanhf(log1pf(expf(x[i])));
}

/* cpu_groupnorm1 with its two statistics (the mean, then the mean of the
 * squared deviations) reduced in double and rounded to float once, instead of
 * the reference's sequential float sums.  Not the reference's arithmetic: a
 * checker for how far those sequential sums alone move the result (over
 * 10^5 values they carry ~1e-5 relative rounding error). */
void orc_groupnorm1_f64stats(const float* x, const float* gamma, const float* beta, uint32_t tokens,
                             uint32_t channels, float eps, float* out) {
    const size_t count = (size_t)tokens * channels;
    double m = 0.0;
    for (size_t i = 0; i < count; ++i) m += x[i];
    m /= (double)count;
    double v = 0.0;
    for (size_t i = 0; i < count; ++i) v += ((double)x[i] - m) * ((double)x[i] - m);
    v /= (double)count;
    const float mean = (float)m;
    const float inv_std = (float)(1.0 / sqrt(v + (double)eps));
    for (uint32_t t = 0; t < tokens; ++t)
        for (uint32_t c = 0; c < channels; ++c) {
            const size_t i = (size_t)t * channels + c;
            out[i] = (x[i] - mean) * inv_std * gamma[c] + beta[c];
        }
}

/* run_length_regulator_full_cpu (gpt.cpp:5298-5313) with its front
 * (gpt.cpp:5271-5281): content_in_proj per input token, nearest
 * interpolation, 4 x (conv k=3, groupnorm1 eps 1e-5, mish), conv k=1.
 * f64_stats != 0 swaps in orc_groupnorm1_f64stats (checker only). */
void orc_length_regulator_ex(const float* input, uint32_t in_tokens, uint32_t out_tokens,
                             const float* proj_w, const float* proj_b,
                             const float* const* conv_w, const float* const* conv_b,
                             const float* const* gn_w, const float* const* gn_b,
                             const float* out_w, const float* out_b, int f64_stats, float* out) {
    float* projected = fbuf((size_t)in_tokens * 512);
    orc_linear_rows(proj_w, proj_b, input, in_tokens, 512, 1024, projected);
    float* x = fbuf((size_t)out_tokens * 512);
    float* y = fbuf((size_t)out_tokens * 512);
    orc_nearest_interpolate(projected, in_tokens, out_tokens, 512, x);
    for (int blk = 0; blk < 4; ++blk) {
        orc_conv1d_same(x, conv_w[blk], conv_b[blk], out_tokens, 512, 512, 3, y);
        if (f64_stats)
            orc_groupnorm1_f64stats(y, gn_w[blk], gn_b[blk], out_tokens, 512, 1e-5f, x);
        else
            orc_groupnorm1(y, gn_w[blk], gn_b[blk], out_tokens, 512, 1e-5f, x);
        orc_mish(x, (size_t)out_tokens * 512, x);
    }
    orc_conv1d_same(x, out_w, out_b, out_tokens, 512, 512, 1, out);
    free(projected);
    free(x);
    free(y);
}

void orc_length_regulator(const float* input, uint32_t in_tokens, uint32_t out_tokens,
                          const float* proj_w, const float* proj_b,
                          const float* const* conv_w, const float* const* conv_b,
                          const float* const* gn_w, const float* const* gn_b,
                          const float* out_w, const float* out_b, float* out) {
    orc_length_regulator_ex(input, in_tokens, out_tokens, proj_w, proj_b, conv_w, conv_b, gn_w, gn_b,
                            out_w, out_b, 0, out);
}

/* ------------------------------------------------------------------------ */
/* conv1d, tokenizer_tests.cpp:3142-3161, 3836-3872                          */
/* ------------------------------------------------------------------------ */
/* One output token of cpu_conv1d_same: acc = bias; for in_c: for k: acc += x*w
 * (taps outside [0,tokens) skipped).  Eight output channels walked together. */
static void conv_token(const float* x, const float* w, const float* b, uint32_t tokens,
                       uint32_t in_ch, uint32_t out_ch, uint32_t kernel, uint32_t t,
                       float* out_row) {
    const int pad = (int)(kernel / 2);
    uint32_t oc = 0;
    for (; oc + 8 <= out_ch; oc += 8) {
        float acc[8];
        for (int j = 0; j < 8; ++j) acc[j] = b[oc + j];
        for (uint32_t ic = 0; ic < in_ch; ++ic) {
            for (uint32_t k = 0; k < kernel; ++k) {
                const int src = (int)t + (int)k - pad;
                if (src >= 0 && src < (int)tokens) {
                    const float xv = x[(size_t)src * in_ch + ic];
                    for (int j = 0; j < 8; ++j)
                        acc[j] += xv * w[((size_t)(oc + j) * in_ch + ic) * kernel + k];
                }
            }
        }
        for (int j = 0; j < 8; ++j) out_row[oc + j] = acc[j];
    }
    for (; oc < out_ch; ++oc) {
        float acc = b[oc];
        for (uint32_t ic = 0; ic < in_ch; ++ic) {
            for (uint32_t k = 0; k < kernel; ++k) {
                const int src = (int)t + (int)k - pad;
                if (src >= 0 && src < (int)tokens)
                    acc += x[(size_t)src * in_ch + ic] * w[((size_t)oc * in_ch + ic) * kernel + k];
            }
        }
        out_row[oc] = acc;
    }
}

void orc_conv1d_same(const float* x, const float* w, const float* b, uint32_t tokens,
                     uint32_t in_ch, uint32_t out_ch, uint32_t kernel, float* out) {
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)tokens; ++t) {
        conv_token(x, w, b, tokens, in_ch, out_ch, kernel, (uint32_t)t, out + (size_t)t * out_ch);
    }
}

void orc_reflect_pad(const float* x, uint32_t tokens, uint32_t channels, uint32_t pad_left,
                     uint32_t pad_right, float* out) {
    const uint32_t out_tokens = tokens + pad_left + pad_right;
    for (uint32_t t = 0; t < out_tokens; ++t) {
        int src = (int)t - (int)pad_left;
        /* The reference loops "while (src<0 || src>=tokens)"; for tokens == 1
         * that loop never ends (src flips between -p and p), so the oracle
         * refuses instead of hanging. */
        if (tokens == 1 && src != 0) {
            fprintf(stderr, "cfm_oracle: reflect padding of a 1-token sequence never terminates "
                            "in the reference\n");
            abort();
        }
        while (src < 0 || src >= (int)tokens) {
            if (src < 0) src = -src;
            if (src >= (int)tokens) src = 2 * (int)tokens - 2 - src;
        }
        memcpy(out + (size_t)t * channels, x + (size_t)src * channels, channels * sizeof(float));
    }
}

void orc_conv1d_reflect_same(const float* x, const float* w, const float* b, uint32_t tokens,
                             uint32_t in_ch, uint32_t out_ch, uint32_t kernel, float* out) {
    const uint32_t pl = kernel / 2;
    const uint32_t pr = kernel - 1 - pl;
    const uint32_t padded_tokens = tokens + pl + pr;
    float* padded = fbuf((size_t)padded_tokens * in_ch);
    orc_reflect_pad(x, tokens, in_ch, pl, pr, padded);
    /* conv over the padded sequence, then slice_tokens(full, pl, tokens): only
     * the kept rows are computed (the others are discarded by the reference). */
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)tokens; ++t) {
        conv_token(padded, w, b, padded_tokens, in_ch, out_ch, kernel, (uint32_t)t + pl,
                   out + (size_t)t * out_ch);
    }
    free(padded);
}

/* ------------------------------------------------------------------------ */
/* timestep embedding, attention, RoPE, weight norm                          */
/* ------------------------------------------------------------------------ */
void orc_timestep_embedding(const float* t, uint32_t n_t, const float* freqs, uint32_t half,
                            float scale, float* out) {
    for (uint32_t b = 0; b < n_t; ++b) {
        for (uint32_t i = 0; i < half; ++i) {
            const float arg = scale * t[b] * freqs[i];
            out[(size_t)b * half * 2 + i] = cosf(arg);
            out[(size_t)b * half * 2 + half + i] = sinf(arg);
        }
    }
}

/* One query row of cpu_attention_single_head_masked (tokenizer_tests.cpp:3960). */
static void attention_query(const float* q, const float* k, const float* v, const uint32_t* key_mask,
                            uint32_t tokens, uint32_t head_dim, uint32_t tq, float* scores,
                            float* out_row) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    float max_score = -INFINITY;
    for (uint32_t tk = 0; tk < tokens; ++tk) {
        if (key_mask[tk] == 0) {
            scores[tk] = -INFINITY;
            continue;
        }
        float score = 0.0f;
        for (uint32_t d = 0; d < head_dim; ++d)
            score += q[(size_t)tq * head_dim + d] * k[(size_t)tk * head_dim + d];
        score *= scale;
        scores[tk] = score;
        if (score > max_score) max_score = score; /* std::max(max_score, score) */
    }
    float denom = 0.0f;
    for (uint32_t tk = 0; tk < tokens; ++tk) {
        float s = scores[tk];
        if (!isfinite(s)) {
            scores[tk] = 0.0f;
            continue;
        }
        s = expf(s - max_score);
        scores[tk] = s;
        denom += s;
    }
    /* scores[tk] / denom is the same value for every d; take it once. */
    for (uint32_t tk = 0; tk < tokens; ++tk) scores[tk] = scores[tk] / denom;
    for (uint32_t d = 0; d < head_dim; ++d) {
        float acc = 0.0f;
        for (uint32_t tk = 0; tk < tokens; ++tk) acc += scores[tk] * v[(size_t)tk * head_dim + d];
        out_row[d] = acc;
    }
}

void orc_attention_head_masked(const float* q, const float* k, const float* v,
                               const uint32_t* key_mask, uint32_t tokens, uint32_t head_dim,
                               float* out) {
    long tq;
#pragma omp parallel num_threads(g_threads)
    {
        float* scores = fbuf(tokens);
#pragma omp for schedule(static)
        for (tq = 0; tq < (long)tokens; ++tq)
            attention_query(q, k, v, key_mask, tokens, head_dim, (uint32_t)tq, scores,
                            out + (size_t)tq * head_dim);
        free(scores);
    }
}

void orc_rope_inplace(float* x, uint32_t tokens, uint32_t heads, uint32_t head_dim) {
    for (uint32_t t = 0; t < tokens; ++t) {
        for (uint32_t pair = 0; pair < head_dim / 2; ++pair) {
            const float theta =
                (float)t / powf(10000.0f, (float)(pair * 2) / (float)head_dim);
            const float c = cosf(theta);
            const float s = sinf(theta);
            for (uint32_t h = 0; h < heads; ++h) {
                const size_t base = ((size_t)t * heads + h) * head_dim + pair * 2;
                const float a = x[base];
                const float bb = x[base + 1];
                x[base] = a * c - bb * s;
                x[base + 1] = bb * c + a * s;
            }
        }
    }
}

void orc_weight_norm_rowmajor(const float* g, const float* v, uint32_t rows, uint32_t cols,
                              float* out) {
    for (uint32_t row = 0; row < rows; ++row) {
        float norm = 0.0f;
        for (uint32_t col = 0; col < cols; ++col) {
            const float value = v[(size_t)row * cols + col];
            norm += value * value;
        }
        norm = sqrtf(norm);
        const float scale = g[row] / norm;
        for (uint32_t col = 0; col < cols; ++col)
            out[(size_t)row * cols + col] = v[(size_t)row * cols + col] * scale;
    }
}

/* ------------------------------------------------------------------------ */
/* model tensor table                                                         */
/* ------------------------------------------------------------------------ */
#define PFX "s2mel.net.cfm.estimator."
#define MAX_TENSORS 320

typedef struct {
    char name[160];
    uint64_t elems;
} tensor_spec;

static tensor_spec g_specs[MAX_TENSORS];
static int g_nspecs = 0;

static void add_spec(uint64_t elems, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    char tail[96];
    vsnprintf(tail, sizeof tail, fmt, ap);
    va_end(ap);
    snprintf(g_specs[g_nspecs].name, sizeof g_specs[0].name, PFX "%s", tail);
    g_specs[g_nspecs].elems = elems;
    ++g_nspecs;
}

static void init_specs(void) {
    if (g_nspecs) return;
    const char* te[2] = {"t_embedder", "t_embedder2"};
    for (int i = 0; i < 2; ++i) {
        add_spec(128, "%s.freqs", te[i]);
        add_spec(512 * 256, "%s.mlp.0.weight", te[i]);
        add_spec(512, "%s.mlp.0.bias", te[i]);
        add_spec(512 * 512, "%s.mlp.2.weight", te[i]);
        add_spec(512, "%s.mlp.2.bias", te[i]);
    }
    add_spec(512 * 512, "cond_projection.weight");
    add_spec(512, "cond_projection.bias");
    add_spec(512 * 864, "cond_x_merge_linear.weight");
    add_spec(512, "cond_x_merge_linear.bias");
    for (int l = 0; l < 13; ++l) {
        const char* nn[2] = {"attention_norm", "ffn_norm"};
        for (int j = 0; j < 2; ++j) {
            add_spec(512, "transformer.layers.%d.%s.norm.weight", l, nn[j]);
            add_spec(1024 * 512, "transformer.layers.%d.%s.project_layer.weight", l, nn[j]);
            add_spec(1024, "transformer.layers.%d.%s.project_layer.bias", l, nn[j]);
        }
        add_spec(1536 * 512, "transformer.layers.%d.attention.wqkv.weight", l);
        add_spec(512 * 512, "transformer.layers.%d.attention.wo.weight", l);
        add_spec(1536 * 512, "transformer.layers.%d.feed_forward.w1.weight", l);
        add_spec(1536 * 512, "transformer.layers.%d.feed_forward.w3.weight", l);
        add_spec(512 * 1536, "transformer.layers.%d.feed_forward.w2.weight", l);
        if (l > 6) {
            add_spec(512 * 1024, "transformer.layers.%d.skip_in_linear.weight", l);
            add_spec(512, "transformer.layers.%d.skip_in_linear.bias", l);
        }
    }
    add_spec(512, "transformer.norm.norm.weight");
    add_spec(1024 * 512, "transformer.norm.project_layer.weight");
    add_spec(1024, "transformer.norm.project_layer.bias");
    add_spec(512 * 592, "skip_linear.weight");
    add_spec(512, "skip_linear.bias");
    add_spec(512 * 512, "conv1.weight");
    add_spec(512, "conv1.bias");
    add_spec(512 * 512, "res_projection.weight");
    add_spec(512, "res_projection.bias");
    add_spec(8192, "wavenet.cond_layer.conv.conv.weight_g");
    add_spec(8192 * 512, "wavenet.cond_layer.conv.conv.weight_v");
    add_spec(8192, "wavenet.cond_layer.conv.conv.bias");
    for (int l = 0; l < 8; ++l) {
        add_spec(1024, "wavenet.in_layers.%d.conv.conv.weight_g", l);
        add_spec(1024 * 512 * 5, "wavenet.in_layers.%d.conv.conv.weight_v", l);
        add_spec(1024, "wavenet.in_layers.%d.conv.conv.bias", l);
    }
    for (int l = 0; l < 8; ++l) {
        const uint64_t c = l < 7 ? 1024 : 512;
        add_spec(c, "wavenet.res_skip_layers.%d.conv.conv.weight_g", l);
        add_spec(c * 512, "wavenet.res_skip_layers.%d.conv.conv.weight_v", l);
        add_spec(c, "wavenet.res_skip_layers.%d.conv.conv.bias", l);
    }
    add_spec(1024 * 512, "final_layer.adaLN_modulation.1.weight");
    add_spec(1024, "final_layer.adaLN_modulation.1.bias");
    add_spec(512, "final_layer.linear.weight_g");
    add_spec(512 * 512, "final_layer.linear.weight_v");
    add_spec(512, "final_layer.linear.bias");
    add_spec(80 * 512, "conv2.weight");
    add_spec(80, "conv2.bias");
}

struct orc_model {
    float* data[MAX_TENSORS];
};

int orc_model_tensor_count(void) {
    init_specs();
    return g_nspecs;
}

const char* orc_model_tensor_name(int i) {
    init_specs();
    return (i >= 0 && i < g_nspecs) ? g_specs[i].name : NULL;
}

uint64_t orc_model_tensor_elems(int i) {
    init_specs();
    return (i >= 0 && i < g_nspecs) ? g_specs[i].elems : 0;
}

orc_model* orc_model_new(void) {
    init_specs();
    orc_model* m = (orc_model*)xmalloc(sizeof *m);
    memset(m, 0, sizeof *m);
    return m;
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    for (int i = 0; i < MAX_TENSORS; ++i) free(m->data[i]);
    free(m);
}

static int spec_index(const char* name) {
    init_specs();
    for (int i = 0; i < g_nspecs; ++i)
        if (strcmp(g_specs[i].name, name) == 0) return i;
    return -1;
}

int orc_model_set(orc_model* m, const char* name, const float* data, uint64_t count) {
    const int i = spec_index(name);
    if (i < 0) {
        set_err("unknown tensor: %s", name);
        return -1;
    }
    if (count != g_specs[i].elems) {
        set_err("tensor %s: %llu elements, expected %llu", name, (unsigned long long)count,
                (unsigned long long)g_specs[i].elems);
        return -1;
    }
    free(m->data[i]);
    m->data[i] = fbuf(count);
    memcpy(m->data[i], data, count * sizeof(float));
    return 0;
}

int orc_model_missing(const orc_model* m) {
    int missing = 0;
    for (int i = 0; i < g_nspecs; ++i) {
        if (!m->data[i]) {
            if (!missing) set_err("missing tensor: %s", g_specs[i].name);
            ++missing;
        }
    }
    return missing;
}

/* tensor_as_f32(bundle, PFX + formatted tail) */
static const float* W(const orc_model* m, const char* fmt, ...) {
    char tail[96], name[160];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(tail, sizeof tail, fmt, ap);
    va_end(ap);
    snprintf(name, sizeof name, PFX "%s", tail);
    const int i = spec_index(name);
    if (i < 0 || !m->data[i]) {
        fprintf(stderr, "cfm_oracle: missing tensor %s\n", name);
        abort();
    }
    return m->data[i];
}

/* weight_norm_conv_weight (gpt.cpp:5126): g, v -> [out, in*k] */
static float* wn_weight(const orc_model* m, const char* prefix, uint32_t out_ch, uint32_t in_ch,
                        uint32_t kernel) {
    float* w = fbuf((size_t)out_ch * in_ch * kernel);
    orc_weight_norm_rowmajor(W(m, "%s.weight_g", prefix), W(m, "%s.weight_v", prefix), out_ch,
                             in_ch * kernel, w);
    return w;
}

/* ------------------------------------------------------------------------ */
/* estimator stages                                                           */
/* ------------------------------------------------------------------------ */
static inline float silu(float v) { return v / (1.0f + expf(-v)); }

/* gpt.cpp:5404-5422 */
void orc_timestep_embedder(const orc_model* m, float t, int which, float* out512) {
    const char* pfx = which == 2 ? "t_embedder2" : "t_embedder";
    float emb[256], h[512];
    orc_timestep_embedding(&t, 1, W(m, "%s.freqs", pfx), 128, 1000.0f, emb);
    orc_linear(W(m, "%s.mlp.0.weight", pfx), W(m, "%s.mlp.0.bias", pfx), emb, 512, 256, h);
    for (int i = 0; i < 512; ++i) h[i] = silu(h[i]);
    orc_linear(W(m, "%s.mlp.2.weight", pfx), W(m, "%s.mlp.2.bias", pfx), h, 512, 512, out512);
}

/* dit_cfm_bigvgan.cpp:1-19 */
void orc_input_merge(const orc_model* m, const float* x, const float* prompt_x, const float* cond,
                     const float* style, uint32_t T, float* out) {
    const float* cw = W(m, "cond_projection.weight");
    const float* cb = W(m, "cond_projection.bias");
    const float* mw = W(m, "cond_x_merge_linear.weight");
    const float* mb = W(m, "cond_x_merge_linear.bias");
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)T; ++t) {
        float merged[864];
        memcpy(merged, x + (size_t)t * 80, 80 * sizeof(float));
        memcpy(merged + 80, prompt_x + (size_t)t * 80, 80 * sizeof(float));
        orc_linear(cw, cb, cond + (size_t)t * 512, 512, 512, merged + 160);
        memcpy(merged + 672, style, 192 * sizeof(float));
        orc_linear(mw, mb, merged, 512, 864, out + (size_t)t * 512);
    }
}

static void norm_prefix(int norm_id, char* buf, size_t n) {
    if (norm_id < 13)
        snprintf(buf, n, "transformer.layers.%d.attention_norm", norm_id);
    else if (norm_id < 26)
        snprintf(buf, n, "transformer.layers.%d.ffn_norm", norm_id - 13);
    else
        snprintf(buf, n, "transformer.norm");
}

/* dit_cfm_bigvgan.cpp:260-276 */
void orc_adaptive_norm(const orc_model* m, const float* in, const float* cond512, uint32_t T,
                       int norm_id, float* out) {
    char p[64];
    norm_prefix(norm_id, p, sizeof p);
    const float* gamma = W(m, "%s.norm.weight", p);
    float wb[1024];
    orc_linear(W(m, "%s.project_layer.weight", p), W(m, "%s.project_layer.bias", p), cond512, 1024,
               512, wb);
    const float* aw = wb;
    const float* ab = wb + 512;
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)T; ++t) {
        float normed[512];
        orc_rmsnorm(in + (size_t)t * 512, gamma, 512, 1e-5f, normed);
        for (int i = 0; i < 512; ++i) out[(size_t)t * 512 + i] = aw[i] * normed[i] + ab[i];
    }
}

/* dit_cfm_bigvgan.cpp:469-512 */
void orc_attention_core(const orc_model* m, const float* in, const uint32_t* mask, uint32_t T,
                        uint32_t layer, float* out) {
    enum { H = 8, HD = 64 };
    const float* wqkv = W(m, "transformer.layers.%u.attention.wqkv.weight", layer);
    const float* wo = W(m, "transformer.layers.%u.attention.wo.weight", layer);
    float* zero = fzeros(1536);
    float* qkv = fbuf((size_t)T * 1536);
    orc_linear_rows(wqkv, zero, in, T, 1536, 512, qkv);
    float* q = fbuf((size_t)T * 512);
    float* k = fbuf((size_t)T * 512);
    float* v = fbuf((size_t)T * 512);
    for (uint32_t t = 0; t < T; ++t) {
        memcpy(q + (size_t)t * 512, qkv + (size_t)t * 1536, 512 * sizeof(float));
        memcpy(k + (size_t)t * 512, qkv + (size_t)t * 1536 + 512, 512 * sizeof(float));
        memcpy(v + (size_t)t * 512, qkv + (size_t)t * 1536 + 1024, 512 * sizeof(float));
    }
    orc_rope_inplace(q, T, H, HD);
    orc_rope_inplace(k, T, H, HD);
    float* concat = fbuf((size_t)T * 512);
    float* qh = fbuf((size_t)T * HD);
    float* kh = fbuf((size_t)T * HD);
    float* vh = fbuf((size_t)T * HD);
    float* yh = fbuf((size_t)T * HD);
    for (uint32_t h = 0; h < H; ++h) {
        for (uint32_t t = 0; t < T; ++t) {
            const size_t src = ((size_t)t * H + h) * HD;
            memcpy(qh + (size_t)t * HD, q + src, HD * sizeof(float));
            memcpy(kh + (size_t)t * HD, k + src, HD * sizeof(float));
            memcpy(vh + (size_t)t * HD, v + src, HD * sizeof(float));
        }
        orc_attention_head_masked(qh, kh, vh, mask, T, HD, yh);
        for (uint32_t t = 0; t < T; ++t)
            memcpy(concat + (size_t)t * 512 + h * HD, yh + (size_t)t * HD, HD * sizeof(float));
    }
    orc_linear_rows(wo, zero, concat, T, 512, 512, out);
    free(zero); free(qkv); free(q); free(k); free(v);
    free(concat); free(qh); free(kh); free(vh); free(yh);
}

/* dit_cfm_bigvgan.cpp:727-746 (SwiGLU: silu(w1 x) * (w3 x), no biases) */
void orc_feed_forward(const orc_model* m, const float* in, uint32_t T, uint32_t layer, float* out) {
    const float* w1 = W(m, "transformer.layers.%u.feed_forward.w1.weight", layer);
    const float* w3 = W(m, "transformer.layers.%u.feed_forward.w3.weight", layer);
    const float* w2 = W(m, "transformer.layers.%u.feed_forward.w2.weight", layer);
    float* zero = fzeros(1536);
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)T; ++t) {
        float h1[1536], h3[1536];
        orc_linear(w1, zero, in + (size_t)t * 512, 1536, 512, h1);
        orc_linear(w3, zero, in + (size_t)t * 512, 1536, 512, h3);
        for (int i = 0; i < 1536; ++i) h1[i] = (h1[i] / (1.0f + expf(-h1[i]))) * h3[i];
        orc_linear(w2, zero, h1, 512, 1536, out + (size_t)t * 512);
    }
    free(zero);
}

/* dit_cfm_bigvgan.cpp:785-798 */
void orc_skip_in(const orc_model* m, const float* in, const float* skip, uint32_t T, uint32_t layer,
                 float* out) {
    const float* w = W(m, "transformer.layers.%u.skip_in_linear.weight", layer);
    const float* b = W(m, "transformer.layers.%u.skip_in_linear.bias", layer);
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)T; ++t) {
        float row[1024];
        memcpy(row, in + (size_t)t * 512, 512 * sizeof(float));
        memcpy(row + 512, skip + (size_t)t * 512, 512 * sizeof(float));
        orc_linear(w, b, row, 512, 1024, out + (size_t)t * 512);
    }
}

/* dit_cfm_bigvgan.cpp:816-832 */
void orc_transformer_block(const orc_model* m, const float* in, const float* t1,
                           const uint32_t* mask, uint32_t T, uint32_t layer, const float* skip,
                           float* out) {
    const size_t n = (size_t)T * 512;
    float* x = fbuf(n);
    if (skip)
        orc_skip_in(m, in, skip, T, layer, x);
    else
        memcpy(x, in, n * sizeof(float));
    float* normed = fbuf(n);
    float* attn = fbuf(n);
    float* h = fbuf(n);
    orc_adaptive_norm(m, x, t1, T, (int)layer, normed);
    orc_attention_core(m, normed, mask, T, layer, attn);
    for (size_t i = 0; i < n; ++i) h[i] = x[i] + attn[i];
    orc_adaptive_norm(m, h, t1, T, 13 + (int)layer, normed);
    orc_feed_forward(m, normed, T, layer, attn);
    for (size_t i = 0; i < n; ++i) out[i] = h[i] + attn[i];
    free(x); free(normed); free(attn); free(h);
}

/* dit_cfm_bigvgan.cpp:868-886: outputs of layers 0..5 are pushed, layers 7..12
 * pop them LIFO as the skip input, then the final adaptive norm. */
void orc_transformer_stack(const orc_model* m, const float* in, const float* t1,
                           const uint32_t* mask, uint32_t T, float* out) {
    const uint32_t layers = 13;
    const size_t n = (size_t)T * 512;
    float* skips[13];
    int nskips = 0;
    float* x = fbuf(n);
    float* y = fbuf(n);
    memcpy(x, in, n * sizeof(float));
    for (uint32_t layer = 0; layer < layers; ++layer) {
        const float* skip = NULL;
        if (layer > layers / 2) skip = skips[nskips - 1];
        orc_transformer_block(m, x, t1, mask, T, layer, skip, y);
        float* tmp = x;
        x = y;
        y = tmp;
        if (layer > layers / 2) free(skips[--nskips]);
        if (layer < layers / 2) {
            skips[nskips] = fbuf(n);
            memcpy(skips[nskips], x, n * sizeof(float));
            ++nskips;
        }
    }
    orc_adaptive_norm(m, x, t1, T, 26, out);
    while (nskips) free(skips[--nskips]);
    free(x); free(y);
}

/* dit_cfm_bigvgan.cpp:1053-1079 (the conv2 output computed there is unused by
 * the estimator and left out) */
void orc_post_transformer(const orc_model* m, const float* xres, const float* xmel, uint32_t T,
                          float* long_skip, float* conv1, float* res_proj) {
    const float* sw = W(m, "skip_linear.weight");
    const float* sb = W(m, "skip_linear.bias");
    const float* c1w = W(m, "conv1.weight");
    const float* c1b = W(m, "conv1.bias");
    const float* rw = W(m, "res_projection.weight");
    const float* rb = W(m, "res_projection.bias");
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)T; ++t) {
        float row[592];
        memcpy(row, xres + (size_t)t * 512, 512 * sizeof(float));
        memcpy(row + 512, xmel + (size_t)t * 80, 80 * sizeof(float));
        float* ls = long_skip + (size_t)t * 512;
        orc_linear(sw, sb, row, 512, 592, ls);
        orc_linear(c1w, c1b, ls, 512, 512, conv1 + (size_t)t * 512);
        orc_linear(rw, rb, ls, 512, 512, res_proj + (size_t)t * 512);
    }
}

/* dit_cfm_bigvgan.cpp:1464-1514 (global conditioning: one t2 vector) */
void orc_wavenet(const orc_model* m, const float* in, const float* t2, const uint32_t* mask,
                 uint32_t T, float* out) {
    const char* cpfx = "wavenet.cond_layer.conv.conv";
    float* cw = wn_weight(m, cpfx, 8192, 512, 1);
    float* cond = fbuf(8192);
    orc_conv1d_same(t2, cw, W(m, "%s.bias", cpfx), 1, 512, 8192, 1, cond);
    free(cw);

    const size_t n = (size_t)T * 512;
    float* x = fbuf(n);
    memcpy(x, in, n * sizeof(float));
    memset(out, 0, n * sizeof(float));
    float* in_layer = fbuf((size_t)T * 1024);
    float* gate = fbuf(n);
    float* res_skip = fbuf((size_t)T * 1024);
    for (uint32_t layer = 0; layer < 8; ++layer) {
        char ip[64], rp[64];
        snprintf(ip, sizeof ip, "wavenet.in_layers.%u.conv.conv", layer);
        float* iw = wn_weight(m, ip, 1024, 512, 5);
        orc_conv1d_reflect_same(x, iw, W(m, "%s.bias", ip), T, 512, 1024, 5, in_layer);
        free(iw);
        const uint32_t off = layer * 1024;
        for (uint32_t t = 0; t < T; ++t) {
            for (uint32_t c = 0; c < 512; ++c) {
                const float a = in_layer[(size_t)t * 1024 + c] + cond[off + c];
                const float b = in_layer[(size_t)t * 1024 + 512 + c] + cond[off + 512 + c];
                gate[(size_t)t * 512 + c] = tanhf(a) * (1.0f / (1.0f + expf(-b)));
            }
        }
        const uint32_t rs_ch = layer < 7 ? 1024 : 512;
        snprintf(rp, sizeof rp, "wavenet.res_skip_layers.%u.conv.conv", layer);
        float* rw = wn_weight(m, rp, rs_ch, 512, 1);
        orc_conv1d_same(gate, rw, W(m, "%s.bias", rp), T, 512, rs_ch, 1, res_skip);
        free(rw);
        if (layer < 7) {
            for (uint32_t t = 0; t < T; ++t) {
                const float mk = mask[t] ? 1.0f : 0.0f;
                for (uint32_t c = 0; c < 512; ++c) {
                    const size_t i = (size_t)t * 512 + c;
                    x[i] = (x[i] + res_skip[(size_t)t * 1024 + c]) * mk;
                    out[i] += res_skip[(size_t)t * 1024 + 512 + c];
                }
            }
        } else {
            for (size_t i = 0; i < n; ++i) out[i] += res_skip[i];
        }
    }
    for (uint32_t t = 0; t < T; ++t) {
        const float mk = mask[t] ? 1.0f : 0.0f;
        for (uint32_t c = 0; c < 512; ++c) out[(size_t)t * 512 + c] *= mk;
    }
    free(cond); free(x); free(in_layer); free(gate); free(res_skip);
}

/* dit_cfm_bigvgan.cpp:1172-1199 */
void orc_final_layer(const orc_model* m, const float* in, const float* t1, uint32_t T, float* out) {
    float* lw = fbuf(512 * 512);
    orc_weight_norm_rowmajor(W(m, "final_layer.linear.weight_g"), W(m, "final_layer.linear.weight_v"),
                             512, 512, lw);
    const float* lb = W(m, "final_layer.linear.bias");
    float t_silu[512], ss[1024];
    for (int i = 0; i < 512; ++i) t_silu[i] = t1[i] / (1.0f + expf(-t1[i]));
    orc_linear(W(m, "final_layer.adaLN_modulation.1.weight"), W(m, "final_layer.adaLN_modulation.1.bias"),
               t_silu, 1024, 512, ss);
    const float* shift = ss;
    const float* scale = ss + 512;
    float gamma[512], beta[512];
    for (int i = 0; i < 512; ++i) {
        gamma[i] = 1.0f;
        beta[i] = 0.0f;
    }
    long t;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (t = 0; t < (long)T; ++t) {
        float normed[512];
        orc_layernorm(in + (size_t)t * 512, gamma, beta, 512, 1e-6f, normed);
        for (int i = 0; i < 512; ++i) normed[i] = normed[i] * (1.0f + scale[i]) + shift[i];
        orc_linear(lw, lb, normed, 512, 512, out + (size_t)t * 512);
    }
    free(lw);
}

/* dit_cfm_bigvgan.cpp:1768-1788 */
void orc_estimator_step(const orc_model* m, const float* x, const float* prompt_x, const float* cond,
                        const float* style, float t, const uint32_t* mask, uint32_t T, float* out) {
    const size_t n = (size_t)T * 512;
    float t1[512], t2[512];
    orc_timestep_embedder(m, t, 1, t1);
    orc_timestep_embedder(m, t, 2, t2);
    float* x_in = fbuf(n);
    float* x_res = fbuf(n);
    orc_input_merge(m, x, prompt_x, cond, style, T, x_in);
    orc_transformer_stack(m, x_in, t1, mask, T, x_res);
    float* ls = fbuf(n);
    float* c1 = fbuf(n);
    float* rp = fbuf(n);
    orc_post_transformer(m, x_res, x, T, ls, c1, rp);
    float* wav = fbuf(n);
    orc_wavenet(m, c1, t2, mask, T, wav);
    for (size_t i = 0; i < n; ++i) wav[i] = wav[i] + rp[i];
    float* hid = fbuf(n);
    orc_final_layer(m, wav, t1, T, hid);
    orc_conv1d_same(hid, W(m, "conv2.weight"), W(m, "conv2.bias"), T, 512, 80, 1, out);
    free(x_in); free(x_res); free(ls); free(c1); free(rp); free(wav); free(hid);
}

/* dit_cfm_bigvgan.cpp:2908-2937.  The reference always passes an all-ones
 * mask; key_mask (NULL = all ones) extends it to a right-padded request,
 * using the estimator's masked semantics at the padded length. */
/* The first run_steps steps of the steps-step schedule (run_steps >= steps:
 * the whole decode). */
static void cfm_euler_impl(const orc_model* m, float* x, const float* prompt, const float* cond,
                           const float* style, const uint32_t* key_mask, uint32_t T, uint32_t P,
                           uint32_t steps, uint32_t run_steps, float cfg_rate, float* x_trace,
                           float* v_trace) {
    const size_t nx = (size_t)T * 80;
    float* prompt_x = fzeros(nx);
    for (uint32_t t = 0; t < P; ++t) {
        memcpy(prompt_x + (size_t)t * 80, prompt + (size_t)t * 80, 80 * sizeof(float));
        memset(x + (size_t)t * 80, 0, 80 * sizeof(float));
    }
    float* null_prompt_x = fzeros(nx);
    float* null_cond = fzeros((size_t)T * 512);
    float* null_style = fzeros(192);
    uint32_t* mask = (uint32_t*)xmalloc(T * sizeof(uint32_t));
    for (uint32_t t = 0; t < T; ++t) mask[t] = key_mask ? key_mask[t] : 1;
    float* dphi = fbuf(nx);
    float* cfg_dphi = fbuf(nx);
    float t = 0.0f;
    const float dt = 1.0f / (float)steps;
    for (uint32_t step = 1; step <= steps && step <= run_steps; ++step) {
        if (x_trace) memcpy(x_trace + (size_t)(step - 1) * nx, x, nx * sizeof(float));
        orc_estimator_step(m, x, prompt_x, cond, style, t, mask, T, dphi);
        if (cfg_rate > 0.0f) {
            orc_estimator_step(m, x, null_prompt_x, null_cond, null_style, t, mask, T, cfg_dphi);
            for (size_t i = 0; i < nx; ++i)
                dphi[i] = (1.0f + cfg_rate) * dphi[i] - cfg_rate * cfg_dphi[i];
        }
        if (v_trace) memcpy(v_trace + (size_t)(step - 1) * nx, dphi, nx * sizeof(float));
        for (size_t i = 0; i < nx; ++i) x[i] += dt * dphi[i];
        t += dt;
        for (uint32_t p = 0; p < P; ++p) memset(x + (size_t)p * 80, 0, 80 * sizeof(float));
    }
    free(prompt_x); free(null_prompt_x); free(null_cond); free(null_style);
    free(mask); free(dphi); free(cfg_dphi);
}

void orc_cfm_euler_trace(const orc_model* m, float* x, const float* prompt, const float* cond,
                         const float* style, uint32_t T, uint32_t P, uint32_t steps, float cfg_rate,
                         float* x_trace, float* v_trace) {
    cfm_euler_impl(m, x, prompt, cond, style, NULL, T, P, steps, steps, cfg_rate, x_trace, v_trace);
}

void orc_cfm_euler_partial(const orc_model* m, float* x, const float* prompt, const float* cond,
                           const float* style, uint32_t T, uint32_t P, uint32_t steps,
                           uint32_t run_steps, float cfg_rate, float* x_trace, float* v_trace) {
    cfm_euler_impl(m, x, prompt, cond, style, NULL, T, P, steps, run_steps, cfg_rate, x_trace,
                   v_trace);
}

void orc_cfm_euler(const orc_model* m, float* x, const float* prompt, const float* cond,
                   const float* style, uint32_t T, uint32_t P, uint32_t steps, float cfg_rate) {
    cfm_euler_impl(m, x, prompt, cond, style, NULL, T, P, steps, steps, cfg_rate, NULL, NULL);
}

void orc_cfm_euler_masked(const orc_model* m, float* x, const float* prompt, const float* cond,
                          const float* style, const uint32_t* key_mask, uint32_t T, uint32_t P,
                          uint32_t steps, float cfg_rate) {
    cfm_euler_impl(m, x, prompt, cond, style, key_mask, T, P, steps, steps, cfg_rate, NULL, NULL);
}
