/*
 * bigvgan_oracle.c -- CPU restatement of the reference's fp32 BigVGAN vocoder
 * primitives (the consumer of the DiT-CFM mel).
 *
 * TEST INFRASTRUCTURE ONLY (see cfm_oracle.h): loaded by tests/, smoke() and
 * bench.py's cpu_baseline leg, to compare results with or as the timed CPU
 * baseline.
 *
 * Each function keeps the reference's loop order and scalar fp32
 * accumulation; threads split output tokens only, so results are bit-identical
 * for every thread count.  The model-level composition (resblocks, the body,
 * the post stage) is in oracle.py on top of these primitives.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "cfm_oracle.h"

/* cpu_conv1d_dilated_same (runtime/impl/tokenizer_tests.cpp:3739-3757):
 * pad = (kernel-1)*dilation/2, zero outside [0, tokens); acc = bias, then
 * for in_c: for k: acc += x * w[(oc*in + ic)*kernel + k].  Eight output
 * channels are walked together; each keeps the reference's order. */
static void dil_conv_token(const float* x, const float* w, const float* b, uint32_t tokens,
                           uint32_t in_ch, uint32_t out_ch, uint32_t kernel, uint32_t dilation,
                           uint32_t t, float* out_row) {
    const int pad = (int)((kernel - 1) * dilation / 2);
    uint32_t oc = 0;
    for (; oc + 8 <= out_ch; oc += 8) {
        float acc[8];
        for (int j = 0; j < 8; ++j) acc[j] = b[oc + j];
        for (uint32_t ic = 0; ic < in_ch; ++ic) {
            for (uint32_t k = 0; k < kernel; ++k) {
                const int src = (int)t + (int)(k * dilation) - pad;
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
                const int src = (int)t + (int)(k * dilation) - pad;
                if (src >= 0 && src < (int)tokens)
                    acc += x[(size_t)src * in_ch + ic] * w[((size_t)oc * in_ch + ic) * kernel + k];
            }
        }
        out_row[oc] = acc;
    }
}

void orc_conv1d_dilated_same(const float* x, const float* w, const float* b, uint32_t tokens,
                             uint32_t in_ch, uint32_t out_ch, uint32_t kernel, uint32_t dilation,
                             float* out) {
    long t;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (t = 0; t < (long)tokens; ++t)
        dil_conv_token(x, w, b, tokens, in_ch, out_ch, kernel, dilation, (uint32_t)t,
                       out + (size_t)t * out_ch);
}

/* cpu_conv_transpose1d (tokenizer_tests.cpp:3760-3784): out_tokens =
 * (tokens-1)*stride + kernel - 2*padding; acc = bias, then for in_c: for k:
 * numerator = out_t + padding - k; a tap counts when numerator >= 0, is a
 * multiple of stride and numerator/stride < tokens; weight [in][out][kernel]. */
void orc_conv_transpose1d(const float* x, const float* w, const float* b, uint32_t tokens,
                          uint32_t in_ch, uint32_t out_ch, uint32_t kernel, uint32_t stride,
                          uint32_t padding, float* out) {
    const uint32_t out_tokens = (tokens - 1) * stride + kernel - 2 * padding;
    long ot;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (ot = 0; ot < (long)out_tokens; ++ot) {
        float* row = out + (size_t)ot * out_ch;
        for (uint32_t oc = 0; oc < out_ch; ++oc) {
            float acc = b[oc];
            for (uint32_t ic = 0; ic < in_ch; ++ic) {
                for (uint32_t k = 0; k < kernel; ++k) {
                    const int num = (int)ot + (int)padding - (int)k;
                    if (num >= 0 && ((uint32_t)num % stride) == 0) {
                        const uint32_t in_t = (uint32_t)num / stride;
                        if (in_t < tokens)
                            acc += x[(size_t)in_t * in_ch + ic] *
                                   w[((size_t)ic * out_ch + oc) * kernel + k];
                    }
                }
            }
            row[oc] = acc;
        }
    }
}

/* clamped_channel_sample (tokenizer_tests.cpp:3787-3794). */
static float clamped_sample(const float* x, int t, uint32_t c, uint32_t tokens, uint32_t channels) {
    if (t < 0) t = 0;
    else if (t >= (int)tokens) t = (int)tokens - 1;
    return x[(size_t)t * channels + c];
}

/* bigvgan_upsample_value (tokenizer_tests.cpp:3796-3809): the 2x
 * anti-aliased upsampler at one upsampled position (12-tap filter, input
 * replicate-padded by 5, output cropped by 15), times the ratio 2. */
static float upsample_value(const float* x, const float* filter, uint32_t up_t, uint32_t c,
                            uint32_t tokens, uint32_t channels) {
    const uint32_t full_t = up_t + 15;
    float acc = 0.0f;
    for (uint32_t k = 0; k < 12; ++k) {
        if (full_t >= k && ((full_t - k) % 2) == 0) {
            const uint32_t padded_t = (full_t - k) / 2;
            const int src = (int)padded_t - 5;
            acc += clamped_sample(x, src, c, tokens, channels) * filter[k];
        }
    }
    return 2.0f * acc;
}

/* cpu_bigvgan_activation (tokenizer_tests.cpp:3811-3834): upsample 2x,
 * SnakeBeta y + sin(alpha*y)^2 / (beta + 1e-9) with alpha = exp(alpha_log),
 * beta = exp(beta_log), then the 12-tap low-pass downsample by 2 (upsampled
 * index 2t + k - 5 clamped to the upsampled range). */
void orc_bigvgan_activation(const float* x, const float* up_filter, const float* down_filter,
                            const float* alpha_log, const float* beta_log, uint32_t tokens,
                            uint32_t channels, float* out) {
    const uint32_t up_tokens = tokens * 2;
    long t;
#pragma omp parallel for schedule(static) num_threads(orc_get_threads())
    for (t = 0; t < (long)tokens; ++t) {
        for (uint32_t c = 0; c < channels; ++c) {
            const float alpha = expf(alpha_log[c]);
            const float beta = expf(beta_log[c]);
            float acc = 0.0f;
            for (uint32_t k = 0; k < 12; ++k) {
                int up_t = (int)(t * 2 + k) - 5;
                if (up_t < 0) up_t = 0;
                else if (up_t >= (int)up_tokens) up_t = (int)up_tokens - 1;
                const float y = upsample_value(x, up_filter, (uint32_t)up_t, c, tokens, channels);
                const float s = sinf(y * alpha);
                acc += (y + (s * s) / (beta + 1e-9f)) * down_filter[k];
            }
            out[(size_t)t * channels + c] = acc;
        }
    }
}
