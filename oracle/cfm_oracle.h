/*
 * cfm_oracle.h -- CPU restatement of the IndexTTS2 DiT-CFM mel decoder's fp32
 * reference path (the "oracle").
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only to compare
 * results with or as the timed CPU baseline.  The product library never links or calls it.
 *
 * Every function restates one reference function (file:line given beside it,
 * paths relative to the reference repository root) with the same loop order
 * and scalar fp32 accumulation.  Weights are handed over already widened to
 * fp32, as tensor_as_f32 (runtime/impl/tokenizer_tests.cpp:4311) does.
 *
 * Multi-threading (orc_set_threads) only splits independent output elements
 * (tokens, heads, queries) across threads; each element is still accumulated
 * by one thread in the reference's order, so results are bit-identical for
 * every thread count.
 */
#ifndef CFM_ORACLE_H
#define CFM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- threading ---------------------------------------------------------- */
void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- primitives (tokenizer_tests.cpp / gpt.cpp) -------------------------- */
float orc_half_to_float(uint16_t h);                              /* tokenizer_tests.cpp:4284 */
void orc_halves_to_floats(const uint16_t* h, size_t n, float* out);
uint64_t orc_splitmix64_next(uint64_t* state);                    /* tokenizer_tests.cpp:2102 */
float orc_uniform_open01(uint64_t* state);                        /* tokenizer_tests.cpp:2109 */
void orc_normal_noise(uint32_t tokens, uint32_t channels, uint64_t seed,
                      float temperature, float* out);              /* tokenizer_tests.cpp:2121 */
void orc_layernorm(const float* x, const float* gamma, const float* beta,
                   uint32_t n, float eps, float* out);              /* tokenizer_tests.cpp:2992 */
void orc_rmsnorm(const float* x, const float* gamma, uint32_t n, float eps,
                 float* out);                                      /* tokenizer_tests.cpp:3012 */
void orc_linear(const float* w, const float* b, const float* x, uint32_t rows,
                uint32_t cols, float* out);                        /* tokenizer_tests.cpp:3026 */
/* cpu_linear applied to `tokens` consecutive input rows (thread-parallel over rows). */
void orc_linear_rows(const float* w, const float* b, const float* x, uint32_t tokens,
                     uint32_t rows, uint32_t cols, float* out);
void orc_conv1d_same(const float* x, const float* w, const float* b, uint32_t tokens,
                     uint32_t in_ch, uint32_t out_ch, uint32_t kernel,
                     float* out);                                  /* tokenizer_tests.cpp:3142 */
void orc_reflect_pad(const float* x, uint32_t tokens, uint32_t channels,
                     uint32_t pad_left, uint32_t pad_right, float* out); /* tokenizer_tests.cpp:3836 */
void orc_conv1d_reflect_same(const float* x, const float* w, const float* b,
                             uint32_t tokens, uint32_t in_ch, uint32_t out_ch,
                             uint32_t kernel, float* out);         /* tokenizer_tests.cpp:3866 */
/* ---- BigVGAN vocoder primitives (bigvgan_oracle.c) ----------------------- */
void orc_conv1d_dilated_same(const float* x, const float* w, const float* b, uint32_t tokens,
                             uint32_t in_ch, uint32_t out_ch, uint32_t kernel, uint32_t dilation,
                             float* out);                          /* tokenizer_tests.cpp:3739 */
void orc_conv_transpose1d(const float* x, const float* w, const float* b, uint32_t tokens,
                          uint32_t in_ch, uint32_t out_ch, uint32_t kernel, uint32_t stride,
                          uint32_t padding, float* out);           /* tokenizer_tests.cpp:3760 */
void orc_bigvgan_activation(const float* x, const float* up_filter, const float* down_filter,
                            const float* alpha_log, const float* beta_log, uint32_t tokens,
                            uint32_t channels, float* out);        /* tokenizer_tests.cpp:3811 */
/* ---- condition producer: the s2mel length regulator (gpt.cpp:5271-5340) -- */
void orc_nearest_interpolate(const float* x, uint32_t in_tokens, uint32_t out_tokens,
                             uint32_t width, float* out);          /* tokenizer_tests.cpp:3127 */
void orc_groupnorm1(const float* x, const float* gamma, const float* beta, uint32_t tokens,
                    uint32_t channels, float eps, float* out);     /* tokenizer_tests.cpp:3874 */
void orc_mish(const float* x, size_t n, float* out);               /* tokenizer_tests.cpp:3898 */
/* run_length_regulator_full_cpu (gpt.cpp:5298): input [in_tokens, 1024] ->
 * out [out_tokens, 512].  proj_w [512, 1024]; conv_w[b] [512, 512, 3] (PyTorch
 * [out, in, k]); gn_w[b], gn_b[b], conv_b[b] [512]; out_w [512, 512] (k = 1). */
void orc_length_regulator(const float* input, uint32_t in_tokens, uint32_t out_tokens,
                          const float* proj_w, const float* proj_b,
                          const float* const* conv_w, const float* const* conv_b,
                          const float* const* gn_w, const float* const* gn_b,
                          const float* out_w, const float* out_b, float* out);
/* The same with f64_stats != 0 computing each GroupNorm's mean and variance in
 * double (orc_groupnorm1_f64stats): a checker, not the reference's arithmetic. */
void orc_length_regulator_ex(const float* input, uint32_t in_tokens, uint32_t out_tokens,
                             const float* proj_w, const float* proj_b,
                             const float* const* conv_w, const float* const* conv_b,
                             const float* const* gn_w, const float* const* gn_b,
                             const float* out_w, const float* out_b, int f64_stats, float* out);
void orc_groupnorm1_f64stats(const float* x, const float* gamma, const float* beta, uint32_t tokens,
                             uint32_t channels, float eps, float* out);
void orc_timestep_embedding(const float* t, uint32_t n_t, const float* freqs,
                            uint32_t half, float scale, float* out); /* tokenizer_tests.cpp:3947 */
void orc_attention_head_masked(const float* q, const float* k, const float* v,
                               const uint32_t* key_mask, uint32_t tokens,
                               uint32_t head_dim, float* out);     /* tokenizer_tests.cpp:3960 */
void orc_rope_inplace(float* x, uint32_t tokens, uint32_t heads,
                      uint32_t head_dim);                          /* tokenizer_tests.cpp:4266 */
void orc_weight_norm_rowmajor(const float* g, const float* v, uint32_t rows,
                              uint32_t cols, float* out);          /* gpt.cpp:5109 */

/* ---- model weights -------------------------------------------------------- */
typedef struct orc_model orc_model;
orc_model* orc_model_new(void);
void orc_model_free(orc_model* m);
/* Copies `count` floats under `name` (full tensor name, prefix included).
 * Returns 0, or -1 for an unknown name / wrong element count. */
int orc_model_set(orc_model* m, const char* name, const float* data, uint64_t count);
/* Number of estimator tensors the oracle needs, and the i-th name / count. */
int orc_model_tensor_count(void);
const char* orc_model_tensor_name(int i);
uint64_t orc_model_tensor_elems(int i);
/* Returns the number of required tensors still missing (0 = complete). */
int orc_model_missing(const orc_model* m);
const char* orc_last_error(void);

/* ---- estimator stages (dit_cfm_bigvgan.cpp / gpt.cpp) ----------------------
 * All activations are token-major row-major fp32.  mask is uint32 0/1 per token.
 * which = 1 -> t_embedder, 2 -> t_embedder2. */
void orc_timestep_embedder(const orc_model* m, float t, int which, float* out512); /* gpt.cpp:5404 */
void orc_input_merge(const orc_model* m, const float* x, const float* prompt_x,
                     const float* cond, const float* style, uint32_t T,
                     float* out);                                  /* dit_cfm_bigvgan.cpp:1 */
/* norm_id: 0..12 = layers.{l}.attention_norm, 13..25 = layers.{l-13}.ffn_norm, 26 = transformer.norm */
void orc_adaptive_norm(const orc_model* m, const float* in, const float* cond512,
                       uint32_t T, int norm_id, float* out);       /* dit_cfm_bigvgan.cpp:260 */
void orc_attention_core(const orc_model* m, const float* in, const uint32_t* mask,
                        uint32_t T, uint32_t layer, float* out);   /* dit_cfm_bigvgan.cpp:469 */
void orc_feed_forward(const orc_model* m, const float* in, uint32_t T, uint32_t layer,
                      float* out);                                 /* dit_cfm_bigvgan.cpp:727 */
void orc_skip_in(const orc_model* m, const float* in, const float* skip, uint32_t T,
                 uint32_t layer, float* out);                      /* dit_cfm_bigvgan.cpp:785 */
void orc_transformer_block(const orc_model* m, const float* in, const float* t1,
                           const uint32_t* mask, uint32_t T, uint32_t layer,
                           const float* skip, float* out);         /* dit_cfm_bigvgan.cpp:816 */
void orc_transformer_stack(const orc_model* m, const float* in, const float* t1,
                           const uint32_t* mask, uint32_t T, float* out); /* dit_cfm_bigvgan.cpp:868 */
void orc_post_transformer(const orc_model* m, const float* xres, const float* xmel,
                          uint32_t T, float* long_skip, float* conv1,
                          float* res_proj);                        /* dit_cfm_bigvgan.cpp:1053 */
void orc_wavenet(const orc_model* m, const float* in, const float* t2,
                 const uint32_t* mask, uint32_t T, float* out);    /* dit_cfm_bigvgan.cpp:1464 */
void orc_final_layer(const orc_model* m, const float* in, const float* t1, uint32_t T,
                     float* out);                                  /* dit_cfm_bigvgan.cpp:1172 */
void orc_estimator_step(const orc_model* m, const float* x, const float* prompt_x,
                        const float* cond, const float* style, float t,
                        const uint32_t* mask, uint32_t T, float* out); /* dit_cfm_bigvgan.cpp:1768 */
/* x is updated in place ([T,80]); prompt is [P,80]. */
void orc_cfm_euler(const orc_model* m, float* x, const float* prompt, const float* cond,
                   const float* style, uint32_t T, uint32_t P, uint32_t steps,
                   float cfg_rate);                                /* dit_cfm_bigvgan.cpp:2908 */
/* Same decode, additionally storing every step's guided velocity
 * v = (1+cfg)*dphi - cfg*null_dphi into v_trace ([steps, T, 80]) and the
 * state before each step into x_trace ([steps, T, 80]); either may be NULL. */
void orc_cfm_euler_trace(const orc_model* m, float* x, const float* prompt,
                         const float* cond, const float* style, uint32_t T, uint32_t P,
                         uint32_t steps, float cfg_rate, float* x_trace, float* v_trace);
/* The first run_steps Euler steps of the steps-step schedule (dt = 1/steps),
 * traced as orc_cfm_euler_trace ([run_steps, T, 80] each, either may be NULL);
 * x holds the state after them. */
void orc_cfm_euler_partial(const orc_model* m, float* x, const float* prompt,
                           const float* cond, const float* style, uint32_t T, uint32_t P,
                           uint32_t steps, uint32_t run_steps, float cfg_rate, float* x_trace,
                           float* v_trace);
/* The decode of one right-padded request: key_mask [T] (0/1) is passed to
 * both estimator calls of every step (the reference passes all ones). */
void orc_cfm_euler_masked(const orc_model* m, float* x, const float* prompt, const float* cond,
                          const float* style, const uint32_t* key_mask, uint32_t T, uint32_t P,
                          uint32_t steps, float cfg_rate);

/* ---- GPT mel-code decoder (gpt_oracle.c; runtime/impl/gpt.cpp) ----------- */
typedef struct orc_gpt orc_gpt;
orc_gpt* orc_gpt_new(int layers);
void orc_gpt_free(orc_gpt* m);
int orc_gpt_set(orc_gpt* m, const char* name, const float* data, uint64_t count);
int orc_gpt_missing(const orc_gpt* m);
const char* orc_gpt_last_error(void);
void orc_gelu_new(const float* x, size_t n, float* out);          /* tokenizer_tests.cpp:3931 */
void orc_attention_single_query(const float* q, const float* k, const float* v,
                                uint32_t key_tokens, uint32_t head_dim,
                                float* out);                       /* tokenizer_tests.cpp:4034 */
void orc_attention_causal(const float* q, const float* k, const float* v, uint32_t tokens,
                          uint32_t head_dim, float* out);           /* tokenizer_tests.cpp:4003 */
void orc_gpt_layer_qkv(const orc_gpt* m, const float* in, uint32_t tokens, uint32_t layer,
                       float* qkv);                                 /* gpt.cpp:1060 */
void orc_gpt_block(const orc_gpt* m, const float* in, uint32_t tokens, uint32_t layer,
                   float* out);                                     /* gpt.cpp:658 */
void orc_gpt_cached_block_current(const orc_gpt* m, const float* cache_k, const float* cache_v,
                                  uint32_t cache_tokens, const float* current,
                                  const float* current_qkv, uint32_t layer,
                                  float* out);                      /* gpt.cpp:1180 */
uint32_t orc_gpt_logits(const orc_gpt* m, const float* in, uint32_t tokens, float* final_norm,
                        float* logits);                             /* gpt.cpp:1310 */
uint32_t orc_gpt_cached_decode(const orc_gpt* m, const float* input, uint32_t prefix_tokens,
                               float* ln_f, float* final_norm, float* logits); /* gpt.cpp:1400 */
typedef struct {
    uint32_t n_predicted, n_input;
    int32_t first_stop_step;
} orc_gpt_greedy_result;
int orc_gpt_kv_greedy(const orc_gpt* m, const float* prefix, uint32_t prefix_tokens, uint32_t steps,
                      int hf_generate_positions, uint32_t* predicted, uint32_t* input_tokens,
                      float* last_logits, orc_gpt_greedy_result* res); /* gpt.cpp:1877 */
int orc_gpt_greedy_full(const orc_gpt* m, const float* prefix, uint32_t prefix_tokens,
                        uint32_t steps, uint32_t* predicted, uint32_t* input_tokens,
                        float* last_logits, orc_gpt_greedy_result* res); /* gpt.cpp:1833 */
int orc_gpt_sampling_processors(const float* logits, uint32_t n, const uint32_t* history,
                                uint32_t n_history, float temperature, uint32_t top_k, float top_p,
                                float repetition_penalty, float* scores); /* gpt.cpp:1618 */
uint32_t orc_gpt_sample_token(const float* processed, uint32_t n, uint64_t* rng_state); /* gpt.cpp:1720 */
int orc_gpt_kv_sample(const orc_gpt* m, const float* prefix, uint32_t prefix_tokens, uint32_t steps,
                      int hf_generate_positions, uint64_t seed, float temperature, uint32_t top_k,
                      float top_p, float repetition_penalty, const uint32_t* history_prefix,
                      uint32_t n_history_prefix, uint32_t* predicted,
                      uint32_t* input_tokens, float* last_logits, float* last_processed,
                      orc_gpt_greedy_result* res);                   /* gpt.cpp:2221-2240 */

#ifdef __cplusplus
}
#endif
#endif
