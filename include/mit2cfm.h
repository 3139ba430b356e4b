/*
 * mit2cfm.h -- C ABI of the MI355X (gfx950) DiT-CFM mel decoder.
 *
 * Drop-in boundary for the acoustic-model hot path of IndexTTS2-Metal: the
 * CFG Euler solver over the DiT estimator (13 AdaRMSNorm blocks with U-ViT
 * skips, WaveNet tail, AdaLN final layer).  It replaces the reference's
 * Metal/MPS backend for this path, i.e. the mit2::MetalContext pass API
 * (runtime/include/mit2/metal_context.hpp:55-297) as driven by
 * run_cfm_euler_metal (runtime/impl/dit_cfm_bigvgan.cpp:3121).
 *
 * Conventions
 *  - Plain C types only.  Host buffers are caller-owned, token-major fp32
 *    ([tokens][channels] row-major), copied in; outputs are written into
 *    caller buffers.  Device memory is owned by the context.
 *  - Every call returns MIT2CFM_OK (0) or an error code; the message of the
 *    last failure is returned by mit2cfm_last_error.  No C++ exception
 *    crosses this boundary.
 *  - A context is bound to one GPU and is not thread-safe: use one context
 *    per thread (the reference's MetalContext has the same rule).  The
 *    timestep-conditioning tables are per context, so the reference's
 *    unlocked process-wide table cache has no counterpart here.
 *  - Tensor names are the reference bundle's names
 *    ("s2mel.net.cfm.estimator.*").
 */
#ifndef MIT2CFM_H
#define MIT2CFM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIT2CFM_ABI_VERSION 2

typedef struct mit2cfm_ctx mit2cfm_ctx;
typedef int32_t mit2cfm_status;

enum {
  MIT2CFM_OK = 0,
  MIT2CFM_E_ARG = 1,      /* invalid argument (shape, size, range)          */
  MIT2CFM_E_MODEL = 2,    /* missing / malformed tensor, bad bundle          */
  MIT2CFM_E_HIP = 3,      /* HIP runtime error or no HIP device              */
  MIT2CFM_E_INTERNAL = 4  /* anything else                                   */
};

enum { MIT2CFM_DTYPE_F32 = 0, MIT2CFM_DTYPE_F16 = 1 };

/* One named host tensor (element count, f32 or f16 payload). */
typedef struct {
  const char* name;
  const void* data;
  uint64_t elems;
  int32_t dtype;
} mit2cfm_tensor;

int32_t mit2cfm_abi_version(void);

/* Message of the last failed call on ctx (ctx may be NULL for calls that
 * failed before a context existed; that message is thread-local). */
const char* mit2cfm_last_error(const mit2cfm_ctx* ctx);

/* ---- context --------------------------------------------------------------
 * Replaces MetalContext construction (metal_context.mm:741-745) plus the lazy
 * resident-weight upload (resident_buffer_f16_from_f32, metal_context.mm:677-694):
 * all estimator weights are uploaded, weight-normed and laid out once here. */
mit2cfm_status mit2cfm_create(const mit2cfm_tensor* tensors, uint32_t count, int32_t device,
                              mit2cfm_ctx** out);
/* Same, reading an MIT2 bundle directory or single-file bundle with the
 * bundle loader (replaces mit2::Bundle, runtime/bundle.cpp). */
mit2cfm_status mit2cfm_create_from_bundle(const char* bundle_path, int32_t device,
                                          mit2cfm_ctx** out);
/* Same, with seeded synthetic weights: N(0, stddev) f16 from seed base_seed + i
 * for the i-th tensor in sorted-name order. */
mit2cfm_status mit2cfm_create_synthetic(uint64_t base_seed, float stddev, int32_t device,
                                        mit2cfm_ctx** out);
void mit2cfm_destroy(mit2cfm_ctx* ctx);

/* ---- decode ----------------------------------------------------------------
 * Full CFG Euler decode: replaces run_cfm_euler_metal
 * (dit_cfm_bigvgan.cpp:3121, via run_cfm_euler_metal_impl :2939 and
 * run_cfm_euler_metal_single_pass :2367); result semantics of
 * run_cfm_euler_cpu (:2908).  x0 [T][80], prompt [P][80], cond [T][512],
 * style [192]; x_out [T][80] receives the final mel (prompt rows zero).
 * cfg_rate > 0 batches the cond/null branches as B = 2; cfg_rate == 0 runs
 * the cond branch only. */
mit2cfm_status mit2cfm_decode(mit2cfm_ctx* ctx, const float* x0, const float* prompt,
                              const float* cond, const float* style, uint32_t tokens,
                              uint32_t prompt_tokens, uint32_t steps, float cfg_rate,
                              float* x_out);
/* The same decode on DEVICE pointers already resident in HBM (x0 [T][80],
 * prompt [P][80], cond [T][512], style [192], x_out [T][80]).  The work is
 * enqueued on the context's stream (mit2cfm_stream); with
 * MIT2CFM_FLAG_SYNC the call waits for it.  No reference counterpart: the
 * reference's unified memory needs no host/device split. */
#define MIT2CFM_FLAG_SYNC 1u
mit2cfm_status mit2cfm_decode_device(mit2cfm_ctx* ctx, const float* x0, const float* prompt,
                                     const float* cond, const float* style, uint32_t tokens,
                                     uint32_t prompt_tokens, uint32_t steps, float cfg_rate,
                                     float* x_out, uint32_t flags);
/* Decode that also returns every step's guided velocity
 * v = (1+cfg)*dphi - cfg*null_dphi in v_trace [steps][T][80]; for the
 * per-step parity check (the reference traces the same quantity in
 * trace_s2mel_cfm_golden, dit_cfm_bigvgan.cpp:3126-3304). */
mit2cfm_status mit2cfm_decode_trace(mit2cfm_ctx* ctx, const float* x0, const float* prompt,
                                    const float* cond, const float* style, uint32_t tokens,
                                    uint32_t prompt_tokens, uint32_t steps, float cfg_rate,
                                    float* x_out, float* v_trace);
/* nreq independent requests right-padded to t_max frames (batched serving):
 * x0, prompt, x_out [nreq][t_max][80], cond [nreq][t_max][512],
 * style [nreq][192], tokens[r] = valid frames, prompt_tokens[r].  Each
 * request's key mask is [t < tokens[r]]; the reference semantics of a masked
 * estimator (dit_cfm_bigvgan.cpp:1768 with mask) apply at the padded length.
 * The reference runs one request per call (server.cpp:477-535). */
mit2cfm_status mit2cfm_decode_batched(mit2cfm_ctx* ctx, uint32_t nreq, uint32_t t_max,
                                      const uint32_t* tokens, const uint32_t* prompt_tokens,
                                      const float* x0, const float* prompt, const float* cond,
                                      const float* style, uint32_t steps, float cfg_rate,
                                      float* x_out);

/* The same batched decode on DEVICE buffers already resident in HBM (x0,
 * prompt, cond, style, x_out as above); tokens and prompt_tokens stay host
 * arrays of nreq values.  Enqueued on the context's stream (flags as for
 * mit2cfm_decode_device).  No reference counterpart. */
mit2cfm_status mit2cfm_decode_batched_device(mit2cfm_ctx* ctx, uint32_t nreq, uint32_t t_max,
                                             const uint32_t* tokens, const uint32_t* prompt_tokens,
                                             const float* x0, const float* prompt, const float* cond,
                                             const float* style, uint32_t steps, float cfg_rate,
                                             float* x_out, uint32_t flags);

/* ---- one estimator forward ---------------------------------------------------
 * Replaces run_dit_estimator_step_metal (dit_cfm_bigvgan.cpp:2778); semantics
 * of run_dit_estimator_step_cpu (:1768) for each of `batch` independent
 * branches: x, prompt_x [B][T][80], cond [B][T][512], style [B][192],
 * key_mask [B][T] (0/1), t the flow time; dphi_out [B][T][80]. */
mit2cfm_status mit2cfm_estimator_step(mit2cfm_ctx* ctx, const float* x, const float* prompt_x,
                                      const float* cond, const float* style,
                                      const uint32_t* key_mask, float t, uint32_t batch,
                                      uint32_t tokens, float* dphi_out);

/* ---- stream control ----------------------------------------------------------- */
void* mit2cfm_stream(mit2cfm_ctx* ctx); /* the context's hipStream_t */
mit2cfm_status mit2cfm_synchronize(mit2cfm_ctx* ctx);
/* Whole-decode hipGraph replay on (1, default) or off (0).  Each decode
 * shape (request count, length, steps, cfg rate and the io pointers) is
 * captured once into a graph; at most *capacity (8) graphs are kept per
 * context, the least recently used destroyed first.
 * mit2cfm_decode_graph_count reports how many are held now.  No reference
 * counterpart (the reference records one command buffer per decode). */
mit2cfm_status mit2cfm_set_graph(mit2cfm_ctx* ctx, int32_t on);
mit2cfm_status mit2cfm_decode_graph_count(mit2cfm_ctx* ctx, uint32_t* count, uint32_t* capacity);

/* Padded rows of a ragged batched decode (mit2cfm_decode_batched[_device]
 * with some tokens[r] < t_max).  MIT2CFM_PADDING_COMPUTE (default): every
 * row is computed, the masked estimator at the padded length.
 * MIT2CFM_PADDING_SKIP: rows from two past each request's valid length on
 * are not computed (row tiles of every product and query blocks of the
 * attention stop there; the two rows after the valid ones are kept because
 * the WaveNet's k=5 conv at the last valid rows reads them).  Valid rows are
 * bit-identical in both modes; x_out's padded rows are unspecified with
 * SKIP.  Full-length batches, single decodes and batches of more than 16
 * branches (8 requests with CFG) compute every row in either mode.  No
 * reference counterpart (the reference decodes one request per call). */
#define MIT2CFM_PADDING_COMPUTE 0
#define MIT2CFM_PADDING_SKIP 1
mit2cfm_status mit2cfm_set_padding(mit2cfm_ctx* ctx, int32_t mode);
mit2cfm_status mit2cfm_get_padding(mit2cfm_ctx* ctx, int32_t* mode);

/* ---- arithmetic of the fp32 stages ---------------------------------------------
 * The reference runs the length regulator (run_length_regulator_full_metal,
 * runtime/impl/gpt.cpp:5313; its test bar max-abs 1e-4, :5382-5401) and the
 * BigVGAN vocoder (kernels.metal:1607-1749, dit_cfm_bigvgan.cpp:4102-4223;
 * bar max-abs 1e-3, :4469-4490) in fp32.  MIT2CFM_PREC_F32 (the default)
 * runs their GEMMs on split f16 operand pairs (hi = f16(v), lo = the
 * rounding remainder; three matrix-core products per term, two where the
 * weight is exact in f16), which gives fp32-level results;
 * MIT2CFM_PREC_F16 runs them on plain f16 operands
 * (faster, about 1e-3 relative).  The DiT-CFM decoder itself always uses f16
 * operands, as the reference's Metal decoder does.  A stage the context has
 * no tensors for is MIT2CFM_E_MODEL.  No reference counterpart. */
#define MIT2CFM_STAGE_LENGTH_REGULATOR 1
#define MIT2CFM_STAGE_VOCODER 2
#define MIT2CFM_PREC_F16 0
#define MIT2CFM_PREC_F32 1
mit2cfm_status mit2cfm_set_precision(mit2cfm_ctx* ctx, int32_t stage, int32_t mode);
mit2cfm_status mit2cfm_get_precision(mit2cfm_ctx* ctx, int32_t stage, int32_t* mode);

/* ---- measurement hook ------------------------------------------------------------
 * Enqueues `count` back-to-back launches of one decode kernel at the shape of
 * the context's last decode (operands: that decode's workspace), on the
 * context stream, without waiting, so a caller can bracket them with events
 * on mit2cfm_stream.  Reports the kernel's algorithmic flops and HBM bytes per
 * launch and its name.  Kernel ids: 0 FFN w1|w3 GEMM + SwiGLU, 1 WaveNet
 * k=5 conv GEMM + gate, 2 QKV GEMM + RoPE, 3 FFN w2 GEMM + residual,
 * 4 masked attention, 5 AdaRMSNorm, 6 attention output projection wo +
 * residual (folded-norm producer), 7 WaveNet res/skip GEMM.  No reference
 * counterpart (the reference times whole command buffers,
 * metal_context.mm:463-477). */
mit2cfm_status mit2cfm_profile_launch(mit2cfm_ctx* ctx, int32_t kernel, uint32_t count,
                                      double* flops_per_launch, double* bytes_per_launch,
                                      const char** name);

/* ---- stage entry points (parity harness; host pointers, synchronous) ---------
 * One per reference CPU stage, mirroring the reference's --test-dit-* harnesses
 * (main.cpp:2909-2989).  rows = batch * tokens; t1/t2 are 512-d embeddings. */
/* gpt.cpp:5404 run_timestep_embedder_cpu; which = 1 (t_embedder) or 2 (t_embedder2) */
mit2cfm_status mit2cfm_stage_timestep_embedder(mit2cfm_ctx* ctx, float t, int32_t which,
                                               float* out512);
/* dit_cfm_bigvgan.cpp:1 run_dit_input_merge_cpu (per branch b: style[b]) */
mit2cfm_status mit2cfm_stage_input_merge(mit2cfm_ctx* ctx, const float* x, const float* prompt_x,
                                         const float* cond, const float* style, uint32_t batch,
                                         uint32_t tokens, float* out);
/* :260 run_adaptive_norm_cpu; norm_id 0..12 attention_norm, 13..25 ffn_norm, 26 transformer.norm.
 * The output is the f16 GEMM operand, widened back to fp32. */
mit2cfm_status mit2cfm_stage_adaptive_norm(mit2cfm_ctx* ctx, const float* in, const float* t1,
                                           uint32_t rows, int32_t norm_id, float* out);
/* :469 run_dit_attention_core_cpu_masked_layer (wqkv, RoPE, masked attention, wo) */
mit2cfm_status mit2cfm_stage_attention_core(mit2cfm_ctx* ctx, const float* in,
                                            const uint32_t* key_mask, uint32_t batch,
                                            uint32_t tokens, int32_t layer, float* out);
/* :727 run_dit_feed_forward_cpu_layer (SwiGLU) */
mit2cfm_status mit2cfm_stage_feed_forward(mit2cfm_ctx* ctx, const float* in, uint32_t rows,
                                          int32_t layer, float* out);
/* :816 run_dit_transformer_block_cpu_layer; skip is NULL for layers 0..6 */
mit2cfm_status mit2cfm_stage_block(mit2cfm_ctx* ctx, const float* in, const float* t1,
                                   const uint32_t* key_mask, uint32_t batch, uint32_t tokens,
                                   int32_t layer, const float* skip, float* out);
/* :868 run_dit_transformer_stack_cpu (13 blocks + final AdaRMSNorm) */
mit2cfm_status mit2cfm_stage_stack(mit2cfm_ctx* ctx, const float* in, const float* t1,
                                   const uint32_t* key_mask, uint32_t batch, uint32_t tokens,
                                   float* out);
/* :1053 run_dit_post_transformer_proj_cpu (long_skip, conv1, res_projection) */
mit2cfm_status mit2cfm_stage_post(mit2cfm_ctx* ctx, const float* xres, const float* xmel,
                                  uint32_t rows, float* long_skip, float* conv1,
                                  float* res_proj);
/* :1464 run_wavenet_stack_global_cond_cpu */
mit2cfm_status mit2cfm_stage_wavenet(mit2cfm_ctx* ctx, const float* in, const float* t2,
                                     const uint32_t* key_mask, uint32_t batch, uint32_t tokens,
                                     float* out);
/* :1172 run_dit_final_layer_cpu */
mit2cfm_status mit2cfm_stage_final_layer(mit2cfm_ctx* ctx, const float* in, const float* t1,
                                         uint32_t rows, float* out);
/* The MFMA GEMM alone (replaces pass_linear_rows_mps, metal_context.mm:328-378):
 * out[M][N] = f16(A)[M][K] . f16(W)[N][K]^T + bias (bias may be NULL);
 * K % 128 == 0, N % 64 == 0. */
mit2cfm_status mit2cfm_op_linear(mit2cfm_ctx* ctx, const float* a, const float* w,
                                 const float* bias, uint32_t m, uint32_t n, uint32_t k,
                                 float* out);

/* ---- seeded synthetic data (tokenizer_tests.cpp:2121 make_deterministic_normal_noise) */
mit2cfm_status mit2cfm_normal_noise(uint32_t tokens, uint32_t channels, uint64_t seed,
                                    float temperature, float* out);
/* Estimator tensor inventory used by mit2cfm_create_synthetic (sorted names). */
uint32_t mit2cfm_synthetic_tensor_count(void);
/* name, ndim (<= 4), shape[4], dtype (MIT2CFM_DTYPE_*) and element count of tensor i. */
mit2cfm_status mit2cfm_synthetic_tensor_info(uint32_t i, const char** name, uint32_t* ndim,
                                             int64_t* shape4, int32_t* dtype, uint64_t* elems);
/* Payload of tensor i (elems * 2 bytes for f16, * 4 for f32) into out. */
mit2cfm_status mit2cfm_synthetic_tensor_fill(uint32_t i, uint64_t base_seed, float stddev,
                                             void* out);
/* ---- device weight image ------------------------------------------------
 * The offline weight preparation the reference's design notes call for
 * (docs/model.md:93: weight norm folded into the bundle, conv taps
 * transposed once; the reference does both at every upload,
 * metal_context.mm:5056-5075, gpt.cpp:5109-5130): mit2cfm_write_image saves
 * a context's prepared device weights (weight norm folded, products folded,
 * rows permuted, taps laid out, f16) with their layout; mit2cfm_create_from_image
 * creates a context by copying them to the device, with no host-side
 * preparation.  The image is specific to this library's ABI version; a
 * malformed, truncated or foreign file is MIT2CFM_E_MODEL. */
mit2cfm_status mit2cfm_write_image(mit2cfm_ctx* ctx, const char* path);
mit2cfm_status mit2cfm_create_from_image(const char* path, int32_t device, mit2cfm_ctx** out);

/* Synthetic tensor sets beyond the estimator (the functions above are set 0):
 * MIT2CFM_SYNTH_LENGTH_REGULATOR, the s2mel length regulator's 20 tensors
 * (N(0, stddev) f16 from base_seed + index, GroupNorm weights 1 + N(0, stddev));
 * MIT2CFM_SYNTH_BIGVGAN, the vocoder's 783 tensors (weight_v and biases
 * N(0, stddev) f16; weight_g = g (1 + N(0, stddev)) with g = 1 for conv_pre
 * and the upsamplers, 0.1 for conv_post, 0.6 for the resblock convs; the
 * 12-tap Kaiser-sinc filters and SnakeBeta's log alpha / log beta N(0, 0.1)
 * in f32); MIT2CFM_SYNTH_GPT, the GPT decoder's 296 tensors (24 layers,
 * ln_f, final_norm, mel_head, the mel and mel-position embeddings; Conv1D
 * weights [in][out]; N(0, stddev) f16, LayerNorm weights 1 + N(0, stddev)).
 * Tensors are sorted by name.  No reference counterpart: the reference's
 * tests use its real weights; these give every run the same random-init
 * model. */
#define MIT2CFM_SYNTH_ESTIMATOR 0
#define MIT2CFM_SYNTH_LENGTH_REGULATOR 1
#define MIT2CFM_SYNTH_BIGVGAN 2
#define MIT2CFM_SYNTH_GPT 3
uint32_t mit2cfm_synthetic_set_count(int32_t set);
mit2cfm_status mit2cfm_synthetic_set_info(int32_t set, uint32_t i, const char** name, uint32_t* ndim,
                                          int64_t* shape4, int32_t* dtype, uint64_t* elems);
mit2cfm_status mit2cfm_synthetic_set_fill(int32_t set, uint32_t i, uint64_t base_seed, float stddev,
                                          void* out);
/* A context with every synthetic set: estimator (base_seed), length
 * regulator (base_seed + 1), vocoder (base_seed + 2). */
mit2cfm_status mit2cfm_create_synthetic_acoustic(uint64_t base_seed, float stddev, int32_t device,
                                                 mit2cfm_ctx** out);
/* Opens a bundle with the loader and applies every validation rule of the
 * format (replaces the --inspect-model-bundle gate, main.cpp; rules in
 * docs/native_bundle.md "Validation Rules"); verify_sha256 != 0 also checks
 * each payload's SHA-256.  Needs no GPU. */
mit2cfm_status mit2cfm_inspect_bundle(const char* bundle_path, uint64_t* tensor_count,
                                      uint64_t* payload_bytes, uint32_t verify_sha256);
/* Writes the synthetic estimator weights as an MIT2 bundle directory. */
mit2cfm_status mit2cfm_write_synthetic_bundle(const char* dir, uint64_t base_seed, float stddev);

/* ---- condition and noise producer (the step before the decode) -----------
 * These need the s2mel length regulator's tensors
 * ("s2mel.net.length_regulator.*", 20 tensors) in the context's weight table;
 * without them they return MIT2CFM_E_MODEL. */

/* Replaces run_length_regulator_full_metal (runtime/impl/gpt.cpp:5313; CPU
 * definition run_length_regulator_full_cpu :5298): s_infer [in_tokens][1024]
 * (the GPT semantic latent plus its VQ embedding) -> out [out_tokens][512]:
 * content_in_proj, nearest interpolation to out_tokens, 4 x (conv k=3 zero
 * padded, GroupNorm with one group, Mish), conv k=1.  Host pointers,
 * synchronous. */
mit2cfm_status mit2cfm_length_regulator(mit2cfm_ctx* ctx, const float* s_infer,
                                        uint32_t in_tokens, uint32_t out_tokens, float* out);
/* The decode condition: replaces the length-regulator and
 * hot_condition_merge_f32 steps of build_hot_codes_condition_inputs_shared
 * (runtime/impl/tts_synthesis/synthesis_pipeline.cpp:1012-1035; merge kernel
 * kernels.metal:843-864).  generated = floor(codes * 1.72f) frames;
 * cond_out [prompt_tokens + generated][512] = the first prompt_tokens rows of
 * prompt_cond followed by the length regulator of s_infer [codes][1024].
 * *generated_out receives generated.  Host pointers, synchronous. */
mit2cfm_status mit2cfm_condition(mit2cfm_ctx* ctx, const float* s_infer, uint32_t codes,
                                 const float* prompt_cond, uint32_t prompt_tokens,
                                 float* cond_out, uint32_t* generated_out);
/* The same on DEVICE pointers, enqueued on the context's stream (flags as for
 * mit2cfm_decode_device), so cond_out can feed mit2cfm_decode_device without
 * a host round trip.  No reference counterpart (unified memory there). */
mit2cfm_status mit2cfm_condition_device(mit2cfm_ctx* ctx, const float* s_infer, uint32_t codes,
                                        const float* prompt_cond, uint32_t prompt_tokens,
                                        float* cond_out, uint32_t* generated_out, uint32_t flags);
/* mit2cfm_condition_device that allocates nothing: no reference counterpart.
 * It is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Its
 * scratch (the length regulator's operand, conv and statistics buffers) is
 * a static device array of about 13.7 MB that every GPU the library runs on
 * holds until the process ends, shared by every context on that GPU.  Calls
 * on one GPU are run one after another: each call's stream waits for an
 * event the previous call recorded after its last kernel (contexts on other
 * streams or threads included).  A call enqueued while its stream is being
 * captured into a graph is not ordered that way (a capture may not wait on
 * work outside it), so replays of such a graph must not overlap other calls
 * on that GPU: they would race on the scratch.  codes above
 * MIT2CFM_NOALLOC_MAX_CODES (1,761 generated frames) is MIT2CFM_E_ARG.
 * Arguments, outputs, flags and results as for mit2cfm_condition_device. */
#define MIT2CFM_NOALLOC_MAX_CODES 1024u
mit2cfm_status mit2cfm_condition_device_noalloc(mit2cfm_ctx* ctx, const float* s_infer, uint32_t codes,
                                                const float* prompt_cond, uint32_t prompt_tokens,
                                                float* cond_out, uint32_t* generated_out, uint32_t flags);
/* Frames the condition producer makes from `codes` semantic tokens:
 * floor(codes * 1.72f) (synthesis_pipeline.cpp:1012). */
uint32_t mit2cfm_generated_frames(uint32_t codes);
/* Seeded decode noise on the GPU: make_deterministic_normal_noise
 * (runtime/impl/tokenizer_tests.cpp:2121) into the DEVICE buffer out
 * [tokens][channels]; the uniforms are bit-identical to the host generator,
 * the Box-Muller transcendentals are the GPU's.  Enqueued on the context's
 * stream (flags as for mit2cfm_decode_device). */
mit2cfm_status mit2cfm_noise_device(mit2cfm_ctx* ctx, uint32_t tokens, uint32_t channels,
                                    uint64_t seed, float temperature, float* out, uint32_t flags);

/* ---- BigVGAN vocoder (the consumer of the mel) ----------------------------
 * These need the vocoder's 783 "bigvgan.*" tensors (weight-normed convs as
 * weight_g / weight_v / bias, the activations' filters and SnakeBeta
 * alpha / beta) in the context's weight table; without them they return
 * MIT2CFM_E_MODEL. */

/* Replaces run_bigvgan_vocoder_metal (runtime/impl/dit_cfm_bigvgan.cpp:4196;
 * CPU definition run_bigvgan_vocoder_cpu :4058): mel [tokens][80] ->
 * wav [256 * tokens], clamped to [-1, 1].  Host pointers, synchronous. */
mit2cfm_status mit2cfm_bigvgan(mit2cfm_ctx* ctx, const float* mel, uint32_t tokens, float* wav);
/* The same on DEVICE pointers, enqueued on the context's stream (flags as for
 * mit2cfm_decode_device), so the decode's mel can feed it directly. */
mit2cfm_status mit2cfm_bigvgan_device(mit2cfm_ctx* ctx, const float* mel, uint32_t tokens, float* wav,
                                      uint32_t flags);
/* One vocoder stage on host pointers, as the reference's stage tests run them
 * (dit_cfm_bigvgan.cpp:3627-4469):
 *   stage 0 conv_pre (run_bigvgan_conv_pre, :3606)      [T][80]   -> [T][1536]
 *   stage 1 upsampler `index` 0..5 (:3690)              [T][Cin]  -> [s T][Cout]
 *   stage 2 activation `index` = 6 j + a for resblock j's activation a, 108
 *           for activation_post (:3810)                 [T][C]    -> [T][C]
 *   stage 3 resblock `index` 0..17 (:3939)              [T][C]    -> [T][C]
 *   stage 4 resblock group `index` 0..5 (:3982)         [T][C]    -> [T][C]
 *   stage 5 post: activation_post, conv_post, clamp (:4030) [T][24] -> [T]
 *   stage 6 body: conv_pre, 6 x (upsampler, group) (:4008) [T][80] -> [256 T][24]
 * out_capacity is the size of out in floats. */
mit2cfm_status mit2cfm_bigvgan_stage(mit2cfm_ctx* ctx, int32_t stage, int32_t index, const float* in,
                                     uint32_t tokens, float* out, uint64_t out_capacity);
/* Floats of a stage's input (output = 0) or output (output = 1) for `tokens`
 * input rows; 0 for an unknown stage or index. */
uint64_t mit2cfm_bigvgan_stage_floats(int32_t stage, int32_t index, uint32_t tokens, int32_t output);

/* ---- the whole acoustic stage ----------------------------------------------
 * Replaces the acoustic half of the reference's hot synthesis path on the
 * GPU, with no host round trip: the length regulator and prompt merge of
 * build_hot_codes_condition_inputs_shared (runtime/impl/tts_synthesis/
 * synthesis_pipeline.cpp:1012-1035), the seeded noise
 * make_deterministic_normal_noise(T, 80, seed, temperature) (:1333), and
 * synthesize_hot_condition_vectors_wav_shared (:1038-1097: the CFG decode,
 * the generated rows sliced off, the vocoder) without the WAV file write.
 * DEVICE pointers: s_infer [codes][1024]; prompt_cond [>= P][512] (the
 * voice's s2mel_prompt); prompt_mel [P][80] token-major (the voice's mel
 * transposed); style [192]; wav_out [256 * generated], generated =
 * floor(codes * 1.72f); mel_out (optional) [P + generated][80].  Needs the
 * estimator, length-regulator and vocoder tensors.  Enqueued on the context's
 * stream (flags as for mit2cfm_decode_device). */
mit2cfm_status mit2cfm_acoustic_device(mit2cfm_ctx* ctx, const float* s_infer, uint32_t codes,
                                       const float* prompt_cond, const float* prompt_mel,
                                       uint32_t prompt_tokens, const float* style, uint64_t noise_seed,
                                       float noise_temperature, uint32_t steps, float cfg_rate,
                                       float* wav_out, float* mel_out, uint32_t* generated_out,
                                       uint32_t flags);

/* ---- GPT mel-code decoder (the producer of the semantic codes) -------------
 * These need the GPT decoder's tensors in the context's weight table:
 * "gpt.gpt.h.<l>.{ln_1,attn.c_attn,attn.c_proj,ln_2,mlp.c_fc,mlp.c_proj}.*"
 * for l = 0..L-1 (the checkpoint has L = 24; Conv1D weights [in][out]),
 * "gpt.gpt.ln_f.*", "gpt.final_norm.*", "gpt.mel_head.*",
 * "gpt.mel_embedding.weight" [8194][1280] and
 * "gpt.mel_pos_embedding.emb.weight" [1818][1280]; without them they return
 * MIT2CFM_E_MODEL.  Weights are f16 on the device (the checkpoint's own
 * precision), activations and the key/value caches fp32. */

/* Layers of the context's GPT decoder (0 when it has none). */
mit2cfm_status mit2cfm_gpt_layers(mit2cfm_ctx* ctx, uint32_t* layers);

/* Replaces run_gpt_kv_greedy_metal (runtime/impl/gpt.cpp:1914; CPU
 * definition run_gpt_kv_greedy_cpu :1877): prefill the key/value caches
 * from prefix [prefix_tokens][1280] (the conditioning + text embeddings),
 * then greedy-decode up to `steps` mel codes from the start token 8192,
 * stopping at the first stop token 8193.  Positions follow
 * gpt_cached_generate_position (:1873): step s uses position s, or s + 1 for
 * s > 0 when hf_generate_positions is nonzero; a `steps` whose last position
 * passes the 1818-row table is MIT2CFM_E_ARG (the reference throws when it
 * gets there).  Outputs (host): predicted_tokens [steps] and *n_predicted
 * (the stop token included), input_tokens [steps + 1] and *n_input (the start
 * token, then every non-stop prediction), *first_stop_step (-1: none),
 * last_logits [8194] (the last step's logits; may be NULL), timings_ms [2]
 * (device time of the prefill and of the decode loop; may be NULL).  Host
 * pointers, synchronous. */
mit2cfm_status mit2cfm_gpt_kv_greedy(mit2cfm_ctx* ctx, const float* prefix, uint32_t prefix_tokens,
                                     uint32_t steps, int32_t hf_generate_positions,
                                     uint32_t* predicted_tokens, uint32_t* n_predicted,
                                     uint32_t* input_tokens, uint32_t* n_input, int32_t* first_stop_step,
                                     float* last_logits, double* timings_ms);

/* GptSamplingConfig (runtime/impl/gpt.cpp:1592-1599) with do_sample set. */
typedef struct mit2cfm_gpt_sampling {
  uint64_t seed;            /* splitmix64 seed, once per call */
  float temperature;        /* > 0 */
  uint32_t top_k;           /* 0: off */
  float top_p;              /* (0, 1]; 1: off */
  float repetition_penalty; /* > 0; 1: off */
} mit2cfm_gpt_sampling;

/* The sampled form of mit2cfm_gpt_kv_greedy (run_gpt_kv_greedy_metal with
 * do_sample, gpt.cpp:2221-2240): each step's logits go through
 * apply_gpt_sampling_processors (:1618: repetition penalty over the distinct
 * history tokens, temperature, top-k, top-p) and sample_gpt_token_from_logits
 * (:1720: one splitmix64 draw) on the GPU.  The history is the reference's
 * repetition_history_prefix (:1918, :2224-2229) followed by the predictions
 * so far: history_prefix [history_prefix_count] (host, at most 8192 tokens;
 * the synthesis path passes the prefix's fake_inputs, [1] x n + [8192],
 * synthesis_pipeline.cpp:795-802), or with history_prefix NULL and the count
 * 0 the start token alone.  A non-NULL history_prefix with count 0 is an
 * empty prefix, as the reference's empty vector is: the history is then the
 * predictions alone.  Outputs as for mit2cfm_gpt_kv_greedy, plus
 * last_processed_logits [8194] (may be NULL).  A setting the reference
 * rejects (temperature or penalty <= 0, top_p outside (0, 1]) is
 * MIT2CFM_E_ARG. */
mit2cfm_status mit2cfm_gpt_kv_sample(mit2cfm_ctx* ctx, const float* prefix, uint32_t prefix_tokens,
                                     uint32_t steps, int32_t hf_generate_positions,
                                     const mit2cfm_gpt_sampling* sampling, const uint32_t* history_prefix,
                                     uint32_t history_prefix_count, uint32_t* predicted_tokens,
                                     uint32_t* n_predicted, uint32_t* input_tokens, uint32_t* n_input,
                                     int32_t* first_stop_step, float* last_logits,
                                     float* last_processed_logits, double* timings_ms);

/* Replaces run_gpt_cached_decode_metal (runtime/impl/gpt.cpp:1427; CPU
 * definition run_gpt_cached_decode_cpu :1400): rows [prefix_tokens + 1][1280];
 * the first prefix_tokens rows fill the key/value caches, the last row is
 * decoded against them.  Outputs (host, each may be NULL): ln_f [1280],
 * final_norm [1280], logits [8194], *argmax.  Synchronous. */
mit2cfm_status mit2cfm_gpt_cached_decode(mit2cfm_ctx* ctx, const float* rows, uint32_t prefix_tokens,
                                         float* ln_f, float* final_norm, float* logits, uint32_t* argmax);

/* Measurement hook of the GPT decode step: enqueues `count` launches of one of
 * its kernels (cycling the layers' weights) on the context's stream without
 * waiting, for timing with events on mit2cfm_stream; count 0 launches
 * nothing.  With graph replay on, the launches are captured into a graph the
 * first time a (kernel, count) pair is asked for and replayed after that, so
 * a second call times the kernels back to back, without the host's launch
 * rate between them.
 * Kernel ids: 0 c_attn GEMV (3840 x 1280, LayerNorm prologue, K/V written to
 * the cache), 1 attention c_proj GEMV (1280 x 1280, + residual), 2 c_fc GEMV
 * (5120 x 1280, LayerNorm prologue, gelu_new), 3 MLP c_proj GEMV
 * (1280 x 5120, + residual), 4 mel_head GEMV (8194 x 1280, ln_f and
 * final_norm prologue, argmax), 5 cached attention over 1024 keys.  Reports
 * the kernel's algorithmic HBM bytes per launch and its name.  No reference
 * counterpart. */
mit2cfm_status mit2cfm_gpt_profile_launch(mit2cfm_ctx* ctx, int32_t kernel, uint32_t count,
                                          double* bytes_per_launch, const char** name);

#ifdef __cplusplus
}
#endif
#endif /* MIT2CFM_H */
