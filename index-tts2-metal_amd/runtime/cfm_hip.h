// cfm_hip.h -- C++ shim with the reference's call signatures over the C ABI.
//
// run_cfm_euler_hip / run_dit_estimator_step_hip take the arguments of
// run_cfm_euler_metal (runtime/impl/dit_cfm_bigvgan.cpp:3121) and
// run_dit_estimator_step_metal (:2778), with HipContext in place of
// mit2::MetalContext; failures throw std::runtime_error as the reference's
// Metal path does.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/mit2cfm.h"
#include "bundle.h"

namespace mit2 {

class HipContext {
 public:
  // Uploads the estimator tensors of `bundle` (and the length regulator's,
  // when the bundle holds them) to GPU `device`.
  explicit HipContext(const Bundle& bundle, int device = 0);
  // Seeded synthetic weights (N(0, stddev) f16; stddev 0 = fan-in scaled);
  // with acoustic, also the length regulator's and the vocoder's; with gpt,
  // also the 24-layer GPT decoder's (seed + 3).
  HipContext(uint64_t synthetic_seed, float stddev, int device = 0, bool acoustic = false, bool gpt = false);
  // From a device image (mit2cfm_write_image): prepared weights, no host-side preparation.
  HipContext(const std::string& image_path, int device);
  ~HipContext();
  HipContext(const HipContext&) = delete;
  HipContext& operator=(const HipContext&) = delete;
  mit2cfm_ctx* get() const { return ctx_; }

 private:
  mit2cfm_ctx* ctx_ = nullptr;
};

std::vector<float> run_cfm_euler_hip(HipContext& hip, const Bundle& bundle, std::vector<float> x,
                                     const std::vector<float>& prompt,
                                     const std::vector<float>& cond,
                                     const std::vector<float>& style, uint32_t tokens,
                                     uint32_t prompt_tokens, uint32_t steps, float cfg_rate);
// Same without a bundle argument (weights already resident in the context).
std::vector<float> run_cfm_euler_hip(HipContext& hip, std::vector<float> x,
                                     const std::vector<float>& prompt,
                                     const std::vector<float>& cond,
                                     const std::vector<float>& style, uint32_t tokens,
                                     uint32_t prompt_tokens, uint32_t steps, float cfg_rate);
std::vector<float> run_dit_estimator_step_hip(HipContext& hip, const std::vector<float>& x,
                                              const std::vector<float>& prompt_x,
                                              const std::vector<float>& cond,
                                              const std::vector<float>& style, float timestep,
                                              const std::vector<uint32_t>& mask, uint32_t tokens);
// run_length_regulator_full_metal (runtime/impl/gpt.cpp:4517, :5313): the
// s2mel length regulator, input [in_tokens][1024] -> [out_tokens][512].  The
// context needs the bundle's "s2mel.net.length_regulator.*" tensors (loaded
// with the estimator by the Bundle constructor above).
std::vector<float> run_length_regulator_full_hip(HipContext& hip, const Bundle& bundle,
                                                 const std::vector<float>& input,
                                                 uint32_t in_tokens, uint32_t out_tokens);

// run_bigvgan_vocoder_metal (runtime/impl/dit_cfm_bigvgan.cpp:4196): mel
// [tokens][80] -> waveform [256 * tokens] in [-1, 1].  The context needs the
// bundle's "bigvgan.*" tensors.
std::vector<float> run_bigvgan_vocoder_hip(HipContext& hip, const Bundle& bundle,
                                           const std::vector<float>& mel, uint32_t tokens);
// Same without a bundle argument (weights already resident in the context).
std::vector<float> run_bigvgan_vocoder_hip(HipContext& hip, const std::vector<float>& mel,
                                           uint32_t tokens);

// The GPT mel-code decoder (runtime/impl/gpt.cpp).  The context needs the
// bundle's GPT decoder tensors (gpt.gpt.h.*, gpt.gpt.ln_f.*, gpt.final_norm.*,
// gpt.mel_head.*, gpt.mel_embedding.weight, gpt.mel_pos_embedding.emb.weight).
struct GptGreedyOutputs {  // gpt.cpp:1583-1590 (without the backend comparison field)
  std::vector<uint32_t> predicted_tokens;
  std::vector<uint32_t> input_tokens;
  std::vector<float> last_logits;
  int32_t first_stop_step = -1;
};
struct GptSamplingConfig {  // gpt.cpp:1592-1599
  bool do_sample = false;
  uint64_t seed = 0;
  float temperature = 1.0f;
  uint32_t top_k = 0;
  float top_p = 1.0f;
  float repetition_penalty = 1.0f;
};
// run_gpt_kv_greedy_metal (gpt.cpp:1914-1918; CPU definition :1877): prefix
// [prefix_tokens][1280] -> codes, stopping at the first stop token; greedy,
// or sampled when sampling->do_sample (gpt.cpp:2221-2240), with the
// repetition penalty over repetition_history_prefix (else the start token)
// followed by the predictions so far.  The reference's argument order; the
// bundle is not read (the weights are resident in the context).
GptGreedyOutputs run_gpt_kv_greedy_hip(HipContext& hip, const Bundle& bundle, const std::vector<float>& prefix,
                                       uint32_t prefix_tokens, uint32_t steps, bool hf_generate_positions = false,
                                       const GptSamplingConfig* sampling = nullptr,
                                       const std::vector<uint32_t>* repetition_history_prefix = nullptr);
// The same without a bundle argument.
GptGreedyOutputs run_gpt_kv_greedy_hip(HipContext& hip, const std::vector<float>& prefix,
                                       uint32_t prefix_tokens, uint32_t steps,
                                       bool hf_generate_positions = false,
                                       const GptSamplingConfig* sampling = nullptr,
                                       const std::vector<uint32_t>* repetition_history_prefix = nullptr);
struct GptCachedDecodeOutputs {  // gpt.cpp:1393-1398
  std::vector<float> ln_f;
  std::vector<float> final_norm;
  std::vector<float> logits;
  uint32_t argmax = 0;
};
// run_gpt_cached_decode_metal (gpt.cpp:1427; CPU definition :1400): input
// [prefix_tokens + 1][1280]; the last row decoded against the others' caches.
GptCachedDecodeOutputs run_gpt_cached_decode_hip(HipContext& hip, const std::vector<float>& input,
                                                 uint32_t prefix_tokens);

// Euler step count for synthesis: env MIT2_CFM_STEPS, default 16, clamped to
// the --cfm_steps range 12..25 (main.cpp:57-88, :3181-3187).
uint32_t cfm_synthesis_steps();
constexpr uint32_t kCfmSteps = 25;
constexpr uint32_t kCfmStepsMin = 12;
constexpr uint32_t kCfmStepsMax = 25;

}  // namespace mit2
