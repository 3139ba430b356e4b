// cfm_hip.cpp -- reference-signature shim over the C ABI (see cfm_hip.h).
#include "cfm_hip.h"

#include <cstdlib>
#include <stdexcept>
#include <string>

namespace mit2 {
namespace {
void check(mit2cfm_status st, const mit2cfm_ctx* ctx) {
  if (st != MIT2CFM_OK) throw std::runtime_error(std::string("mit2cfm: ") + mit2cfm_last_error(ctx));
}
}  // namespace

HipContext::HipContext(const Bundle& bundle, int device) {
  std::vector<mit2cfm_tensor> ts;
  for (const auto& info : bundle.tensors()) {
    static const char* const kPrefixes[] = {"s2mel.net.cfm.estimator.", "s2mel.net.length_regulator.", "bigvgan.",
                                            "gpt.gpt.h.", "gpt.gpt.ln_f.", "gpt.final_norm.", "gpt.mel_head.",
                                            "gpt.mel_embedding.", "gpt.mel_pos_embedding."};
    bool wanted = false;
    for (const char* pfx : kPrefixes) wanted = wanted || info.name.rfind(pfx, 0) == 0;
    if (!wanted) continue;
    if (info.dtype != "f32" && info.dtype != "f16") continue;
    const bool f16 = info.dtype == "f16";
    ts.push_back({info.name.c_str(), bundle.tensor_data(info), info.nbytes / (f16 ? 2 : 4),
                  f16 ? MIT2CFM_DTYPE_F16 : MIT2CFM_DTYPE_F32});
  }
  check(mit2cfm_create(ts.data(), (uint32_t)ts.size(), device, &ctx_), nullptr);
}

HipContext::HipContext(uint64_t synthetic_seed, float stddev, int device, bool acoustic, bool gpt) {
  if (!gpt) {
    check(acoustic ? mit2cfm_create_synthetic_acoustic(synthetic_seed, stddev, device, &ctx_)
                   : mit2cfm_create_synthetic(synthetic_seed, stddev, device, &ctx_),
          nullptr);
    return;
  }
  // every synthetic set the context asks for, set s from seed + s
  std::vector<std::string> names;
  std::vector<std::vector<uint8_t>> bufs;
  std::vector<mit2cfm_tensor> ts;
  std::vector<int32_t> sets = {MIT2CFM_SYNTH_ESTIMATOR, MIT2CFM_SYNTH_GPT};
  if (acoustic) sets = {MIT2CFM_SYNTH_ESTIMATOR, MIT2CFM_SYNTH_LENGTH_REGULATOR, MIT2CFM_SYNTH_BIGVGAN,
                        MIT2CFM_SYNTH_GPT};
  size_t total = 0;
  for (int32_t set : sets) total += mit2cfm_synthetic_set_count(set);
  names.reserve(total);
  bufs.reserve(total);
  for (int32_t set : sets) {
    for (uint32_t i = 0; i < mit2cfm_synthetic_set_count(set); ++i) {
      const char* name = nullptr;
      uint32_t ndim = 0;
      int64_t shape[4];
      int32_t dt = 0;
      uint64_t elems = 0;
      check(mit2cfm_synthetic_set_info(set, i, &name, &ndim, shape, &dt, &elems), nullptr);
      names.emplace_back(name);
      bufs.emplace_back(elems * (dt == MIT2CFM_DTYPE_F16 ? 2 : 4));
      check(mit2cfm_synthetic_set_fill(set, i, synthetic_seed + (uint64_t)set, stddev, bufs.back().data()),
            nullptr);
      ts.push_back({names.back().c_str(), bufs.back().data(), elems, dt});
    }
  }
  check(mit2cfm_create(ts.data(), (uint32_t)ts.size(), device, &ctx_), nullptr);
}

HipContext::HipContext(const std::string& image_path, int device) {
  check(mit2cfm_create_from_image(image_path.c_str(), device, &ctx_), nullptr);
}

HipContext::~HipContext() { mit2cfm_destroy(ctx_); }

std::vector<float> run_cfm_euler_hip(HipContext& hip, std::vector<float> x,
                                     const std::vector<float>& prompt,
                                     const std::vector<float>& cond,
                                     const std::vector<float>& style, uint32_t tokens,
                                     uint32_t prompt_tokens, uint32_t steps, float cfg_rate) {
  if (x.size() != (size_t)tokens * 80 || prompt.size() < (size_t)prompt_tokens * 80 ||
      cond.size() != (size_t)tokens * 512 || style.size() != 192)
    throw std::runtime_error("run_cfm_euler_hip: input size mismatch");
  std::vector<float> out((size_t)tokens * 80);
  check(mit2cfm_decode(hip.get(), x.data(), prompt.data(), cond.data(), style.data(), tokens,
                       prompt_tokens, steps, cfg_rate, out.data()),
        hip.get());
  return out;
}

std::vector<float> run_cfm_euler_hip(HipContext& hip, const Bundle& /*bundle*/, std::vector<float> x,
                                     const std::vector<float>& prompt,
                                     const std::vector<float>& cond,
                                     const std::vector<float>& style, uint32_t tokens,
                                     uint32_t prompt_tokens, uint32_t steps, float cfg_rate) {
  return run_cfm_euler_hip(hip, std::move(x), prompt, cond, style, tokens, prompt_tokens, steps,
                           cfg_rate);
}

std::vector<float> run_dit_estimator_step_hip(HipContext& hip, const std::vector<float>& x,
                                              const std::vector<float>& prompt_x,
                                              const std::vector<float>& cond,
                                              const std::vector<float>& style, float timestep,
                                              const std::vector<uint32_t>& mask, uint32_t tokens) {
  if (x.size() != (size_t)tokens * 80 || prompt_x.size() != (size_t)tokens * 80 ||
      cond.size() != (size_t)tokens * 512 || style.size() != 192 || mask.size() != tokens)
    throw std::runtime_error("run_dit_estimator_step_hip: input size mismatch");
  std::vector<float> out((size_t)tokens * 80);
  check(mit2cfm_estimator_step(hip.get(), x.data(), prompt_x.data(), cond.data(), style.data(),
                               mask.data(), timestep, 1, tokens, out.data()),
        hip.get());
  return out;
}

std::vector<float> run_length_regulator_full_hip(HipContext& hip, const Bundle& /*bundle*/,
                                                 const std::vector<float>& input,
                                                 uint32_t in_tokens, uint32_t out_tokens) {
  if (input.size() != (size_t)in_tokens * 1024)
    throw std::runtime_error("run_length_regulator_full_hip: input size mismatch");
  std::vector<float> out((size_t)out_tokens * 512);
  check(mit2cfm_length_regulator(hip.get(), input.data(), in_tokens, out_tokens, out.data()),
        hip.get());
  return out;
}

std::vector<float> run_bigvgan_vocoder_hip(HipContext& hip, const std::vector<float>& mel,
                                           uint32_t tokens) {
  if (tokens == 0 || mel.size() != (size_t)tokens * 80)
    throw std::runtime_error("run_bigvgan_vocoder_hip: mel must have shape [tokens,80]");
  std::vector<float> wav((size_t)tokens * 256);
  check(mit2cfm_bigvgan(hip.get(), mel.data(), tokens, wav.data()), hip.get());
  return wav;
}

std::vector<float> run_bigvgan_vocoder_hip(HipContext& hip, const Bundle& /*bundle*/,
                                           const std::vector<float>& mel, uint32_t tokens) {
  return run_bigvgan_vocoder_hip(hip, mel, tokens);
}

GptGreedyOutputs run_gpt_kv_greedy_hip(HipContext& hip, const std::vector<float>& prefix,
                                       uint32_t prefix_tokens, uint32_t steps, bool hf_generate_positions,
                                       const GptSamplingConfig* sampling,
                                       const std::vector<uint32_t>* repetition_history_prefix) {
  if (prefix.size() != (size_t)prefix_tokens * 1280)
    throw std::runtime_error("run_gpt_kv_greedy_hip: prefix must have shape [prefix_tokens,1280]");
  GptGreedyOutputs out;
  out.predicted_tokens.resize(steps);
  out.input_tokens.resize((size_t)steps + 1);
  out.last_logits.resize(steps ? 8194 : 0);
  uint32_t n_pred = 0, n_in = 0;
  if (sampling && sampling->do_sample) {
    mit2cfm_gpt_sampling s{sampling->seed, sampling->temperature, sampling->top_k, sampling->top_p,
                           sampling->repetition_penalty};
    const bool h = repetition_history_prefix && !repetition_history_prefix->empty();
    check(mit2cfm_gpt_kv_sample(hip.get(), prefix_tokens ? prefix.data() : nullptr, prefix_tokens, steps,
                                hf_generate_positions ? 1 : 0, &s, h ? repetition_history_prefix->data() : nullptr,
                                h ? (uint32_t)repetition_history_prefix->size() : 0u, out.predicted_tokens.data(),
                                &n_pred, out.input_tokens.data(), &n_in, &out.first_stop_step,
                                steps ? out.last_logits.data() : nullptr, nullptr, nullptr),
          hip.get());
  } else {
    check(mit2cfm_gpt_kv_greedy(hip.get(), prefix_tokens ? prefix.data() : nullptr, prefix_tokens, steps,
                                hf_generate_positions ? 1 : 0, out.predicted_tokens.data(), &n_pred,
                                out.input_tokens.data(), &n_in, &out.first_stop_step,
                                steps ? out.last_logits.data() : nullptr, nullptr),
          hip.get());
  }
  out.predicted_tokens.resize(n_pred);
  out.input_tokens.resize(n_in);
  return out;
}

GptGreedyOutputs run_gpt_kv_greedy_hip(HipContext& hip, const Bundle& /*bundle*/, const std::vector<float>& prefix,
                                       uint32_t prefix_tokens, uint32_t steps, bool hf_generate_positions,
                                       const GptSamplingConfig* sampling,
                                       const std::vector<uint32_t>* repetition_history_prefix) {
  return run_gpt_kv_greedy_hip(hip, prefix, prefix_tokens, steps, hf_generate_positions, sampling,
                               repetition_history_prefix);
}

GptCachedDecodeOutputs run_gpt_cached_decode_hip(HipContext& hip, const std::vector<float>& input,
                                                 uint32_t prefix_tokens) {
  if (input.size() != ((size_t)prefix_tokens + 1) * 1280)
    throw std::runtime_error("run_gpt_cached_decode_hip: input must have shape [prefix_tokens+1,1280]");
  GptCachedDecodeOutputs out;
  out.ln_f.resize(1280);
  out.final_norm.resize(1280);
  out.logits.resize(8194);
  check(mit2cfm_gpt_cached_decode(hip.get(), input.data(), prefix_tokens, out.ln_f.data(), out.final_norm.data(),
                                  out.logits.data(), &out.argmax),
        hip.get());
  return out;
}

uint32_t cfm_synthesis_steps() {
  uint32_t steps = 16;
  if (const char* e = std::getenv("MIT2_CFM_STEPS")) {
    const long v = std::strtol(e, nullptr, 10);
    if (v > 0) steps = (uint32_t)v;
  }
  if (steps < kCfmStepsMin) steps = kCfmStepsMin;
  if (steps > kCfmStepsMax) steps = kCfmStepsMax;
  return steps;
}

}  // namespace mit2
