// cfm_hip.cpp -- reference-signature shim over the C ABI (see cfm_hip.h).
#include "cfm_hip.h"

#include <cstdlib>
#include <stdexcept>

namespace mit2 {
namespace {
void check(mit2cfm_status st, const mit2cfm_ctx* ctx) {
  if (st != MIT2CFM_OK) throw std::runtime_error(std::string("mit2cfm: ") + mit2cfm_last_error(ctx));
}
}  // namespace

HipContext::HipContext(const Bundle& bundle, int device) {
  std::vector<mit2cfm_tensor> ts;
  for (const auto& info : bundle.tensors()) {
    if (info.name.rfind("s2mel.net.cfm.estimator.", 0) != 0 &&
        info.name.rfind("s2mel.net.length_regulator.", 0) != 0 && info.name.rfind("bigvgan.", 0) != 0)
      continue;
    if (info.dtype != "f32" && info.dtype != "f16") continue;
    const bool f16 = info.dtype == "f16";
    ts.push_back({info.name.c_str(), bundle.tensor_data(info), info.nbytes / (f16 ? 2 : 4),
                  f16 ? MIT2CFM_DTYPE_F16 : MIT2CFM_DTYPE_F32});
  }
  check(mit2cfm_create(ts.data(), (uint32_t)ts.size(), device, &ctx_), nullptr);
}

HipContext::HipContext(uint64_t synthetic_seed, float stddev, int device, bool acoustic) {
  check(acoustic ? mit2cfm_create_synthetic_acoustic(synthetic_seed, stddev, device, &ctx_)
                 : mit2cfm_create_synthetic(synthetic_seed, stddev, device, &ctx_),
        nullptr);
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
