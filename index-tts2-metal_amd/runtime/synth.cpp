// synth.cpp -- seeded synthetic inputs and weights (see synth.h).
#include "synth.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>

namespace mit2 {

uint64_t splitmix64_next(uint64_t& state) {
  uint64_t z = (state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

float splitmix64_uniform_open01(uint64_t& state) {
  constexpr double scale = 1.0 / static_cast<double>(1ull << 53);
  const uint64_t bits = splitmix64_next(state) >> 11;
  double v = (static_cast<double>(bits) + 0.5) * scale;
  if (v <= 0.0) v = scale;
  if (v >= 1.0) v = 1.0 - scale;
  return static_cast<float>(v);
}

std::vector<float> make_deterministic_normal_noise(uint32_t tokens, uint32_t channels,
                                                   uint64_t seed, float temperature) {
  if (tokens == 0 || channels == 0) throw std::runtime_error("noise shape must be non-empty");
  constexpr float two_pi = 6.2831853071795864769f;
  std::vector<float> out(static_cast<size_t>(tokens) * channels);
  uint64_t state = seed;
  size_t i = 0;
  while (i < out.size()) {
    const float u1 = splitmix64_uniform_open01(state);
    const float u2 = splitmix64_uniform_open01(state);
    const float radius = std::sqrt(-2.0f * std::log(u1));
    const float angle = two_pi * u2;
    out[i++] = radius * std::cos(angle) * temperature;
    if (i < out.size()) out[i++] = radius * std::sin(angle) * temperature;
  }
  return out;
}

const std::vector<SynthSpec>& estimator_tensor_specs() {
  static const std::vector<SynthSpec> specs = [] {
    std::vector<SynthSpec> v;
    const std::string p = "s2mel.net.cfm.estimator.";
    auto add = [&](const std::string& n, std::vector<int64_t> s, const char* dt = "f16") {
      v.push_back({p + n, std::move(s), dt});
    };
    for (const char* te : {"t_embedder", "t_embedder2"}) {
      const std::string t = te;
      add(t + ".freqs", {128}, "f32");
      add(t + ".mlp.0.weight", {512, 256});
      add(t + ".mlp.0.bias", {512});
      add(t + ".mlp.2.weight", {512, 512});
      add(t + ".mlp.2.bias", {512});
    }
    add("cond_projection.weight", {512, 512});
    add("cond_projection.bias", {512});
    add("cond_x_merge_linear.weight", {512, 864});
    add("cond_x_merge_linear.bias", {512});
    for (int l = 0; l < 13; ++l) {
      const std::string b = "transformer.layers." + std::to_string(l);
      for (const char* nn : {".attention_norm", ".ffn_norm"}) {
        add(b + nn + ".norm.weight", {512});
        add(b + nn + ".project_layer.weight", {1024, 512});
        add(b + nn + ".project_layer.bias", {1024});
      }
      add(b + ".attention.wqkv.weight", {1536, 512});
      add(b + ".attention.wo.weight", {512, 512});
      add(b + ".feed_forward.w1.weight", {1536, 512});
      add(b + ".feed_forward.w3.weight", {1536, 512});
      add(b + ".feed_forward.w2.weight", {512, 1536});
      if (l > 6) {
        add(b + ".skip_in_linear.weight", {512, 1024});
        add(b + ".skip_in_linear.bias", {512});
      }
    }
    add("transformer.norm.norm.weight", {512});
    add("transformer.norm.project_layer.weight", {1024, 512});
    add("transformer.norm.project_layer.bias", {1024});
    add("skip_linear.weight", {512, 592});
    add("skip_linear.bias", {512});
    add("conv1.weight", {512, 512});
    add("conv1.bias", {512});
    add("res_projection.weight", {512, 512});
    add("res_projection.bias", {512});
    add("wavenet.cond_layer.conv.conv.weight_g", {8192, 1, 1});
    add("wavenet.cond_layer.conv.conv.weight_v", {8192, 512, 1});
    add("wavenet.cond_layer.conv.conv.bias", {8192});
    for (int l = 0; l < 8; ++l) {
      const std::string b = "wavenet.in_layers." + std::to_string(l) + ".conv.conv";
      add(b + ".weight_g", {1024, 1, 1});
      add(b + ".weight_v", {1024, 512, 5});
      add(b + ".bias", {1024});
      const int64_t c = l < 7 ? 1024 : 512;
      const std::string r = "wavenet.res_skip_layers." + std::to_string(l) + ".conv.conv";
      add(r + ".weight_g", {c, 1, 1});
      add(r + ".weight_v", {c, 512, 1});
      add(r + ".bias", {c});
    }
    add("final_layer.adaLN_modulation.1.weight", {1024, 512});
    add("final_layer.adaLN_modulation.1.bias", {1024});
    add("final_layer.linear.weight_g", {512, 1});
    add("final_layer.linear.weight_v", {512, 512});
    add("final_layer.linear.bias", {512});
    add("conv2.weight", {80, 512, 1});
    add("conv2.bias", {80});
    std::sort(v.begin(), v.end(), [](const SynthSpec& a, const SynthSpec& b) { return a.name < b.name; });
    return v;
  }();
  return specs;
}

std::vector<uint8_t> synth_tensor_bytes(size_t i, uint64_t base_seed, float stddev) {
  const auto& specs = estimator_tensor_specs();
  if (i >= specs.size()) throw std::out_of_range("synthetic tensor index");
  const SynthSpec& s = specs[i];
  size_t n = 1;
  for (int64_t d : s.shape) n *= (size_t)d;
  if (s.dtype == "f32") {  // *.freqs
    std::vector<float> f(n);
    const float neg_log = -std::log(10000.0f);
    for (size_t k = 0; k < n; ++k) f[k] = std::exp(neg_log * (float)k / (float)n);
    std::vector<uint8_t> out(n * 4);
    std::memcpy(out.data(), f.data(), out.size());
    return out;
  }
  // stddev > 0: every tensor N(0, stddev).  stddev == 0: activation-preserving
  // scales -- matrices N(0, 1/sqrt(fan_in)), norm weights and weight-norm
  // gains 1 + N(0, 0.02), other vectors N(0, 0.02).
  float scale = stddev, offset = 0.0f;
  if (stddev == 0.0f) {
    const bool gain = s.name.size() >= 12 && (s.name.compare(s.name.size() - 12, 12, ".norm.weight") == 0 ||
                                              s.name.compare(s.name.size() - 9, 9, ".weight_g") == 0);
    if (s.shape.size() >= 2 && s.name.compare(s.name.size() - 9, 9, ".weight_g") != 0) {
      size_t fan_in = 1;
      for (size_t d = 1; d < s.shape.size(); ++d) fan_in *= (size_t)s.shape[d];
      scale = 1.0f / std::sqrt((float)fan_in);
    } else {
      scale = 0.02f;
      offset = gain ? 1.0f : 0.0f;
    }
  }
  const auto v = make_deterministic_normal_noise((uint32_t)n, 1, base_seed + i, scale);
  std::vector<uint8_t> out(n * 2);
  for (size_t k = 0; k < n; ++k) {
    const _Float16 h = (_Float16)(v[k] + offset);
    std::memcpy(&out[k * 2], &h, 2);
  }
  return out;
}

namespace {

size_t elems_of(const SynthSpec& s) {
  size_t n = 1;
  for (int64_t d : s.shape) n *= (size_t)d;
  return n;
}

bool ends_with(const std::string& s, const char* suffix) {
  const size_t n = std::strlen(suffix);
  return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
}

std::vector<uint8_t> to_f16_bytes(const std::vector<float>& v) {
  std::vector<uint8_t> out(v.size() * 2);
  for (size_t k = 0; k < v.size(); ++k) {
    const _Float16 h = (_Float16)v[k];
    std::memcpy(&out[k * 2], &h, 2);
  }
  return out;
}

std::vector<uint8_t> to_f32_bytes(const std::vector<float>& v) {
  std::vector<uint8_t> out(v.size() * 4);
  std::memcpy(out.data(), v.data(), out.size());
  return out;
}

void sort_specs(std::vector<SynthSpec>& v) {
  std::sort(v.begin(), v.end(), [](const SynthSpec& a, const SynthSpec& b) { return a.name < b.name; });
}

}  // namespace

const std::vector<SynthSpec>& length_regulator_tensor_specs() {
  static const std::vector<SynthSpec> specs = [] {
    std::vector<SynthSpec> v;
    const std::string p = "s2mel.net.length_regulator.";
    v.push_back({p + "content_in_proj.weight", {512, 1024}, "f16"});
    v.push_back({p + "content_in_proj.bias", {512}, "f16"});
    v.push_back({p + "model.12.weight", {512, 512, 1}, "f16"});
    v.push_back({p + "model.12.bias", {512}, "f16"});
    for (int i : {0, 3, 6, 9}) {
      v.push_back({p + "model." + std::to_string(i) + ".weight", {512, 512, 3}, "f16"});
      v.push_back({p + "model." + std::to_string(i) + ".bias", {512}, "f16"});
    }
    for (int i : {1, 4, 7, 10}) {
      v.push_back({p + "model." + std::to_string(i) + ".weight", {512}, "f16"});
      v.push_back({p + "model." + std::to_string(i) + ".bias", {512}, "f16"});
    }
    sort_specs(v);
    return v;
  }();
  return specs;
}

std::vector<uint8_t> synth_lr_tensor_bytes(size_t i, uint64_t base_seed, float stddev) {
  const auto& specs = length_regulator_tensor_specs();
  if (i >= specs.size()) throw std::out_of_range("synthetic tensor index");
  const SynthSpec& s = specs[i];
  auto v = make_deterministic_normal_noise((uint32_t)elems_of(s), 1, base_seed + i, stddev);
  if (ends_with(s.name, ".weight") && s.shape.size() == 1)  // GroupNorm weight
    for (float& x : v) x = x + 1.0f;
  return to_f16_bytes(v);
}

const std::vector<SynthSpec>& bigvgan_tensor_specs() {
  static const std::vector<SynthSpec> specs = [] {
    std::vector<SynthSpec> v;
    auto conv = [&](const std::string& p, int64_t rows, int64_t cols, int64_t k, bool bias, int64_t nb) {
      v.push_back({p + ".weight_g", {rows, 1, 1}, "f16"});
      v.push_back({p + ".weight_v", {rows, cols, k}, "f16"});
      if (bias) v.push_back({p + ".bias", {nb}, "f16"});
    };
    auto act = [&](const std::string& p, int64_t c) {
      v.push_back({p + ".upsample.filter", {1, 1, 12}, "f32"});
      v.push_back({p + ".downsample.lowpass.filter", {1, 1, 12}, "f32"});
      v.push_back({p + ".act.alpha", {c}, "f32"});
      v.push_back({p + ".act.beta", {c}, "f32"});
    };
    conv("bigvgan.conv_pre", 1536, 80, 7, true, 1536);
    const int64_t ups[6][4] = {{1536, 768, 8, 0}, {768, 384, 8, 1}, {384, 192, 4, 2},
                               {192, 96, 4, 3},   {96, 48, 4, 4},   {48, 24, 4, 5}};
    for (const auto& u : ups)
      conv("bigvgan.ups." + std::to_string(u[3]) + ".0", u[0], u[1], u[2], true, u[1]);
    for (int j = 0; j < 18; ++j) {
      const int64_t c = 768 >> (j / 3), k = (j % 3 == 0) ? 3 : (j % 3 == 1) ? 7 : 11;
      const std::string p = "bigvgan.resblocks." + std::to_string(j);
      for (int pr = 0; pr < 3; ++pr) {
        conv(p + ".convs1." + std::to_string(pr), c, c, k, true, c);
        conv(p + ".convs2." + std::to_string(pr), c, c, k, true, c);
      }
      for (int a = 0; a < 6; ++a) act(p + ".activations." + std::to_string(a), c);
    }
    act("bigvgan.activation_post", 24);
    conv("bigvgan.conv_post", 1, 24, 7, false, 0);
    sort_specs(v);
    return v;
  }();
  return specs;
}

std::vector<float> kaiser_sinc_filter12() {
  constexpr int kTaps = 12, kHalf = 6;
  const double cutoff = 0.25, half_width = 0.3, pi = 3.14159265358979323846;
  // Kaiser's empirical beta for attenuation A = 2.285 (N/2 - 1) pi (4 half_width) + 7.95.
  const double a = 2.285 * (kHalf - 1) * pi * (4.0 * half_width) + 7.95;
  const double beta = a > 50.0 ? 0.1102 * (a - 8.7)
                               : (a >= 21.0 ? 0.5842 * std::pow(a - 21.0, 0.4) + 0.07886 * (a - 21.0) : 0.0);
  const double centre = (kTaps - 1) / 2.0;
  double f[kTaps], sum = 0.0;
  for (int n = 0; n < kTaps; ++n) {
    const double r = (n - centre) / centre;
    const double window = std::cyl_bessel_i(0.0, beta * std::sqrt(1.0 - r * r)) / std::cyl_bessel_i(0.0, beta);
    const double x = 2.0 * cutoff * (n - kHalf + 0.5);
    const double sinc = x == 0.0 ? 1.0 : std::sin(pi * x) / (pi * x);
    f[n] = 2.0 * cutoff * window * sinc;
    sum += f[n];
  }
  std::vector<float> out(kTaps);
  for (int n = 0; n < kTaps; ++n) out[n] = (float)(f[n] / sum);
  return out;
}

std::vector<uint8_t> synth_bigvgan_tensor_bytes(size_t i, uint64_t base_seed, float stddev) {
  const auto& specs = bigvgan_tensor_specs();
  if (i >= specs.size()) throw std::out_of_range("synthetic tensor index");
  const SynthSpec& s = specs[i];
  const uint32_t n = (uint32_t)elems_of(s);
  if (ends_with(s.name, ".filter")) return to_f32_bytes(kaiser_sinc_filter12());
  if (ends_with(s.name, ".act.alpha") || ends_with(s.name, ".act.beta"))
    return to_f32_bytes(make_deterministic_normal_noise(n, 1, base_seed + i, 0.1f));
  auto v = make_deterministic_normal_noise(n, 1, base_seed + i, stddev);
  if (ends_with(s.name, ".weight_g")) {
    float g = 0.6f;
    if (s.name.rfind("bigvgan.conv_pre", 0) == 0 || s.name.rfind("bigvgan.ups", 0) == 0) g = 1.0f;
    if (s.name.rfind("bigvgan.conv_post", 0) == 0) g = 0.1f;
    for (float& x : v) x = g * (1.0f + x);
  }
  return to_f16_bytes(v);
}

const std::vector<SynthSpec>& gpt_tensor_specs() {
  static const std::vector<SynthSpec> specs = [] {
    std::vector<SynthSpec> v;
    for (int l = 0; l < 24; ++l) {
      const std::string p = "gpt.gpt.h." + std::to_string(l) + ".";
      v.push_back({p + "ln_1.weight", {1280}, "f16"});
      v.push_back({p + "ln_1.bias", {1280}, "f16"});
      v.push_back({p + "attn.c_attn.weight", {1280, 3840}, "f16"});
      v.push_back({p + "attn.c_attn.bias", {3840}, "f16"});
      v.push_back({p + "attn.c_proj.weight", {1280, 1280}, "f16"});
      v.push_back({p + "attn.c_proj.bias", {1280}, "f16"});
      v.push_back({p + "ln_2.weight", {1280}, "f16"});
      v.push_back({p + "ln_2.bias", {1280}, "f16"});
      v.push_back({p + "mlp.c_fc.weight", {1280, 5120}, "f16"});
      v.push_back({p + "mlp.c_fc.bias", {5120}, "f16"});
      v.push_back({p + "mlp.c_proj.weight", {5120, 1280}, "f16"});
      v.push_back({p + "mlp.c_proj.bias", {1280}, "f16"});
    }
    v.push_back({"gpt.gpt.ln_f.weight", {1280}, "f16"});
    v.push_back({"gpt.gpt.ln_f.bias", {1280}, "f16"});
    v.push_back({"gpt.final_norm.weight", {1280}, "f16"});
    v.push_back({"gpt.final_norm.bias", {1280}, "f16"});
    v.push_back({"gpt.mel_head.weight", {8194, 1280}, "f16"});
    v.push_back({"gpt.mel_head.bias", {8194}, "f16"});
    v.push_back({"gpt.mel_embedding.weight", {8194, 1280}, "f16"});
    v.push_back({"gpt.mel_pos_embedding.emb.weight", {1818, 1280}, "f16"});
    sort_specs(v);
    return v;
  }();
  return specs;
}

std::vector<uint8_t> synth_gpt_tensor_bytes(size_t i, uint64_t base_seed, float stddev) {
  const auto& specs = gpt_tensor_specs();
  if (i >= specs.size()) throw std::out_of_range("synthetic tensor index");
  const SynthSpec& s = specs[i];
  auto v = make_deterministic_normal_noise((uint32_t)elems_of(s), 1, base_seed + i, stddev);
  const bool norm_weight = s.shape.size() == 1 && ends_with(s.name, ".weight");
  if (norm_weight)
    for (float& x : v) x = x + 1.0f;
  return to_f16_bytes(v);
}

}  // namespace mit2
