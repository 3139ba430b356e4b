// cli.cpp -- mtts-cfm: the decoder's command-line entry points.
//
// Keeps the reference CLI's flags for this path (runtime/main.cpp):
//   --bench-cfm MODEL T STEPS ITERS     (main.cpp:2925-2930, run_bench_cfm :3065)
//   --test-cfm-euler MODEL [--expect FILE]      (3 steps, cfg 0; :3342)
//   --test-cfm-euler-cfg MODEL [--expect FILE]  (25 steps, cfg 0.5; :3405)
//   --test-cfm-euler-cfg-large MODEL [--expect FILE]
//                                       (T=173, P=8, cfg 0.5, steps 1 and 3;
//                                        :3411-3443)
//   --test-s2mel-full-inputs MODEL NOISE PROMPT COND STYLE STEPS CFG EXPECTED
//                                       (caller's tensor files; :3516-3604)
//   --test-dit-attention-tokens MODEL N [--expect FILE]
//                                       (layer-0 attention core at N tokens,
//                                        batch 2, repeat determinism; :584-638)
//   --decode MODEL T P [--cfm_steps N] [--cfg R] [--seed S] [--out FILE]
//   --cfm_steps N                       (12..25, main.cpp:3181-3187)
//   --inspect-model-bundle DIR, --write-synthetic-bundle DIR [SEED] [STDDEV]
//   --bench-bigvgan MODEL T ITERS       (main.cpp:2931, run_bench_bigvgan
//                                        dit_cfm_bigvgan.cpp:4225)
//   --test-bigvgan-vocoder MODEL        (one mel frame, :4469)
//   --write-image MODEL FILE            (the prepared device weights)
//   --test-gpt-kv-decode MODEL          (gpt.cpp:1469, run_gpt_kv_decode_test)
//   --test-gpt-kv-greedy MODEL          (gpt.cpp:2305, run_gpt_kv_greedy_test)
//   --bench-gpt MODEL P CODES ITERS     (greedy decode of CODES after P prefix rows)
// MODEL is a bundle path, "synthetic[:SEED[:STDDEV]]" or "image:FILE" (a
// device image written by --write-image).  The reference's
// --test-cfm-* compare its Metal path with its CPU path (max-abs 1e-4 on
// its real weights, dit_cfm_bigvgan.cpp:3306-3340).  The library never links
// a CPU restatement, so here the CPU path's output for the same inputs comes
// from a file (--expect FILE: raw float32 [5][80], as the test suite writes
// it from the CPU oracle); the harness reports the max-abs and relative L2
// error against it and passes at the decode's parity bar (final mel
// rel-L2 <= 1e-2), printing whether the reference's max-abs bar also holds.
// Without --expect it checks the invariants the reference's tests also rely
// on: finiteness, zero prompt rows and repeat determinism.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "cfm_hip.h"
#include "synth.h"

namespace {

using Clock = std::chrono::steady_clock;

std::unique_ptr<mit2::HipContext> open_model(const std::string& model, bool acoustic = false, bool gpt = false) {
  if (model.rfind("image:", 0) == 0) return std::make_unique<mit2::HipContext>(model.substr(6), 0);
  if (model.rfind("synthetic", 0) == 0) {
    uint64_t seed = 20240605;
    float stddev = 0.02f;
    const auto c1 = model.find(':');
    if (c1 != std::string::npos) {
      const auto c2 = model.find(':', c1 + 1);
      seed = std::stoull(model.substr(c1 + 1, c2 == std::string::npos ? std::string::npos : c2 - c1 - 1));
      if (c2 != std::string::npos) stddev = std::stof(model.substr(c2 + 1));
    }
    return std::make_unique<mit2::HipContext>(seed, stddev, 0, acoustic, gpt);
  }
  mit2::Bundle b(model);
  return std::make_unique<mit2::HipContext>(b, 0);
}

std::vector<float> series(size_t n, float a, float amp1, int mod, float b, float amp2, bool cos_first) {
  std::vector<float> v(n);
  for (size_t i = 0; i < n; ++i) {
    const float p = cos_first ? std::cos((float)i * a) : std::sin((float)i * a);
    const float q = cos_first ? std::sin((float)(i % mod) * b) : std::cos((float)(i % mod) * b);
    v[i] = p * amp1 + q * amp2;
  }
  return v;
}

int bench_cfm(const std::string& model, uint32_t tokens, uint32_t steps, uint32_t iters) {
  auto hip = open_model(model);
  const uint32_t prompt_tokens = tokens * 6 / 7;
  std::vector<float> x((size_t)tokens * 80), prompt((size_t)prompt_tokens * 80),
      cond((size_t)tokens * 512), style(192);
  for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin((float)i * 0.013f) * 0.4f;
  for (size_t i = 0; i < prompt.size(); ++i) prompt[i] = std::cos((float)i * 0.011f) * 0.5f;
  for (size_t i = 0; i < cond.size(); ++i) cond[i] = std::sin((float)i * 0.007f) * 0.3f;
  for (size_t i = 0; i < style.size(); ++i) style[i] = std::cos((float)i * 0.015f) * 0.18f;
  (void)mit2::run_cfm_euler_hip(*hip, x, prompt, cond, style, tokens, prompt_tokens, steps, 0.7f);
  const auto t0 = Clock::now();
  for (uint32_t i = 0; i < iters; ++i)
    (void)mit2::run_cfm_euler_hip(*hip, x, prompt, cond, style, tokens, prompt_tokens, steps, 0.7f);
  const double total = std::chrono::duration<double>(Clock::now() - t0).count();
  std::cout << "{\n  \"stage\": \"bench_cfm\",\n  \"tokens\": " << tokens << ",\n  \"steps\": " << steps
            << ",\n  \"iters\": " << iters << ",\n  \"seconds_per_call\": " << total / iters
            << ",\n  \"ms_per_step\": " << total / iters / steps * 1000.0
            << ",\n  \"frames_per_second\": " << tokens / (total / iters) << "\n}\n";
  return 0;
}

// The reference's vocoder bench input (dit_cfm_bigvgan.cpp:4228-4231).
std::vector<float> bigvgan_bench_mel(uint32_t tokens) {
  std::vector<float> mel((size_t)tokens * 80);
  for (size_t i = 0; i < mel.size(); ++i)
    mel[i] = std::sin((float)i * 0.017f) * 0.35f + std::cos((float)(i % 97) * 0.013f) * 0.12f;
  return mel;
}

int bench_bigvgan(const std::string& model, uint32_t tokens, uint32_t iters) {
  auto hip = open_model(model, true);
  const auto mel = bigvgan_bench_mel(tokens);
  (void)mit2::run_bigvgan_vocoder_hip(*hip, mel, tokens);
  size_t samples = 0;
  const auto t0 = Clock::now();
  for (uint32_t i = 0; i < iters; ++i) samples = mit2::run_bigvgan_vocoder_hip(*hip, mel, tokens).size();
  const double total = std::chrono::duration<double>(Clock::now() - t0).count();
  std::cout << "{\n  \"stage\": \"bench_bigvgan\",\n  \"tokens\": " << tokens << ",\n  \"samples\": " << samples
            << ",\n  \"iters\": " << iters << ",\n  \"seconds_per_call\": " << total / iters
            << ",\n  \"rtf_vocoder_only\": " << (total / iters) / ((double)samples / 22050.0) << "\n}\n";
  return 0;
}

// Vocoder invariants on run_bigvgan_vocoder_test's input (one mel frame,
// dit_cfm_bigvgan.cpp:4469-4490): finite, inside the clamp, repeatable.  The
// comparison with the CPU path lives in the test suite.
int test_bigvgan_vocoder(const std::string& model) {
  auto hip = open_model(model, true);
  const uint32_t tokens = 1;
  std::vector<float> mel(80);
  for (size_t i = 0; i < mel.size(); ++i)
    mel[i] = std::sin((float)i * 0.017f) * 0.10f + std::cos((float)(i % 71) * 0.029f) * 0.025f;
  const auto a = mit2::run_bigvgan_vocoder_hip(*hip, mel, tokens);
  const auto b = mit2::run_bigvgan_vocoder_hip(*hip, mel, tokens);
  size_t nonfinite = 0;
  float peak = 0.0f, repeat_err = 0.0f;
  for (size_t i = 0; i < a.size(); ++i) {
    if (!std::isfinite(a[i])) ++nonfinite;
    peak = std::max(peak, std::fabs(a[i]));
    repeat_err = std::max(repeat_err, std::fabs(a[i] - b[i]));
  }
  std::cout << "{\n  \"stage\": \"bigvgan_vocoder\",\n  \"input_tokens\": " << tokens << ",\n  \"samples\": "
            << a.size() << ",\n  \"nonfinite\": " << nonfinite << ",\n  \"peak_abs\": " << peak
            << ",\n  \"repeat_max_abs_error\": " << repeat_err << "\n}\n";
  return (nonfinite == 0 && peak <= 1.0f && repeat_err == 0.0f && a.size() == 256) ? 0 : 1;
}

// run_gpt_kv_decode_test's input (gpt.cpp:1469-1479): 3 prefix rows + 1 of
// sin(0.009 i) 0.065 + cos(0.013 (i % 307)) 0.021.  Checks: finite outputs, the
// reported argmax is the logits' first maximum, repeatable.
int test_gpt_kv_decode(const std::string& model) {
  auto hip = open_model(model, false, true);
  const uint32_t prefix_tokens = 3;
  const auto input = series((size_t)(prefix_tokens + 1) * 1280, 0.009f, 0.065f, 307, 0.013f, 0.021f, false);
  const auto a = mit2::run_gpt_cached_decode_hip(*hip, input, prefix_tokens);
  const auto b = mit2::run_gpt_cached_decode_hip(*hip, input, prefix_tokens);
  size_t nonfinite = 0, first_max = 0;
  float repeat_err = 0.0f;
  for (size_t i = 0; i < a.logits.size(); ++i) {
    if (!std::isfinite(a.logits[i])) ++nonfinite;
    if (a.logits[i] > a.logits[first_max]) first_max = i;
    repeat_err = std::max(repeat_err, std::fabs(a.logits[i] - b.logits[i]));
  }
  for (float v : a.final_norm) nonfinite += std::isfinite(v) ? 0 : 1;
  const bool ok = nonfinite == 0 && a.argmax == first_max && repeat_err == 0.0f && b.argmax == a.argmax;
  std::cout << "{\n  \"stage\": \"gpt_kv_decode\",\n  \"prefix_tokens\": " << prefix_tokens
            << ",\n  \"decode_tokens\": 1,\n  \"argmax\": " << a.argmax << ",\n  \"nonfinite\": " << nonfinite
            << ",\n  \"repeat_max_abs_error\": " << repeat_err << ",\n  \"ok\": " << (ok ? "true" : "false")
            << "\n}\n";
  return ok ? 0 : 1;
}

// run_gpt_kv_greedy_test's conditioning series (gpt.cpp:2313-2316) as the
// prefix (its two text rows come from the text embedding, outside this
// library), 3 steps.  Checks: finite logits, tokens in the vocabulary, the
// inputs are the start token then the non-stop predictions, repeatable.
int test_gpt_kv_greedy(const std::string& model) {
  auto hip = open_model(model, false, true);
  const uint32_t prefix_tokens = 8, steps = 3;
  const auto prefix = series((size_t)prefix_tokens * 1280, 0.007f, 0.045f, 251, 0.011f, 0.018f, false);
  const auto a = mit2::run_gpt_kv_greedy_hip(*hip, prefix, prefix_tokens, steps);
  const auto b = mit2::run_gpt_kv_greedy_hip(*hip, prefix, prefix_tokens, steps);
  size_t nonfinite = 0;
  for (float v : a.last_logits) nonfinite += std::isfinite(v) ? 0 : 1;
  bool ok = nonfinite == 0 && a.predicted_tokens == b.predicted_tokens && a.last_logits == b.last_logits &&
            !a.input_tokens.empty() && a.input_tokens[0] == 8192;
  for (size_t i = 0; i < a.predicted_tokens.size(); ++i) {
    ok = ok && a.predicted_tokens[i] < 8194;
    if (a.predicted_tokens[i] != 8193) ok = ok && i + 1 < a.input_tokens.size() && a.input_tokens[i + 1] == a.predicted_tokens[i];
  }
  std::cout << "{\n  \"stage\": \"gpt_kv_greedy_loop\",\n  \"prefix_tokens\": " << prefix_tokens
            << ",\n  \"steps\": " << steps << ",\n  \"predicted_tokens\": [";
  for (size_t i = 0; i < a.predicted_tokens.size(); ++i) std::cout << (i ? ", " : "") << a.predicted_tokens[i];
  std::cout << "],\n  \"first_stop_step\": " << a.first_stop_step << ",\n  \"nonfinite\": " << nonfinite
            << ",\n  \"ok\": " << (ok ? "true" : "false") << "\n}\n";
  return ok ? 0 : 1;
}

int bench_gpt(const std::string& model, uint32_t prefix_tokens, uint32_t codes, uint32_t iters) {
  auto hip = open_model(model, false, true);
  const auto prefix = mit2::make_deterministic_normal_noise(prefix_tokens, 1280, 2, 0.05f);
  mit2::run_gpt_kv_greedy_hip(*hip, prefix, prefix_tokens, 16);  // warm-up
  size_t n = 0;
  const auto t0 = Clock::now();
  for (uint32_t i = 0; i < iters; ++i) n = mit2::run_gpt_kv_greedy_hip(*hip, prefix, prefix_tokens, codes).predicted_tokens.size();
  const double total = std::chrono::duration<double>(Clock::now() - t0).count();
  std::cout << "{\n  \"stage\": \"bench_gpt\",\n  \"prefix_tokens\": " << prefix_tokens << ",\n  \"codes\": " << n
            << ",\n  \"iters\": " << iters << ",\n  \"seconds_per_call\": " << total / iters
            << ",\n  \"ms_per_code_incl_prefill\": " << 1e3 * total / iters / std::max<size_t>(n, 1) << "\n}\n";
  return 0;
}

int test_cfm_euler(const std::string& model, const char* stage, uint32_t steps, float cfg,
                   const std::string& expect) {
  auto hip = open_model(model);
  const uint32_t tokens = 5, prompt_tokens = 2;
  const auto x = series((size_t)tokens * 80, 0.018f, 0.07f, 61, 0.011f, 0.03f, false);
  const auto prompt = series((size_t)prompt_tokens * 80, 0.022f, 0.09f, 37, 0.019f, 0.02f, true);
  const auto cond = series((size_t)tokens * 512, 0.009f, 0.08f, 109, 0.014f, 0.04f, false);
  std::vector<float> style(192);
  for (size_t i = 0; i < style.size(); ++i) style[i] = std::cos((float)i * 0.015f) * 0.18f;
  const auto a = mit2::run_cfm_euler_hip(*hip, x, prompt, cond, style, tokens, prompt_tokens, steps, cfg);
  const auto b = mit2::run_cfm_euler_hip(*hip, x, prompt, cond, style, tokens, prompt_tokens, steps, cfg);
  size_t nonfinite = 0;
  float prompt_abs = 0.0f, repeat_err = 0.0f;
  for (size_t i = 0; i < a.size(); ++i) {
    if (!std::isfinite(a[i])) ++nonfinite;
    if (i < (size_t)prompt_tokens * 80) prompt_abs = std::max(prompt_abs, std::fabs(a[i]));
    repeat_err = std::max(repeat_err, std::fabs(a[i] - b[i]));
  }
  bool ok = nonfinite == 0 && prompt_abs == 0.0f && repeat_err == 0.0f;
  std::cout << "{\n  \"stage\": \"" << stage << "\",\n  \"tokens\": " << tokens
            << ",\n  \"prompt_tokens\": " << prompt_tokens << ",\n  \"steps\": " << steps
            << ",\n  \"cfg_rate\": " << cfg << ",\n  \"nonfinite\": " << nonfinite
            << ",\n  \"prompt_rows_max_abs\": " << prompt_abs
            << ",\n  \"repeat_max_abs_error\": " << repeat_err;
  if (!expect.empty()) {
    std::ifstream f(expect, std::ios::binary | std::ios::ate);
    const size_t bytes = f ? (size_t)f.tellg() : 0;
    if (bytes != a.size() * 4) {
      std::cout << "\n}\n";
      std::cerr << "error: --expect " << expect << " must hold " << a.size() << " float32 values\n";
      return 1;
    }
    std::vector<float> ref(a.size());
    f.seekg(0);
    f.read(reinterpret_cast<char*>(ref.data()), (std::streamsize)bytes);
    double num = 0.0, den = 0.0;
    float max_abs = 0.0f;
    for (size_t i = 0; i < a.size(); ++i) {
      const double d = (double)a[i] - (double)ref[i];
      num += d * d;
      den += (double)ref[i] * ref[i];
      max_abs = std::max(max_abs, (float)std::fabs(d));
    }
    const double rel = std::sqrt(num / std::max(den, 1e-60));
    ok = ok && rel <= 1e-2;
    std::cout << ",\n  \"max_abs_error\": " << max_abs << ",\n  \"rel_l2_error\": " << rel
              << ",\n  \"parity_bar_rel_l2\": 0.01,\n  \"reference_bar_max_abs\": 0.0001"
              << ",\n  \"meets_reference_bar\": " << (max_abs <= 1e-4f ? "true" : "false");
  }
  std::cout << "\n}\n";
  return ok ? 0 : 1;
}

// Raw float32 file (native byte order), as the reference's read_raw_f32.
std::vector<float> read_raw_f32(const std::string& path) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("cannot open " + path);
  const std::streamsize bytes = f.tellg();
  if (bytes < 0 || bytes % 4 != 0) throw std::runtime_error(path + " is not a whole number of float32 values");
  std::vector<float> v((size_t)bytes / 4);
  f.seekg(0);
  f.read(reinterpret_cast<char*>(v.data()), bytes);
  if (!f) throw std::runtime_error("short read from " + path);
  return v;
}

struct Errors {
  float max_abs = 0.0f;
  double rel_l2 = 0.0;
};

// max |got - ref| and ||got - ref|| / ||ref|| over [begin, end) of both.
Errors errors(const std::vector<float>& got, const std::vector<float>& ref, size_t begin, size_t end) {
  Errors e;
  double num = 0.0, den = 0.0;
  for (size_t i = begin; i < end; ++i) {
    const double d = (double)got[i] - (double)ref[i];
    num += d * d;
    den += (double)ref[i] * ref[i];
    e.max_abs = std::max(e.max_abs, (float)std::fabs(d));
  }
  e.rel_l2 = std::sqrt(num / std::max(den, 1e-60));
  return e;
}

size_t count_nonfinite(const std::vector<float>& v) {
  size_t n = 0;
  for (float x : v) n += std::isfinite(x) ? 0 : 1;
  return n;
}

// run_cfm_euler_cfg_large_test (dit_cfm_bigvgan.cpp:3411-3443): T=173, P=8,
// cfg 0.5, the reference's input series, decoded with 1 and with 3 steps.
// The reference compares each with its CPU path at max-abs 3e-3; here the CPU
// path's outputs come from --expect FILE (raw float32 [2][173][80]: the
// 1-step decode, then the 3-step one, as the test suite writes them from
// the CPU oracle).  Without it: finiteness, zero prompt rows, repeatability.
int test_cfm_euler_cfg_large(const std::string& model, const std::string& expect) {
  auto hip = open_model(model);
  constexpr uint32_t tokens = 173, prompt_tokens = 8;
  constexpr float cfg = 0.5f;
  const auto x = series((size_t)tokens * 80, 0.018f, 0.07f, 61, 0.011f, 0.03f, false);
  const auto prompt = series((size_t)prompt_tokens * 80, 0.022f, 0.09f, 37, 0.019f, 0.02f, true);
  const auto cond = series((size_t)tokens * 512, 0.009f, 0.08f, 109, 0.014f, 0.04f, false);
  std::vector<float> style(192);
  for (size_t i = 0; i < style.size(); ++i) style[i] = std::cos((float)i * 0.015f) * 0.18f;
  const size_t n = (size_t)tokens * 80;
  std::vector<float> ref;
  if (!expect.empty()) {
    ref = read_raw_f32(expect);
    if (ref.size() != 2 * n) throw std::runtime_error("--expect must hold 2 x 173 x 80 float32 values");
  }
  std::cout << "{\n  \"stage\": \"cfm_euler_cfg_large\",\n  \"tokens\": " << tokens
            << ",\n  \"prompt_tokens\": " << prompt_tokens << ",\n  \"cfg_rate\": " << cfg
            << ",\n  \"steps\": [\n";
  bool ok = true;
  const uint32_t step_counts[2] = {1u, 3u};
  for (int k = 0; k < 2; ++k) {
    const uint32_t steps = step_counts[k];
    const auto a = mit2::run_cfm_euler_hip(*hip, x, prompt, cond, style, tokens, prompt_tokens, steps, cfg);
    const auto b = mit2::run_cfm_euler_hip(*hip, x, prompt, cond, style, tokens, prompt_tokens, steps, cfg);
    float prompt_abs = 0.0f;
    for (size_t i = 0; i < (size_t)prompt_tokens * 80; ++i) prompt_abs = std::max(prompt_abs, std::fabs(a[i]));
    const float repeat = errors(a, b, 0, n).max_abs;
    const size_t nonfinite = count_nonfinite(a);
    bool pass = nonfinite == 0 && prompt_abs == 0.0f && repeat == 0.0f;
    std::cout << "    {\"steps\": " << steps << ", \"nonfinite\": " << nonfinite
              << ", \"prompt_rows_max_abs\": " << prompt_abs << ", \"repeat_max_abs_error\": " << repeat;
    if (!ref.empty()) {
      std::vector<float> r(ref.begin() + (std::ptrdiff_t)(k * n), ref.begin() + (std::ptrdiff_t)((k + 1) * n));
      const Errors e = errors(a, r, 0, n);
      pass = pass && e.max_abs <= 3e-3f;
      std::cout << ", \"max_abs_error\": " << e.max_abs << ", \"rel_l2_error\": " << e.rel_l2;
    }
    std::cout << ", \"pass\": " << (pass ? "true" : "false") << "}" << (k == 0 ? ",\n" : "\n");
    ok = ok && pass;
  }
  std::cout << "  ],\n  \"bar_max_abs\": 0.003,\n  \"ok\": " << (ok ? "true" : "false") << "\n}\n";
  return ok ? 0 : 1;
}

// run_s2mel_full_inputs_test (dit_cfm_bigvgan.cpp:3516-3604): the decode of
// the caller's tensors -- noise [T][80], prompt mel [P][80], condition
// [T][512], style [192], raw float32 files -- against the expected full mel
// [T][80], over the full mel and the generated rows, at the reference's
// max-abs 3e-3.  Unlike the reference, a failing comparison is reported as
// it is (no second attempt).
int test_s2mel_full_inputs(const std::string& model, const std::string& noise_path,
                           const std::string& prompt_path, const std::string& cond_path,
                           const std::string& style_path, uint32_t steps, float cfg,
                           const std::string& expected_path) {
  const auto started = Clock::now();
  const auto noise = read_raw_f32(noise_path);
  const auto prompt = read_raw_f32(prompt_path);
  const auto cond = read_raw_f32(cond_path);
  const auto style = read_raw_f32(style_path);
  const auto expected = read_raw_f32(expected_path);
  if (noise.empty() || noise.size() % 80 != 0) throw std::runtime_error("noise must have shape [tokens,80]");
  if (prompt.empty() || prompt.size() % 80 != 0)
    throw std::runtime_error("prompt_mel must have shape [prompt_tokens,80]");
  if (steps == 0) throw std::runtime_error("steps must be positive");
  const uint32_t tokens = (uint32_t)(noise.size() / 80), prompt_tokens = (uint32_t)(prompt.size() / 80);
  if (prompt_tokens > tokens) throw std::runtime_error("prompt_tokens exceeds total tokens");
  if (cond.size() != (size_t)tokens * 512) throw std::runtime_error("condition must have shape [tokens,512]");
  if (style.size() != 192) throw std::runtime_error("style must have shape [192]");
  if (expected.size() != noise.size()) throw std::runtime_error("expected full mel size mismatch");
  auto hip = open_model(model);  // after the inputs are checked: a bad file needs no GPU
  const auto got = mit2::run_cfm_euler_hip(*hip, noise, prompt, cond, style, tokens, prompt_tokens, steps, cfg);
  const Errors full = errors(got, expected, 0, got.size());
  const Errors gen = errors(got, expected, (size_t)prompt_tokens * 80, got.size());
  const bool ok = full.max_abs <= 3e-3f && gen.max_abs <= 3e-3f && count_nonfinite(got) == 0;
  const double elapsed = std::chrono::duration<double>(Clock::now() - started).count();
  std::cout << "{\n  \"stage\": \"s2mel_full_inputs_test\",\n  \"tokens\": " << tokens
            << ",\n  \"prompt_tokens\": " << prompt_tokens << ",\n  \"generated_tokens\": "
            << tokens - prompt_tokens << ",\n  \"steps\": " << steps << ",\n  \"cfg_rate\": " << cfg
            << ",\n  \"full_vs_expected_max_abs_error\": " << full.max_abs
            << ",\n  \"generated_vs_expected_max_abs_error\": " << gen.max_abs
            << ",\n  \"full_vs_expected_rel_l2_error\": " << full.rel_l2
            << ",\n  \"bar_max_abs\": 0.003,\n  \"ok\": " << (ok ? "true" : "false")
            << ",\n  \"elapsed_seconds\": " << elapsed << "\n}\n";
  return ok ? 0 : 1;
}

// run_dit_attention_core_tokens_test (dit_cfm_bigvgan.cpp:584-638): the layer-0
// attention core (wqkv, RoPE, attention, wo) on the reference's input series
// at N tokens.  Against the CPU path's output for that input (--expect FILE,
// raw float32 [N][512], written by the test suite from the CPU oracle) at the
// reference's max-abs 1e-3; a batch of two (the series, then a second one)
// whose first branch must match the single run at that bar, and which must
// repeat exactly (repeat error 0, the reference's determinism gate).
int test_dit_attention_tokens(const std::string& model, uint32_t tokens, const std::string& expect) {
  if (tokens == 0) throw std::runtime_error("N must be positive");
  auto hip = open_model(model);
  const size_t n = (size_t)tokens * 512;
  std::vector<float> input(n);
  for (size_t i = 0; i < n; ++i)
    input[i] = std::sin((float)i * 0.017f) * 0.13f + std::cos((float)(i % 97) * 0.011f) * 0.09f;
  auto stage = [&](const std::vector<float>& in, uint32_t batch) {
    std::vector<uint32_t> mask((size_t)batch * tokens, 1u);
    std::vector<float> out(in.size());
    const mit2cfm_status st =
        mit2cfm_stage_attention_core(hip->get(), in.data(), mask.data(), batch, tokens, 0, out.data());
    if (st != MIT2CFM_OK) throw std::runtime_error(mit2cfm_last_error(hip->get()));
    return out;
  };
  const auto single = stage(input, 1);
  std::vector<float> input_b(2 * n);
  std::copy(input.begin(), input.end(), input_b.begin());
  for (size_t i = 0; i < n; ++i) input_b[n + i] = std::cos((float)i * 0.019f) * 0.11f;
  const auto b1 = stage(input_b, 2);
  const auto b2 = stage(input_b, 2);
  const float repeat = errors(b1, b2, 0, 2 * n).max_abs;
  const std::vector<float> branch0(b1.begin(), b1.begin() + (std::ptrdiff_t)n);
  const float batched = errors(branch0, single, 0, n).max_abs;
  bool ok = repeat == 0.0f && batched <= 1e-3f && count_nonfinite(b1) == 0;
  std::cout << "{\n  \"stage\": \"dit_attention_core_tokens\",\n  \"tokens\": " << tokens;
  if (!expect.empty()) {
    const auto ref = read_raw_f32(expect);
    if (ref.size() != n) throw std::runtime_error("--expect must hold N x 512 float32 values");
    const Errors e = errors(single, ref, 0, n);
    const Errors eb = errors(branch0, ref, 0, n);
    ok = ok && e.max_abs <= 1e-3f && eb.max_abs <= 1e-3f;
    std::cout << ",\n  \"max_abs_error\": " << e.max_abs << ",\n  \"rel_l2_error\": " << e.rel_l2
              << ",\n  \"batched_branch0_err\": " << eb.max_abs;
  }
  std::cout << ",\n  \"batched_vs_single_max_abs\": " << batched << ",\n  \"batched_repeat_err\": " << repeat
            << ",\n  \"ok\": " << (ok ? "true" : "false") << "\n}\n";
  return ok ? 0 : 1;
}

int decode(const std::string& model, uint32_t tokens, uint32_t prompt_tokens, uint32_t steps, float cfg,
           uint64_t seed, const std::string& out) {
  auto hip = open_model(model);
  const auto x = mit2::make_deterministic_normal_noise(tokens, 80, seed, 1.0f);
  auto prompt = mit2::make_deterministic_normal_noise(std::max(prompt_tokens, 1u), 80, seed + 1, 2.0f);
  for (auto& v : prompt) v -= 5.0f;
  const auto cond = mit2::make_deterministic_normal_noise(tokens, 512, seed + 2, 1.0f);
  const auto style = mit2::make_deterministic_normal_noise(1, 192, seed + 3, 1.0f);
  const auto t0 = Clock::now();
  const auto mel = mit2::run_cfm_euler_hip(*hip, x, prompt, cond, style, tokens, prompt_tokens, steps, cfg);
  const double sec = std::chrono::duration<double>(Clock::now() - t0).count();
  if (!out.empty()) {
    std::ofstream f(out, std::ios::binary);
    f.write(reinterpret_cast<const char*>(mel.data()), (std::streamsize)(mel.size() * 4));
  }
  double ss = 0;
  for (float v : mel) ss += (double)v * v;
  std::cout << "{\"stage\": \"decode\", \"tokens\": " << tokens << ", \"prompt_tokens\": " << prompt_tokens
            << ", \"steps\": " << steps << ", \"cfg_rate\": " << cfg << ", \"seconds\": " << sec
            << ", \"rms\": " << std::sqrt(ss / mel.size()) << "}\n";
  return 0;
}

int usage() {
  std::cerr << "usage: mtts-cfm --bench-cfm MODEL T STEPS ITERS | --test-cfm-euler MODEL [--expect FILE] |\n"
               "       --test-cfm-euler-cfg MODEL [--expect FILE] | --test-cfm-euler-cfg-large MODEL [--expect FILE] |\n"
               "       --test-s2mel-full-inputs MODEL NOISE PROMPT COND STYLE STEPS CFG EXPECTED |\n"
               "       --test-dit-attention-tokens MODEL N [--expect FILE] |\n"
               "       --decode MODEL T P [--cfm_steps N] [--cfg R]\n"
               "       [--seed S] [--out FILE] | --inspect-model-bundle DIR |\n"
               "       --write-synthetic-bundle DIR [SEED] [STDDEV] |\n"
               "       --bench-bigvgan MODEL T ITERS | --test-bigvgan-vocoder MODEL |\n"
               "       --write-image MODEL FILE | --test-gpt-kv-decode MODEL |\n"
               "       --test-gpt-kv-greedy MODEL | --bench-gpt MODEL P CODES ITERS\n"
               "MODEL: bundle path, synthetic[:SEED[:STDDEV]] or image:FILE\n";
  return 2;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    uint32_t steps = mit2::cfm_synthesis_steps();
    float cfg = 0.7f;
    uint64_t seed = 1;
    std::string out, expect;
    for (int i = 1; i < argc; ++i) {
      const std::string a = argv[i];
      if (a == "--cfm_steps" && i + 1 < argc) {
        const long n = std::strtol(argv[i + 1], nullptr, 10);
        if (n < (long)mit2::kCfmStepsMin || n > (long)mit2::kCfmStepsMax) {
          std::cerr << "error: --cfm_steps must be between 12 and 25 (got " << n << ")\n";
          return 1;
        }
        steps = (uint32_t)n;
      } else if (a == "--cfg" && i + 1 < argc) {
        cfg = std::stof(argv[i + 1]);
      } else if (a == "--seed" && i + 1 < argc) {
        seed = std::stoull(argv[i + 1]);
      } else if (a == "--out" && i + 1 < argc) {
        out = argv[i + 1];
      } else if (a == "--expect" && i + 1 < argc) {
        expect = argv[i + 1];
      }
    }
    for (int i = 1; i < argc; ++i) {
      const std::string a = argv[i];
      if (a == "--bench-cfm" && i + 4 < argc)
        return bench_cfm(argv[i + 1], (uint32_t)std::stoul(argv[i + 2]), (uint32_t)std::stoul(argv[i + 3]),
                         (uint32_t)std::stoul(argv[i + 4]));
      if (a == "--test-cfm-euler" && i + 1 < argc)
        return test_cfm_euler(argv[i + 1], "cfm_euler", 3, 0.0f, expect);
      if (a == "--write-image" && i + 2 < argc) {
        auto hip = open_model(argv[i + 1], true);
        const mit2cfm_status st = mit2cfm_write_image(hip->get(), argv[i + 2]);
        if (st != MIT2CFM_OK) std::cerr << mit2cfm_last_error(hip->get()) << "\n";
        return st == MIT2CFM_OK ? 0 : 1;
      }
      if (a == "--bench-bigvgan" && i + 3 < argc)
        return bench_bigvgan(argv[i + 1], (uint32_t)std::stoul(argv[i + 2]), (uint32_t)std::stoul(argv[i + 3]));
      if (a == "--test-bigvgan-vocoder" && i + 1 < argc) return test_bigvgan_vocoder(argv[i + 1]);
      if (a == "--test-gpt-kv-decode" && i + 1 < argc) return test_gpt_kv_decode(argv[i + 1]);
      if (a == "--test-gpt-kv-greedy" && i + 1 < argc) return test_gpt_kv_greedy(argv[i + 1]);
      if (a == "--bench-gpt" && i + 4 < argc)
        return bench_gpt(argv[i + 1], (uint32_t)std::stoul(argv[i + 2]), (uint32_t)std::stoul(argv[i + 3]),
                         (uint32_t)std::stoul(argv[i + 4]));
      if (a == "--test-cfm-euler-cfg" && i + 1 < argc)
        return test_cfm_euler(argv[i + 1], "cfm_euler_cfg", 25, 0.5f, expect);
      if (a == "--test-cfm-euler-cfg-large" && i + 1 < argc) return test_cfm_euler_cfg_large(argv[i + 1], expect);
      if (a == "--test-s2mel-full-inputs" && i + 8 < argc)
        return test_s2mel_full_inputs(argv[i + 1], argv[i + 2], argv[i + 3], argv[i + 4], argv[i + 5],
                                      (uint32_t)std::stoul(argv[i + 6]), std::stof(argv[i + 7]), argv[i + 8]);
      if (a == "--test-dit-attention-tokens" && i + 2 < argc)
        return test_dit_attention_tokens(argv[i + 1], (uint32_t)std::stoul(argv[i + 2]), expect);
      if (a == "--decode" && i + 3 < argc)
        return decode(argv[i + 1], (uint32_t)std::stoul(argv[i + 2]), (uint32_t)std::stoul(argv[i + 3]), steps,
                      cfg, seed, out);
      if (a == "--inspect-model-bundle" && i + 1 < argc) {
        uint64_t n = 0, bytes = 0;
        const mit2cfm_status st = mit2cfm_inspect_bundle(argv[i + 1], &n, &bytes, 1);
        std::cout << "{\"ok\": " << (st == MIT2CFM_OK ? "true" : "false") << ", \"tensors\": " << n
                  << ", \"payload_bytes\": " << bytes
                  << ", \"sha256_verified\": " << (st == MIT2CFM_OK ? "true" : "false")
                  << ", \"error\": \"" << (st == MIT2CFM_OK ? "" : mit2cfm_last_error(nullptr)) << "\"}\n";
        return st == MIT2CFM_OK ? 0 : 1;
      }
      if (a == "--write-synthetic-bundle" && i + 1 < argc) {
        const uint64_t s = i + 2 < argc ? std::stoull(argv[i + 2]) : 20240605ull;
        const float sd = i + 3 < argc ? std::stof(argv[i + 3]) : 0.02f;
        const mit2cfm_status st = mit2cfm_write_synthetic_bundle(argv[i + 1], s, sd);
        if (st != MIT2CFM_OK) std::cerr << mit2cfm_last_error(nullptr) << "\n";
        return st == MIT2CFM_OK ? 0 : 1;
      }
    }
    return usage();
  } catch (const std::exception& e) {
    std::cerr << "error: " << e.what() << "\n";
    return 1;
  }
}
