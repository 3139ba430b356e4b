// cli.cpp -- mtts-cfm: the decoder's command-line entry points.
//
// Keeps the reference CLI's flags for this path (runtime/main.cpp):
//   --bench-cfm MODEL T STEPS ITERS     (main.cpp:2925-2930, run_bench_cfm :3065)
//   --test-cfm-euler MODEL [--expect FILE]      (3 steps, cfg 0; :3342)
//   --test-cfm-euler-cfg MODEL [--expect FILE]  (25 steps, cfg 0.5; :3405)
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
               "       --test-cfm-euler-cfg MODEL [--expect FILE] | --decode MODEL T P [--cfm_steps N] [--cfg R]\n"
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
