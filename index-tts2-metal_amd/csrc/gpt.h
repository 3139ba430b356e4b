// gpt.h -- the GPT mel-code decoder of IndexTTS2 on the GPU: a 24-layer
// GPT-2 stack (width 1280, 20 heads of 64, MLP 5120 with gelu_new) that
// turns a conditioning prefix into mel codes, one token per step, with a
// key/value cache (runtime/impl/gpt.cpp: run_gpt_kv_greedy_cpu :1877 and
// run_gpt_kv_greedy_metal :1914, run_gpt_cached_decode_cpu :1400).
//
// A decode step reads every weight once (about 0.98 GB of f16), so it is a
// chain of HBM-bound matrix-vector products; see gpt.hip for the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace mit2hip {

class GptDecoder {
 public:
  static constexpr int kWidth = 1280;
  static constexpr int kVocab = 8194;
  static constexpr int kPositions = 1818;  // rows of the mel position table
  static constexpr uint32_t kStartToken = 8192;
  static constexpr uint32_t kStopToken = 8193;

  // Tensors named "gpt.gpt.h.<l>.*", "gpt.gpt.ln_f.*", "gpt.final_norm.*",
  // "gpt.mel_head.*", "gpt.mel_embedding.weight" and
  // "gpt.mel_pos_embedding.emb.weight" (fp32 on the host, checkpoint
  // layouts: the Conv1D matrices are [in][out]).  Layers 0..L-1 must all be
  // present (the checkpoint has 24); throws std::invalid_argument otherwise.
  GptDecoder(const std::unordered_map<std::string, std::vector<float>>& t, hipStream_t stream);
  // From the GPT section of a device image (see append_image).
  GptDecoder(const uint8_t* image, size_t bytes, hipStream_t stream);
  // Appends the prepared weights (arena bytes and layout) to an image.
  void append_image(std::vector<uint8_t>& out) const;
  ~GptDecoder();
  GptDecoder(const GptDecoder&) = delete;
  GptDecoder& operator=(const GptDecoder&) = delete;

  // True when any GPT decoder tensor ("gpt.gpt.h.*") is present.
  static bool present(const std::unordered_map<std::string, std::vector<float>>& t);
  size_t weight_bytes() const;
  int layers() const;

  struct Greedy {
    std::vector<uint32_t> predicted;     // one per step taken (the stop token included)
    std::vector<uint32_t> input_tokens;  // start token, then every non-stop prediction
    std::vector<float> last_logits;      // [8194] logits of the last step taken
    std::vector<float> last_processed_logits;  // [8194] after the sampling processors (greedy: = last_logits)
    int32_t first_stop_step = -1;
    double prefill_ms = 0, decode_ms = 0;  // device time of the two phases
  };

  // run_gpt_kv_greedy (gpt.cpp:1877): prefix HOST rows [prefix_tokens][1280];
  // greedy decode of up to `steps` tokens, stopping at the first stop token.
  // Positions follow gpt_cached_generate_position (gpt.cpp:1873).
  void kv_greedy(const float* prefix, int prefix_tokens, int steps, bool hf_generate_positions,
                 Greedy& out);

  // GptSamplingConfig (gpt.cpp:1592-1599) with do_sample set.
  struct Sampling {
    uint64_t seed = 0;
    float temperature = 1.0f;
    uint32_t top_k = 0;  // 0: off
    float top_p = 1.0f;
    float repetition_penalty = 1.0f;
    // repetition_history_prefix (gpt.cpp:1918, :2224-2229): when given
    // (non-NULL, even with n_history 0), the repetition-penalty history is
    // these tokens followed by the predictions so far, instead of the start
    // token followed by them.  Host array.
    const uint32_t* history = nullptr;
    uint32_t n_history = 0;
  };
  static constexpr uint32_t kMaxHistory = 8192;  // history-prefix tokens one call may pass
  // The sampled loop (run_gpt_kv_greedy_metal with do_sample, gpt.cpp:
  // 2221-2240): each step's logits go through the sampling processors over
  // the history ([start token] or the caller's prefix, then the predictions
  // so far) and one splitmix64 draw (seeded once per call) picks the token.
  // Throws std::invalid_argument for the settings the reference rejects.
  void kv_sample(const float* prefix, int prefix_tokens, int steps, bool hf_generate_positions,
                 const Sampling& sampling, Greedy& out);

  // run_gpt_cached_decode (gpt.cpp:1400): HOST rows [prefix_tokens + 1][1280];
  // the last row is decoded against the caches of the others.  Outputs (host,
  // any may be null): ln_f [1280], final_norm [1280], logits [8194].  Returns
  // the argmax of the logits.
  uint32_t cached_decode(const float* rows, int prefix_tokens, float* ln_f, float* final_norm,
                         float* logits);

  // Launches one of the decode step's kernels `launches` times on the stream
  // (for timing): 0 = c_attn (3840 x 1280), 1 = attn c_proj (1280 x 1280),
  // 2 = c_fc (5120 x 1280), 3 = mlp c_proj (1280 x 5120), 4 = mel_head
  // (8194 x 1280), 5 = cached attention at 1024 keys.  Returns the kernel's
  // name; *bytes = its algorithmic HBM bytes per launch.
  const char* profile_launch(int kernel, int launches, double* bytes);

  struct Impl;

 private:
  void generate(const float* prefix, int prefix_tokens, int steps, bool hf, const Sampling* sampling, Greedy& out);
  Impl* d_;
};

}  // namespace mit2hip
