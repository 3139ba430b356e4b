// engine.h -- host-side engine of the HIP DiT-CFM decoder: resident weights,
// workspace, kernel sequences for one estimator forward and for a whole Euler
// decode (captured once per shape as a hipGraph and replayed).
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "device_common.h"

namespace mit2hip {

struct HipError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// One named host tensor handed to the engine (f32 or f16 payload).
struct HostTensor {
  std::string name;
  const void* data = nullptr;
  uint64_t elems = 0;
  int dtype = 0;  // 0 = f32, 1 = f16
};

// Device arena: one hipMalloc, bump-allocated, 256-byte aligned slices.
class Arena {
 public:
  Arena() = default;
  ~Arena();
  Arena(const Arena&) = delete;
  Arena& operator=(const Arena&) = delete;
  void reserve(size_t bytes);  // frees any previous block
  void* take(size_t bytes);
  size_t used() const { return used_; }
  size_t capacity() const { return cap_; }
  char* base() const { return base_; }
  // Makes the first `bytes` bytes taken (for an arena filled by a bulk copy).
  void set_used(size_t bytes) { used_ = bytes; }

 private:
  char* base_ = nullptr;
  size_t cap_ = 0;
  size_t used_ = 0;
};

struct Weights;    // resident weights (engine.hip)
struct Workspace;  // activations (engine.hip)
class Vocoder;     // BigVGAN (vocoder.hip)
class GptDecoder;  // GPT mel-code decoder (gpt.hip)

// Device buffers of the timestep-conditioning tables for S step slots:
// t values, their embeddings and MLP intermediates, the per-step table rows
// (kTcondPerStep floats each) and the folded-norm column biases.
struct TableBufs {
  float* tvals = nullptr;  // [S]
  float* temb = nullptr;   // [S][256]
  float* th = nullptr;     // [S][512]
  float* t1 = nullptr;     // [S][512]
  float* t2 = nullptr;     // [S][512]
  float* tab = nullptr;    // [S][36864]
  float* nbq = nullptr;    // [S][13][1536]
  float* nbw = nullptr;    // [S][13][3072]
};

class Engine {
 public:
  Engine(const std::vector<HostTensor>& tensors, int device);
  // From a device image written by write_image: the prepared weights (weight
  // norm folded, rows permuted, taps laid out, f16) are copied to the device
  // as they are, with no host-side preparation.
  Engine(const std::string& image_path, int device);
  ~Engine();

  // Writes the prepared device weights (the decoder's, and the length
  // regulator's and vocoder's when present) to an image file.
  void write_image(const std::string& path) const;

  int device() const { return device_; }
  hipStream_t stream() const { return stream_; }
  size_t weight_bytes() const;

  // Full CFG Euler decode (run_cfm_euler_cpu semantics), nreq independent
  // requests padded to T tokens.  All pointers are DEVICE pointers:
  //   x0, prompt: [nreq][T][80]; cond: [nreq][T][512]; style: [nreq][192];
  //   valid_T, P: per-request valid length and prompt length (host arrays);
  //   x_out: [nreq][T][80]; vtrace (optional): [steps][nreq][T][80].
  // Enqueues on stream(); does not synchronise.
  void decode_device(const float* x0, const float* prompt, const float* cond, const float* style,
                     int nreq, int T, const uint32_t* valid_T, const uint32_t* P, int steps,
                     float cfg, float* x_out, float* vtrace);

  // One estimator forward for B independent branches (run_dit_estimator_step_cpu
  // semantics) on DEVICE pointers: x, prompt_x [B][T][80], cond [B][T][512],
  // style [B][192], mask [B][T]; dphi [B][T][80].  Synchronous.
  void estimator_step_device(const float* x, const float* prompt_x, const float* cond,
                             const float* style, const uint32_t* mask, float t, int B, int T,
                             float* dphi);

  // ---- stage entry points (host pointers, synchronous), one per reference
  // CPU stage, used by the parity tests.  rows = B*T.
  void stage_timestep_embedder(float t, int which, float* out512);
  void stage_input_merge(const float* x, const float* prompt_x, const float* cond,
                         const float* style, int B, int T, float* out);
  void stage_adaptive_norm(const float* in, const float* t1, int rows, int norm_id, float* out);
  void stage_attention_core(const float* in, const uint32_t* mask, int B, int T, int layer,
                            float* out);
  void stage_feed_forward(const float* in, int rows, int layer, float* out);
  void stage_block(const float* in, const float* t1, const uint32_t* mask, int B, int T,
                   int layer, const float* skip, float* out);
  void stage_stack(const float* in, const float* t1, const uint32_t* mask, int B, int T,
                   float* out);
  void stage_post(const float* xres, const float* xmel, int rows, float* long_skip, float* conv1,
                  float* res_proj);
  void stage_wavenet(const float* in, const float* t2, const uint32_t* mask, int B, int T,
                     float* out);
  void stage_final_layer(const float* in, const float* t1, int rows, float* out);
  // Plain MFMA GEMM on f16-rounded operands: out[M][N] = A . W^T + bias.
  void op_linear(const float* A, const float* W, const float* bias, int M, int N, int K,
                 float* out);

  // Enqueues `count` launches of one decode kernel at the shape of the last
  // decode (its workspace contents as operands), on stream(), without
  // synchronising; returns the kernel's algorithmic flops and HBM bytes per
  // launch.  A measurement hook: kernel ids are listed in mit2cfm.h.
  void profile_launch(int kernel, int count, double* flops, double* bytes, std::string* name);

  // ---- condition and noise producer (the step before the decode).
  bool has_length_regulator() const;
  // run_length_regulator_full (gpt.cpp:5298/5313) on DEVICE pointers:
  // s_infer [in_tokens][1024] fp32 -> out [out_tokens][512] fp32.  Enqueued
  // on stream(), not synchronised.
  void length_regulator_device(const float* s_infer, int in_tokens, int out_tokens, float* out);
  // The decode condition (synthesis_pipeline.cpp:1027-1035): generated =
  // floor(codes * 1.72f) frames; cond [prompt_tokens + generated][512] =
  // [prompt_cond rows 0..prompt_tokens-1 ; length_regulator(s_infer)].
  // DEVICE pointers, enqueued on stream(); returns generated.
  int condition_device(const float* s_infer, int codes, const float* prompt_cond,
                       int prompt_tokens, float* cond);
  // condition_device with every scratch buffer taken from the library's
  // static per-GPU scratch array instead of the context's workspace: it
  // allocates nothing, for callers that cannot (graph capture, serving
  // loops).  codes <= kNoAllocMaxCodes; calls that overlap on one GPU race.
  int condition_device_noalloc(const float* s_infer, int codes, const float* prompt_cond,
                               int prompt_tokens, float* cond);
  static constexpr int kNoAllocMaxCodes = 1024;
  // Host-pointer versions of the two above (synchronous).
  void length_regulator_host(const float* s_infer, int in_tokens, int out_tokens, float* out);
  int condition_host(const float* s_infer, int codes, const float* prompt_cond,
                     int prompt_tokens, float* cond);
  // make_deterministic_normal_noise (tokenizer_tests.cpp:2121) into a DEVICE
  // buffer of n floats, on stream().
  void normal_noise_device(size_t n, uint64_t seed, float temperature, float* out);
  // Frames the condition producer makes from `codes` semantic tokens.
  static int generated_frames(int codes);

  // ---- BigVGAN vocoder (the consumer of the mel), present when the tensor
  // table holds the "bigvgan.*" weights.
  bool has_vocoder() const { return voc_ != nullptr; }
  // mel [tokens][80] -> wav [256 tokens], DEVICE pointers, on stream().
  void vocode_device(const float* mel, int tokens, float* wav);
  // Host-pointer version (synchronous).
  void vocode_host(const float* mel, int tokens, float* wav);
  // One vocoder stage on host pointers (stage ids in vocoder.h); returns the
  // output floats written.
  size_t vocoder_stage_host(int stage, int index, const float* in, int tokens, float* out);

  // ---- the whole acoustic stage on the device (synthesis_pipeline.cpp:
  // build_hot_codes_condition_inputs_shared :1012-1035, the seeded noise :1333,
  // synthesize_hot_condition_vectors_wav_shared :1038-1097): condition from
  // s_infer [codes][1024] and the voice's prompt_cond rows, x0 =
  // make_deterministic_normal_noise(T, 80, seed, temperature), the CFG decode
  // with the voice's prompt_mel [P][80] (token-major) and style [192], then the
  // vocoder on the generated rows.  DEVICE pointers; wav [256 * generated];
  // mel (optional) receives the full decoded mel [T][80].  Enqueued on
  // stream(); returns generated.
  int acoustic_device(const float* s_infer, int codes, const float* prompt_cond,
                      const float* prompt_mel, int prompt_tokens, const float* style,
                      uint64_t seed, float temperature, int steps, float cfg, float* wav,
                      float* mel);

  // ---- GPT mel-code decoder (the producer of the semantic codes), present
  // when the tensor table holds the "gpt.gpt.h.*" weights.  gpt() makes the
  // context's device current and throws when the decoder is absent.
  bool has_gpt() const { return gpt_ != nullptr; }
  GptDecoder& gpt();

  // Graph replay on/off (default on; env MIT2CFM_GRAPH=0 turns it off).
  void set_use_graph(bool on) { use_graph_ = on; }
  // Padded rows of a ragged multi-request decode: computed (default; the
  // masked estimator at the padded length), or skipped -- every product,
  // and the attention's query blocks, stop two rows past each request's
  // valid length, and the rest of the padded rows' outputs are unspecified.
  void set_skip_padding(bool on) { skip_padding_ = on; }
  bool skip_padding() const { return skip_padding_; }
  // Arithmetic of the stages the reference runs in fp32 (the length
  // regulator, stage 1; the vocoder, stage 2): f32 = true (default) runs
  // their GEMMs on split f16 operand pairs (fp32-level products), false on
  // plain f16 operands.
  void set_f32(int stage, bool f32);
  bool f32(int stage) const;
  void sync();

 private:
  void ensure_workspace(int B, int T, int S, int nreq);
  void ensure_rope(int T);
  void enqueue_tables(const TableBufs& tb, int S);
  void enqueue_norm_bias(const TableBufs& tb, int S);
  const TableBufs& decode_tables(int steps);
  void enqueue_layer(int l, int B, int T, const float* tab, const float* nbq, const float* nbw,
                     float* cur, float* hbuf, const half_t* skip16, half_t* out16,
                     bool skip_in_done = false, const half_t* next_skip16 = nullptr);
  void enqueue_transformer(int B, int T, const float* tab, const float* nbq, const float* nbw);
  void enqueue_estimator(int B, int T, const float* tab, const float* nbq, const float* nbw);
  void enqueue_decode(const float* x0, const float* prompt, const float* cond, const float* style,
                      int nreq, int T, int steps, float cfg, float* vtrace, const TableBufs& tb);
  void upload_stage_tables(const float* t1_host, const float* t2_host);

  int device_ = 0;
  int last_B_ = 0, last_T_ = 0;
  bool lr_f32_ = true;
  hipStream_t stream_ = nullptr;
  bool use_graph_ = true;
  // Set while a decode of a batch with a request shorter than T is enqueued:
  // its attention launches skip each branch's fully masked key tiles.
  bool branch_keys_ = false;
  bool skip_padding_ = false;
  // Set while a decode with skipped padding is enqueued: each branch's
  // needed rows (valid length + 2, at most T).
  RowSkip row_skip_;
  std::unique_ptr<Weights> w_;
  std::unique_ptr<Workspace> ws_;
  std::unique_ptr<Vocoder> voc_;
  std::unique_ptr<GptDecoder> gpt_;
  float* voc_io_ = nullptr;  // host-path staging: mel, then wav
  size_t voc_io_floats_ = 0;
  // Acoustic-stage buffers (condition [T][512], x0 and mel [T][80]), grown on
  // demand and kept, so the decode graphs captured on them stay valid.
  Arena ac_;
  int ac_cap_ = 0;
  float *ac_cond_ = nullptr, *ac_x0_ = nullptr, *ac_mel_ = nullptr;
  // Length-regulator buffers, grown on demand (separate from the decode's
  // workspace so a condition call never invalidates captured decode graphs).
  struct LrBufs {
    Arena arena;
    int cap_in = 0, cap_out = 0;
    float* in32;   // [cap_in][1024]  host staging
    half_t* s16;   // [cap_in][1024]
    half_t* p16;   // [cap_in][512]   content_in_proj output
    half_t* x16;   // [cap_out + 1][512] conv operand (last used row all zero)
    float* y32;    // [cap_out][512]  conv output
    float* sum_p;  // [cap_out][16]   per-row partial sums
    float* ssq_p;  // [cap_out][16]   per-row partial sums of squares
    float* out32;  // [cap_out + prompt][512] host staging of the result
    int cap_cond = 0;
  };
  LrBufs lr_;
  void ensure_lr(int in_tokens, int out_tokens, int cond_rows);
  // The length regulator's device buffers (split operand pairs: lo halves at
  // + cap_in * 1024, + cap_in * 512 and + (cap_out + 1) * 512 elements).
  struct LrView {
    half_t* s16;
    half_t* p16;
    half_t* x16;
    float* y32;
    float* sum_p;
    float* ssq_p;
    int cap_in, cap_out;
  };
  void length_regulator_on(const LrView& v, const float* s_infer, int in_tokens, int out_tokens,
                           float* out);
  // Decode tables per step count, computed once per context (decode_tables).
  struct TableSet {
    Arena arena;
    TableBufs bufs;
  };
  std::map<int, std::unique_ptr<TableSet>> table_cache_;
  struct GraphEntry {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t last_use = 0;  // use_tick_ of the latest launch
  };
  // Captured whole-decode graphs, least recently used evicted past
  // kMaxGraphs.  key: nreq, T, steps, cfg bits, vtrace ptr, io pointers,
  // whether some request is shorter than T, whether its padding is skipped.
  std::map<std::tuple<int, int, int, uint32_t, const void*, const void*, const void*, const void*,
                      const void*, const void*, bool, bool>,
           GraphEntry>
      graphs_;
  uint64_t use_tick_ = 0;
  void clear_graphs();
  // Captured condition-producer graphs (condition_device and
  // length_regulator_device).  key: input tokens, output tokens, prompt
  // rows, s_infer, prompt and output pointers, f32 mode.  Dropped when the
  // regulator's buffers grow.
  std::map<std::tuple<int, int, int, const void*, const void*, const void*, bool>, GraphEntry>
      cond_graphs_;
  // Enqueues `enqueue`'s launches on stream_ as a replay of the graph cached
  // in `graphs` under `key`, capturing it first when there is none (the least
  // recently used graph evicted past kMaxGraphs).  With graphs off, or while
  // stream_ is being captured by the caller, the launches are enqueued
  // directly.
  template <typename Key, typename F>
  void run_graph(std::map<Key, GraphEntry>& graphs, const Key& key, F&& enqueue);
  template <typename Map>
  static void destroy_graphs(Map& graphs);

 public:
  static constexpr size_t kMaxGraphs = 8;
  size_t graph_count() const { return graphs_.size(); }
};

}  // namespace mit2hip
