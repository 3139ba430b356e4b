// api.hip -- extern "C" boundary (include/mit2cfm.h) over the HIP engine.
// No exception crosses the boundary: every entry point catches, records the
// message on the context (or thread-locally) and returns a status code.
#include "../../include/mit2cfm.h"

#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../runtime/bundle.h"
#include "../runtime/synth.h"
#include "engine.h"
#include "gpt.h"
#include "vocoder.h"

struct mit2cfm_ctx {
  std::unique_ptr<mit2hip::Engine> eng;
  std::string err;
  // device staging for the host-pointer decode entry points
  void* io = nullptr;
  size_t io_bytes = 0;
};

namespace {

thread_local std::string g_err;

mit2cfm_status fail(mit2cfm_ctx* ctx, mit2cfm_status code, const std::string& msg) {
  if (ctx)
    ctx->err = msg;
  else
    g_err = msg;
  return code;
}

template <typename F>
mit2cfm_status guarded(mit2cfm_ctx* ctx, F&& f) {
  try {
    f();
    return MIT2CFM_OK;
  } catch (const std::invalid_argument& e) {
    return fail(ctx, MIT2CFM_E_ARG, e.what());
  } catch (const mit2hip::HipError& e) {
    return fail(ctx, MIT2CFM_E_HIP, e.what());
  } catch (const std::out_of_range& e) {
    return fail(ctx, MIT2CFM_E_ARG, e.what());
  } catch (const std::runtime_error& e) {
    return fail(ctx, MIT2CFM_E_MODEL, e.what());
  } catch (const std::exception& e) {
    return fail(ctx, MIT2CFM_E_INTERNAL, e.what());
  } catch (...) {
    return fail(ctx, MIT2CFM_E_INTERNAL, "unknown error");
  }
}

void require(bool ok, const char* msg) {
  if (!ok) throw std::invalid_argument(msg);
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw mit2hip::HipError(std::string(what) + ": " + hipGetErrorString(e));
}

mit2cfm_status make_ctx(const std::vector<mit2hip::HostTensor>& ts, int32_t device,
                        mit2cfm_ctx** out) {
  if (!out) return fail(nullptr, MIT2CFM_E_ARG, "out must not be NULL");
  *out = nullptr;
  auto* c = new mit2cfm_ctx();
  const mit2cfm_status st = guarded(nullptr, [&] {
    int n = 0;
    hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (device < 0 || device >= n)
      throw mit2hip::HipError("HIP device " + std::to_string(device) + " not available (" +
                              std::to_string(n) + " devices)");
    c->eng = std::make_unique<mit2hip::Engine>(ts, device);
  });
  if (st != MIT2CFM_OK) {
    delete c;
    return st;
  }
  *out = c;
  return MIT2CFM_OK;
}

// Device staging buffer of the context, grown on demand.
float* staging(mit2cfm_ctx* c, size_t floats) {
  const size_t bytes = floats * sizeof(float);
  if (bytes > c->io_bytes) {
    if (c->io) hip_check(hipFree(c->io), "hipFree");
    c->io = nullptr;
    c->io_bytes = 0;
    hip_check(hipMalloc(&c->io, bytes), "hipMalloc");
    c->io_bytes = bytes;
  }
  return static_cast<float*>(c->io);
}

// Host-pointer decode for nreq padded requests (x0/prompt/x_out [nreq][T][80]).
void host_decode(mit2cfm_ctx* c, uint32_t nreq, uint32_t T, const uint32_t* valid,
                 const uint32_t* P, const float* x0, const float* prompt, const float* cond,
                 const float* style, uint32_t steps, float cfg, float* x_out, float* v_trace) {
  const size_t nx = (size_t)nreq * T * 80;
  const size_t nc = (size_t)nreq * T * 512;
  const size_t ns = (size_t)nreq * 192;
  const size_t nv = v_trace ? nx * steps : 0;
  float* base = staging(c, 3 * nx + nc + ns + nv);
  float* d_x0 = base;
  float* d_prompt = d_x0 + nx;
  float* d_cond = d_prompt + nx;
  float* d_style = d_cond + nc;
  float* d_out = d_style + ns;
  float* d_v = v_trace ? d_out + nx : nullptr;
  hipStream_t s = c->eng->stream();
  hip_check(hipMemcpyAsync(d_x0, x0, nx * 4, hipMemcpyHostToDevice, s), "copy x0");
  hip_check(hipMemcpyAsync(d_prompt, prompt, nx * 4, hipMemcpyHostToDevice, s), "copy prompt");
  hip_check(hipMemcpyAsync(d_cond, cond, nc * 4, hipMemcpyHostToDevice, s), "copy cond");
  hip_check(hipMemcpyAsync(d_style, style, ns * 4, hipMemcpyHostToDevice, s), "copy style");
  c->eng->decode_device(d_x0, d_prompt, d_cond, d_style, (int)nreq, (int)T, valid, P, (int)steps,
                        cfg, d_out, d_v);
  hip_check(hipMemcpyAsync(x_out, d_out, nx * 4, hipMemcpyDeviceToHost, s), "copy x_out");
  if (v_trace) hip_check(hipMemcpyAsync(v_trace, d_v, nv * 4, hipMemcpyDeviceToHost, s), "copy v");
  c->eng->sync();
}

// Packs a single request's [P][80] prompt into [T][80].
std::vector<float> pad_prompt(const float* prompt, uint32_t T, uint32_t P) {
  std::vector<float> p((size_t)T * 80, 0.0f);
  if (P) std::memcpy(p.data(), prompt, (size_t)P * 80 * 4);
  return p;
}

}  // namespace

extern "C" {

int32_t mit2cfm_abi_version(void) { return MIT2CFM_ABI_VERSION; }

const char* mit2cfm_last_error(const mit2cfm_ctx* ctx) {
  return ctx ? ctx->err.c_str() : g_err.c_str();
}

mit2cfm_status mit2cfm_create(const mit2cfm_tensor* tensors, uint32_t count, int32_t device,
                              mit2cfm_ctx** out) {
  if (!tensors && count) return fail(nullptr, MIT2CFM_E_ARG, "tensors must not be NULL");
  std::vector<mit2hip::HostTensor> ts;
  for (uint32_t i = 0; i < count; ++i) {
    if (!tensors[i].name || !tensors[i].data)
      return fail(nullptr, MIT2CFM_E_ARG, "tensor " + std::to_string(i) + " has no name or data");
    ts.push_back({tensors[i].name, tensors[i].data, tensors[i].elems, tensors[i].dtype});
  }
  return make_ctx(ts, device, out);
}

}  // extern "C"

namespace {
// The bundle tensors a context uses: the DiT-CFM estimator, the length
// regulator, the vocoder and the GPT decoder (not the GPT's conditioning
// encoders, text embedding or emotion layers).
bool wanted_bundle_tensor(const std::string& n) {
  static const char* const prefixes[] = {"s2mel.net.cfm.estimator.", "s2mel.net.length_regulator.",
                                         "bigvgan.", "gpt.gpt.h.", "gpt.gpt.ln_f.", "gpt.final_norm.",
                                         "gpt.mel_head.", "gpt.mel_embedding.", "gpt.mel_pos_embedding."};
  for (const char* p : prefixes)
    if (n.rfind(p, 0) == 0) return true;
  return false;
}
}  // namespace

extern "C" {

mit2cfm_status mit2cfm_create_from_bundle(const char* bundle_path, int32_t device,
                                          mit2cfm_ctx** out) {
  if (!bundle_path || !out) return fail(nullptr, MIT2CFM_E_ARG, "bundle_path/out must not be NULL");
  std::unique_ptr<mit2::Bundle> b;
  const mit2cfm_status st = guarded(nullptr, [&] { b = std::make_unique<mit2::Bundle>(bundle_path); });
  if (st != MIT2CFM_OK) return st;
  std::vector<mit2hip::HostTensor> ts;
  for (const auto& info : b->tensors()) {
    if (!wanted_bundle_tensor(info.name)) continue;
    int dt;
    if (info.dtype == "f32")
      dt = 0;
    else if (info.dtype == "f16")
      dt = 1;
    else
      continue;
    ts.push_back({info.name, b->tensor_data(info), info.nbytes / (dt ? 2 : 4), dt});
  }
  return make_ctx(ts, device, out);
}

mit2cfm_status mit2cfm_create_synthetic(uint64_t base_seed, float stddev, int32_t device,
                                        mit2cfm_ctx** out) {
  std::vector<std::vector<uint8_t>> bufs;
  std::vector<mit2hip::HostTensor> ts;
  const mit2cfm_status st = guarded(nullptr, [&] {
    const auto& specs = mit2::estimator_tensor_specs();
    bufs.reserve(specs.size());
    for (size_t i = 0; i < specs.size(); ++i) {
      bufs.push_back(mit2::synth_tensor_bytes(i, base_seed, stddev));
      const bool f16 = specs[i].dtype == "f16";
      ts.push_back({specs[i].name, bufs.back().data(), bufs.back().size() / (f16 ? 2 : 4),
                    f16 ? 1 : 0});
    }
  });
  if (st != MIT2CFM_OK) return st;
  return make_ctx(ts, device, out);
}

}  // extern "C"

namespace {
const std::vector<mit2::SynthSpec>* synth_set(int32_t set) {
  switch (set) {
    case MIT2CFM_SYNTH_ESTIMATOR: return &mit2::estimator_tensor_specs();
    case MIT2CFM_SYNTH_LENGTH_REGULATOR: return &mit2::length_regulator_tensor_specs();
    case MIT2CFM_SYNTH_BIGVGAN: return &mit2::bigvgan_tensor_specs();
    case MIT2CFM_SYNTH_GPT: return &mit2::gpt_tensor_specs();
    default: return nullptr;
  }
}
std::vector<uint8_t> synth_set_bytes(int32_t set, size_t i, uint64_t base_seed, float stddev) {
  if (set == MIT2CFM_SYNTH_ESTIMATOR) return mit2::synth_tensor_bytes(i, base_seed, stddev);
  if (set == MIT2CFM_SYNTH_LENGTH_REGULATOR) return mit2::synth_lr_tensor_bytes(i, base_seed, stddev);
  if (set == MIT2CFM_SYNTH_GPT) return mit2::synth_gpt_tensor_bytes(i, base_seed, stddev);
  return mit2::synth_bigvgan_tensor_bytes(i, base_seed, stddev);
}
}  // namespace

extern "C" {

mit2cfm_status mit2cfm_create_synthetic_acoustic(uint64_t base_seed, float stddev, int32_t device,
                                                 mit2cfm_ctx** out) {
  std::vector<std::vector<uint8_t>> bufs;
  std::vector<mit2hip::HostTensor> ts;
  const mit2cfm_status st = guarded(nullptr, [&] {
    for (int32_t set = MIT2CFM_SYNTH_ESTIMATOR; set <= MIT2CFM_SYNTH_BIGVGAN; ++set) {
      const auto& specs = *synth_set(set);
      bufs.reserve(bufs.size() + specs.size());
      for (size_t i = 0; i < specs.size(); ++i) {
        bufs.push_back(synth_set_bytes(set, i, base_seed + (uint64_t)set, stddev));
        const bool f16 = specs[i].dtype == "f16";
        ts.push_back({specs[i].name, bufs.back().data(), bufs.back().size() / (f16 ? 2 : 4), f16 ? 1 : 0});
      }
    }
  });
  if (st != MIT2CFM_OK) return st;
  return make_ctx(ts, device, out);
}

mit2cfm_status mit2cfm_write_image(mit2cfm_ctx* ctx, const char* path) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(path != nullptr, "path must not be NULL");
    ctx->eng->write_image(path);
  });
}

mit2cfm_status mit2cfm_create_from_image(const char* path, int32_t device, mit2cfm_ctx** out) {
  if (!path || !out) return fail(nullptr, MIT2CFM_E_ARG, "path/out must not be NULL");
  *out = nullptr;
  auto* c = new mit2cfm_ctx();
  const mit2cfm_status st = guarded(nullptr, [&] {
    int n = 0;
    hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (device < 0 || device >= n)
      throw mit2hip::HipError("HIP device " + std::to_string(device) + " not available (" +
                              std::to_string(n) + " devices)");
    c->eng = std::make_unique<mit2hip::Engine>(std::string(path), device);
  });
  if (st != MIT2CFM_OK) {
    delete c;
    return st;
  }
  *out = c;
  return MIT2CFM_OK;
}

void mit2cfm_destroy(mit2cfm_ctx* ctx) {
  if (!ctx) return;
  try {
    if (ctx->io) (void)hipFree(ctx->io);
    ctx->eng.reset();
  } catch (...) {
  }
  delete ctx;
}

mit2cfm_status mit2cfm_decode(mit2cfm_ctx* ctx, const float* x0, const float* prompt,
                              const float* cond, const float* style, uint32_t tokens,
                              uint32_t prompt_tokens, uint32_t steps, float cfg_rate,
                              float* x_out) {
  return mit2cfm_decode_trace(ctx, x0, prompt, cond, style, tokens, prompt_tokens, steps, cfg_rate,
                              x_out, nullptr);
}

mit2cfm_status mit2cfm_decode_trace(mit2cfm_ctx* ctx, const float* x0, const float* prompt,
                                    const float* cond, const float* style, uint32_t tokens,
                                    uint32_t prompt_tokens, uint32_t steps, float cfg_rate,
                                    float* x_out, float* v_trace) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(x0 && cond && style && x_out, "x0, cond, style and x_out must not be NULL");
    require(prompt || prompt_tokens == 0, "prompt must not be NULL when prompt_tokens > 0");
    require(tokens > 0 && prompt_tokens <= tokens, "need 0 < tokens and prompt_tokens <= tokens");
    const auto p = pad_prompt(prompt, tokens, prompt_tokens);
    host_decode(ctx, 1, tokens, &tokens, &prompt_tokens, x0, p.data(), cond, style, steps,
                cfg_rate, x_out, v_trace);
  });
}

mit2cfm_status mit2cfm_decode_device(mit2cfm_ctx* ctx, const float* x0, const float* prompt,
                                     const float* cond, const float* style, uint32_t tokens,
                                     uint32_t prompt_tokens, uint32_t steps, float cfg_rate,
                                     float* x_out, uint32_t flags) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(x0 && cond && style && x_out, "x0, cond, style and x_out must not be NULL");
    require(prompt || prompt_tokens == 0, "prompt must not be NULL when prompt_tokens > 0");
    require(tokens > 0 && prompt_tokens <= tokens, "need 0 < tokens and prompt_tokens <= tokens");
    ctx->eng->decode_device(x0, prompt ? prompt : x0, cond, style, 1, (int)tokens, &tokens,
                            &prompt_tokens, (int)steps, cfg_rate, x_out, nullptr);
    if (flags & MIT2CFM_FLAG_SYNC) ctx->eng->sync();
  });
}

mit2cfm_status mit2cfm_decode_batched(mit2cfm_ctx* ctx, uint32_t nreq, uint32_t t_max,
                                      const uint32_t* tokens, const uint32_t* prompt_tokens,
                                      const float* x0, const float* prompt, const float* cond,
                                      const float* style, uint32_t steps, float cfg_rate,
                                      float* x_out) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(nreq > 0 && t_max > 0, "nreq and t_max must be positive");
    require(tokens && prompt_tokens && x0 && prompt && cond && style && x_out,
            "pointer arguments must not be NULL");
    host_decode(ctx, nreq, t_max, tokens, prompt_tokens, x0, prompt, cond, style, steps, cfg_rate,
                x_out, nullptr);
  });
}

mit2cfm_status mit2cfm_decode_batched_device(mit2cfm_ctx* ctx, uint32_t nreq, uint32_t t_max,
                                             const uint32_t* tokens, const uint32_t* prompt_tokens,
                                             const float* x0, const float* prompt, const float* cond,
                                             const float* style, uint32_t steps, float cfg_rate,
                                             float* x_out, uint32_t flags) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(nreq > 0 && t_max > 0, "nreq and t_max must be positive");
    require(tokens && prompt_tokens && x0 && prompt && cond && style && x_out,
            "pointer arguments must not be NULL");
    ctx->eng->decode_device(x0, prompt, cond, style, (int)nreq, (int)t_max, tokens, prompt_tokens,
                            (int)steps, cfg_rate, x_out, nullptr);
    if (flags & MIT2CFM_FLAG_SYNC) ctx->eng->sync();
  });
}

mit2cfm_status mit2cfm_estimator_step(mit2cfm_ctx* ctx, const float* x, const float* prompt_x,
                                      const float* cond, const float* style,
                                      const uint32_t* key_mask, float t, uint32_t batch,
                                      uint32_t tokens, float* dphi_out) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(x && prompt_x && cond && style && key_mask && dphi_out,
            "pointer arguments must not be NULL");
    require(batch > 0 && tokens > 0, "batch and tokens must be positive");
    const size_t R = (size_t)batch * tokens;
    float* base = staging(ctx, R * 80 * 3 + R * 512 + (size_t)batch * 192 + R);
    float* d_x = base;
    float* d_p = d_x + R * 80;
    float* d_c = d_p + R * 80;
    float* d_s = d_c + R * 512;
    float* d_o = d_s + (size_t)batch * 192;
    uint32_t* d_m = reinterpret_cast<uint32_t*>(d_o + R * 80);
    hipStream_t s = ctx->eng->stream();
    hip_check(hipMemcpyAsync(d_x, x, R * 320, hipMemcpyHostToDevice, s), "copy x");
    hip_check(hipMemcpyAsync(d_p, prompt_x, R * 320, hipMemcpyHostToDevice, s), "copy prompt_x");
    hip_check(hipMemcpyAsync(d_c, cond, R * 2048, hipMemcpyHostToDevice, s), "copy cond");
    hip_check(hipMemcpyAsync(d_s, style, (size_t)batch * 768, hipMemcpyHostToDevice, s), "copy style");
    hip_check(hipMemcpyAsync(d_m, key_mask, R * 4, hipMemcpyHostToDevice, s), "copy mask");
    ctx->eng->estimator_step_device(d_x, d_p, d_c, d_s, d_m, t, (int)batch, (int)tokens, d_o);
    hip_check(hipMemcpyAsync(dphi_out, d_o, R * 320, hipMemcpyDeviceToHost, s), "copy dphi");
    ctx->eng->sync();
  });
}

void* mit2cfm_stream(mit2cfm_ctx* ctx) { return ctx && ctx->eng ? (void*)ctx->eng->stream() : nullptr; }

mit2cfm_status mit2cfm_synchronize(mit2cfm_ctx* ctx) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] { ctx->eng->sync(); });
}

mit2cfm_status mit2cfm_set_graph(mit2cfm_ctx* ctx, int32_t on) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  ctx->eng->set_use_graph(on != 0);
  return MIT2CFM_OK;
}

mit2cfm_status mit2cfm_set_padding(mit2cfm_ctx* ctx, int32_t mode) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  if (mode != MIT2CFM_PADDING_COMPUTE && mode != MIT2CFM_PADDING_SKIP)
    return fail(ctx, MIT2CFM_E_ARG, "padding mode must be MIT2CFM_PADDING_COMPUTE or MIT2CFM_PADDING_SKIP");
  ctx->eng->set_skip_padding(mode == MIT2CFM_PADDING_SKIP);
  return MIT2CFM_OK;
}

mit2cfm_status mit2cfm_get_padding(mit2cfm_ctx* ctx, int32_t* mode) {
  if (!ctx || !mode) return fail(ctx, MIT2CFM_E_ARG, "ctx and mode must not be NULL");
  *mode = ctx->eng->skip_padding() ? MIT2CFM_PADDING_SKIP : MIT2CFM_PADDING_COMPUTE;
  return MIT2CFM_OK;
}

mit2cfm_status mit2cfm_decode_graph_count(mit2cfm_ctx* ctx, uint32_t* count, uint32_t* capacity) {
  if (!ctx || !count) return fail(ctx, MIT2CFM_E_ARG, "ctx and count must not be NULL");
  *count = (uint32_t)ctx->eng->graph_count();
  if (capacity) *capacity = (uint32_t)mit2hip::Engine::kMaxGraphs;
  return MIT2CFM_OK;
}

mit2cfm_status mit2cfm_set_precision(mit2cfm_ctx* ctx, int32_t stage, int32_t mode) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  if (mode != MIT2CFM_PREC_F16 && mode != MIT2CFM_PREC_F32)
    return fail(ctx, MIT2CFM_E_ARG, "precision mode must be MIT2CFM_PREC_F16 or MIT2CFM_PREC_F32");
  if (stage == MIT2CFM_STAGE_LENGTH_REGULATOR && !ctx->eng->has_length_regulator())
    return fail(ctx, MIT2CFM_E_MODEL, "the context has no length-regulator tensors");
  if (stage == MIT2CFM_STAGE_VOCODER && !ctx->eng->has_vocoder())
    return fail(ctx, MIT2CFM_E_MODEL, "the context has no vocoder tensors");
  if (stage != MIT2CFM_STAGE_LENGTH_REGULATOR && stage != MIT2CFM_STAGE_VOCODER)
    return fail(ctx, MIT2CFM_E_ARG, "stage must be MIT2CFM_STAGE_LENGTH_REGULATOR or MIT2CFM_STAGE_VOCODER");
  return guarded(ctx, [&] { ctx->eng->set_f32(stage, mode == MIT2CFM_PREC_F32); });
}

mit2cfm_status mit2cfm_get_precision(mit2cfm_ctx* ctx, int32_t stage, int32_t* mode) {
  if (!ctx || !mode) return fail(ctx, MIT2CFM_E_ARG, "ctx and mode must not be NULL");
  if ((stage == MIT2CFM_STAGE_LENGTH_REGULATOR && !ctx->eng->has_length_regulator()) ||
      (stage == MIT2CFM_STAGE_VOCODER && !ctx->eng->has_vocoder()))
    return fail(ctx, MIT2CFM_E_MODEL, "the context has no tensors for that stage");
  if (stage != MIT2CFM_STAGE_LENGTH_REGULATOR && stage != MIT2CFM_STAGE_VOCODER)
    return fail(ctx, MIT2CFM_E_ARG, "stage must be MIT2CFM_STAGE_LENGTH_REGULATOR or MIT2CFM_STAGE_VOCODER");
  return guarded(ctx, [&] { *mode = ctx->eng->f32(stage) ? MIT2CFM_PREC_F32 : MIT2CFM_PREC_F16; });
}

mit2cfm_status mit2cfm_profile_launch(mit2cfm_ctx* ctx, int32_t kernel, uint32_t count,
                                      double* flops_per_launch, double* bytes_per_launch,
                                      const char** name) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    static thread_local std::string nm;
    ctx->eng->profile_launch(kernel, (int)count, flops_per_launch, bytes_per_launch, &nm);
    if (name) *name = nm.c_str();
  });
}

// ---- stages
#define STAGE_BODY(...)                                                   \
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL"); \
  return guarded(ctx, [&] { __VA_ARGS__; })

mit2cfm_status mit2cfm_stage_timestep_embedder(mit2cfm_ctx* ctx, float t, int32_t which,
                                               float* out512) {
  STAGE_BODY(require(out512 && (which == 1 || which == 2), "bad arguments");
             ctx->eng->stage_timestep_embedder(t, which, out512));
}

mit2cfm_status mit2cfm_stage_input_merge(mit2cfm_ctx* ctx, const float* x, const float* prompt_x,
                                         const float* cond, const float* style, uint32_t batch,
                                         uint32_t tokens, float* out) {
  STAGE_BODY(require(x && prompt_x && cond && style && out && batch && tokens, "bad arguments");
             ctx->eng->stage_input_merge(x, prompt_x, cond, style, (int)batch, (int)tokens, out));
}

mit2cfm_status mit2cfm_stage_adaptive_norm(mit2cfm_ctx* ctx, const float* in, const float* t1,
                                           uint32_t rows, int32_t norm_id, float* out) {
  STAGE_BODY(require(in && t1 && out && rows, "bad arguments");
             ctx->eng->stage_adaptive_norm(in, t1, (int)rows, norm_id, out));
}

mit2cfm_status mit2cfm_stage_attention_core(mit2cfm_ctx* ctx, const float* in,
                                            const uint32_t* key_mask, uint32_t batch,
                                            uint32_t tokens, int32_t layer, float* out) {
  STAGE_BODY(require(in && key_mask && out && batch && tokens, "bad arguments");
             ctx->eng->stage_attention_core(in, key_mask, (int)batch, (int)tokens, layer, out));
}

mit2cfm_status mit2cfm_stage_feed_forward(mit2cfm_ctx* ctx, const float* in, uint32_t rows,
                                          int32_t layer, float* out) {
  STAGE_BODY(require(in && out && rows, "bad arguments");
             ctx->eng->stage_feed_forward(in, (int)rows, layer, out));
}

mit2cfm_status mit2cfm_stage_block(mit2cfm_ctx* ctx, const float* in, const float* t1,
                                   const uint32_t* key_mask, uint32_t batch, uint32_t tokens,
                                   int32_t layer, const float* skip, float* out) {
  STAGE_BODY(require(in && t1 && key_mask && out && batch && tokens, "bad arguments");
             ctx->eng->stage_block(in, t1, key_mask, (int)batch, (int)tokens, layer, skip, out));
}

mit2cfm_status mit2cfm_stage_stack(mit2cfm_ctx* ctx, const float* in, const float* t1,
                                   const uint32_t* key_mask, uint32_t batch, uint32_t tokens,
                                   float* out) {
  STAGE_BODY(require(in && t1 && key_mask && out && batch && tokens, "bad arguments");
             ctx->eng->stage_stack(in, t1, key_mask, (int)batch, (int)tokens, out));
}

mit2cfm_status mit2cfm_stage_post(mit2cfm_ctx* ctx, const float* xres, const float* xmel,
                                  uint32_t rows, float* long_skip, float* conv1,
                                  float* res_proj) {
  STAGE_BODY(require(xres && xmel && long_skip && conv1 && res_proj && rows, "bad arguments");
             ctx->eng->stage_post(xres, xmel, (int)rows, long_skip, conv1, res_proj));
}

mit2cfm_status mit2cfm_stage_wavenet(mit2cfm_ctx* ctx, const float* in, const float* t2,
                                     const uint32_t* key_mask, uint32_t batch, uint32_t tokens,
                                     float* out) {
  STAGE_BODY(require(in && t2 && key_mask && out && batch && tokens, "bad arguments");
             ctx->eng->stage_wavenet(in, t2, key_mask, (int)batch, (int)tokens, out));
}

mit2cfm_status mit2cfm_stage_final_layer(mit2cfm_ctx* ctx, const float* in, const float* t1,
                                         uint32_t rows, float* out) {
  STAGE_BODY(require(in && t1 && out && rows, "bad arguments");
             ctx->eng->stage_final_layer(in, t1, (int)rows, out));
}

mit2cfm_status mit2cfm_op_linear(mit2cfm_ctx* ctx, const float* a, const float* w,
                                 const float* bias, uint32_t m, uint32_t n, uint32_t k,
                                 float* out) {
  STAGE_BODY(require(a && w && out, "bad arguments");
             ctx->eng->op_linear(a, w, bias, (int)m, (int)n, (int)k, out));
}

// ---- synthetic data
mit2cfm_status mit2cfm_normal_noise(uint32_t tokens, uint32_t channels, uint64_t seed,
                                    float temperature, float* out) {
  if (!out) return fail(nullptr, MIT2CFM_E_ARG, "out must not be NULL");
  return guarded(nullptr, [&] {
    const auto v = mit2::make_deterministic_normal_noise(tokens, channels, seed, temperature);
    std::memcpy(out, v.data(), v.size() * 4);
  });
}

uint32_t mit2cfm_synthetic_tensor_count(void) {
  return (uint32_t)mit2::estimator_tensor_specs().size();
}

mit2cfm_status mit2cfm_synthetic_tensor_info(uint32_t i, const char** name, uint32_t* ndim,
                                             int64_t* shape4, int32_t* dtype, uint64_t* elems) {
  const auto& specs = mit2::estimator_tensor_specs();
  if (i >= specs.size()) return fail(nullptr, MIT2CFM_E_ARG, "tensor index out of range");
  const auto& s = specs[i];
  if (name) *name = s.name.c_str();
  if (ndim) *ndim = (uint32_t)s.shape.size();
  uint64_t n = 1;
  for (size_t d = 0; d < s.shape.size(); ++d) {
    if (shape4 && d < 4) shape4[d] = s.shape[d];
    n *= (uint64_t)s.shape[d];
  }
  if (dtype) *dtype = s.dtype == "f16" ? MIT2CFM_DTYPE_F16 : MIT2CFM_DTYPE_F32;
  if (elems) *elems = n;
  return MIT2CFM_OK;
}

mit2cfm_status mit2cfm_synthetic_tensor_fill(uint32_t i, uint64_t base_seed, float stddev,
                                             void* out) {
  if (!out) return fail(nullptr, MIT2CFM_E_ARG, "out must not be NULL");
  return guarded(nullptr, [&] {
    const auto b = mit2::synth_tensor_bytes(i, base_seed, stddev);
    std::memcpy(out, b.data(), b.size());
  });
}


uint32_t mit2cfm_synthetic_set_count(int32_t set) {
  const auto* specs = synth_set(set);
  return specs ? (uint32_t)specs->size() : 0u;
}

mit2cfm_status mit2cfm_synthetic_set_info(int32_t set, uint32_t i, const char** name, uint32_t* ndim,
                                          int64_t* shape4, int32_t* dtype, uint64_t* elems) {
  const auto* specs = synth_set(set);
  if (!specs) return fail(nullptr, MIT2CFM_E_ARG, "unknown synthetic tensor set");
  if (i >= specs->size()) return fail(nullptr, MIT2CFM_E_ARG, "tensor index out of range");
  const auto& s = (*specs)[i];
  if (name) *name = s.name.c_str();
  if (ndim) *ndim = (uint32_t)s.shape.size();
  uint64_t n = 1;
  for (size_t d = 0; d < s.shape.size(); ++d) {
    if (shape4 && d < 4) shape4[d] = s.shape[d];
    n *= (uint64_t)s.shape[d];
  }
  if (dtype) *dtype = s.dtype == "f16" ? MIT2CFM_DTYPE_F16 : MIT2CFM_DTYPE_F32;
  if (elems) *elems = n;
  return MIT2CFM_OK;
}

mit2cfm_status mit2cfm_synthetic_set_fill(int32_t set, uint32_t i, uint64_t base_seed, float stddev,
                                          void* out) {
  if (!out) return fail(nullptr, MIT2CFM_E_ARG, "out must not be NULL");
  const auto* specs = synth_set(set);
  if (!specs) return fail(nullptr, MIT2CFM_E_ARG, "unknown synthetic tensor set");
  return guarded(nullptr, [&] {
    const auto b = synth_set_bytes(set, i, base_seed, stddev);
    std::memcpy(out, b.data(), b.size());
  });
}

mit2cfm_status mit2cfm_inspect_bundle(const char* bundle_path, uint64_t* tensor_count,
                                      uint64_t* payload_bytes, uint32_t verify_sha256) {
  if (!bundle_path) return fail(nullptr, MIT2CFM_E_ARG, "bundle_path must not be NULL");
  return guarded(nullptr, [&] {
    mit2::Bundle b(bundle_path);
    if (verify_sha256) {
      for (const auto& t : b.tensors()) {
        if (mit2::sha256_hex(b.tensor_data(t), (size_t)t.nbytes) != t.sha256)
          throw std::runtime_error("sha256 mismatch: " + t.name);
      }
    }
    if (tensor_count) *tensor_count = b.tensor_count();
    if (payload_bytes) *payload_bytes = b.total_tensor_bytes();
  });
}

mit2cfm_status mit2cfm_write_synthetic_bundle(const char* dir, uint64_t base_seed, float stddev) {
  if (!dir) return fail(nullptr, MIT2CFM_E_ARG, "dir must not be NULL");
  return guarded(nullptr, [&] {
    const auto& specs = mit2::estimator_tensor_specs();
    std::vector<mit2::TensorPayload> ts;
    for (size_t i = 0; i < specs.size(); ++i)
      ts.push_back({specs[i].name, specs[i].shape, specs[i].dtype, "s2mel",
                    mit2::synth_tensor_bytes(i, base_seed, stddev)});
    mit2::write_bundle(dir, ts);
  });
}

}  // extern "C"

mit2cfm_status mit2cfm_length_regulator(mit2cfm_ctx* ctx, const float* s_infer,
                                        uint32_t in_tokens, uint32_t out_tokens, float* out) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(s_infer && out, "s_infer and out must not be NULL");
    require(in_tokens > 0 && out_tokens > 0, "in_tokens and out_tokens must be positive");
    ctx->eng->length_regulator_host(s_infer, (int)in_tokens, (int)out_tokens, out);
  });
}

mit2cfm_status mit2cfm_condition(mit2cfm_ctx* ctx, const float* s_infer, uint32_t codes,
                                 const float* prompt_cond, uint32_t prompt_tokens,
                                 float* cond_out, uint32_t* generated_out) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(s_infer && prompt_cond && cond_out, "s_infer, prompt_cond and cond_out must not be NULL");
    require(codes > 0 && prompt_tokens > 0, "codes and prompt_tokens must be positive");
    const int gen = ctx->eng->condition_host(s_infer, (int)codes, prompt_cond, (int)prompt_tokens,
                                             cond_out);
    if (generated_out) *generated_out = (uint32_t)gen;
  });
}

mit2cfm_status mit2cfm_condition_device(mit2cfm_ctx* ctx, const float* s_infer, uint32_t codes,
                                        const float* prompt_cond, uint32_t prompt_tokens,
                                        float* cond_out, uint32_t* generated_out, uint32_t flags) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(s_infer && prompt_cond && cond_out, "s_infer, prompt_cond and cond_out must not be NULL");
    require(codes > 0 && prompt_tokens > 0, "codes and prompt_tokens must be positive");
    const int gen = ctx->eng->condition_device(s_infer, (int)codes, prompt_cond, (int)prompt_tokens,
                                               cond_out);
    if (generated_out) *generated_out = (uint32_t)gen;
    if (flags & MIT2CFM_FLAG_SYNC) ctx->eng->sync();
  });
}

static_assert(MIT2CFM_NOALLOC_MAX_CODES == (unsigned)mit2hip::Engine::kNoAllocMaxCodes,
              "the header's no-alloc limit is the engine's scratch limit");

mit2cfm_status mit2cfm_condition_device_noalloc(mit2cfm_ctx* ctx, const float* s_infer, uint32_t codes,
                                                const float* prompt_cond, uint32_t prompt_tokens,
                                                float* cond_out, uint32_t* generated_out, uint32_t flags) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(s_infer && prompt_cond && cond_out, "s_infer, prompt_cond and cond_out must not be NULL");
    require(codes > 0 && prompt_tokens > 0, "codes and prompt_tokens must be positive");
    require(codes <= MIT2CFM_NOALLOC_MAX_CODES, "codes exceeds MIT2CFM_NOALLOC_MAX_CODES (the scratch limit)");
    const int gen = ctx->eng->condition_device_noalloc(s_infer, (int)codes, prompt_cond,
                                                       (int)prompt_tokens, cond_out);
    if (generated_out) *generated_out = (uint32_t)gen;
    if (flags & MIT2CFM_FLAG_SYNC) ctx->eng->sync();
  });
}

uint32_t mit2cfm_generated_frames(uint32_t codes) {
  return (uint32_t)mit2hip::Engine::generated_frames((int)codes);
}

mit2cfm_status mit2cfm_noise_device(mit2cfm_ctx* ctx, uint32_t tokens, uint32_t channels,
                                    uint64_t seed, float temperature, float* out, uint32_t flags) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(out != nullptr, "out must not be NULL");
    require(tokens > 0 && channels > 0, "noise shape must be non-empty");
    ctx->eng->normal_noise_device((size_t)tokens * channels, seed, temperature, out);
    if (flags & MIT2CFM_FLAG_SYNC) ctx->eng->sync();
  });
}

// ---- BigVGAN vocoder ------------------------------------------------------
mit2cfm_status mit2cfm_bigvgan(mit2cfm_ctx* ctx, const float* mel, uint32_t tokens, float* wav) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(mel && wav, "mel and wav must not be NULL");
    require(tokens > 0 && tokens <= (1u << 20), "tokens must be in [1, 2^20]");
    ctx->eng->vocode_host(mel, (int)tokens, wav);
  });
}

mit2cfm_status mit2cfm_bigvgan_device(mit2cfm_ctx* ctx, const float* mel, uint32_t tokens, float* wav,
                                      uint32_t flags) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(mel && wav, "mel and wav must not be NULL");
    require(tokens > 0 && tokens <= (1u << 20), "tokens must be in [1, 2^20]");
    ctx->eng->vocode_device(mel, (int)tokens, wav);
    if (flags & MIT2CFM_FLAG_SYNC) ctx->eng->sync();
  });
}

uint64_t mit2cfm_bigvgan_stage_floats(int32_t stage, int32_t index, uint32_t tokens, int32_t output) {
  if (tokens == 0 || tokens > (1u << 20)) return 0;
  return output ? mit2hip::Vocoder::stage_out_floats(stage, index, (int)tokens)
                : mit2hip::Vocoder::stage_in_floats(stage, index, (int)tokens);
}

mit2cfm_status mit2cfm_bigvgan_stage(mit2cfm_ctx* ctx, int32_t stage, int32_t index, const float* in,
                                     uint32_t tokens, float* out, uint64_t out_capacity) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(in && out, "in and out must not be NULL");
    require(tokens > 0 && tokens <= (1u << 20), "tokens must be in [1, 2^20]");
    const uint64_t n = mit2cfm_bigvgan_stage_floats(stage, index, tokens, 1);
    require(n > 0, "unknown vocoder stage or index");
    require(out_capacity >= n, "out is smaller than the stage output");
    ctx->eng->vocoder_stage_host(stage, index, in, (int)tokens, out);
  });
}

// ---- the whole acoustic stage ---------------------------------------------
mit2cfm_status mit2cfm_acoustic_device(mit2cfm_ctx* ctx, const float* s_infer, uint32_t codes,
                                       const float* prompt_cond, const float* prompt_mel,
                                       uint32_t prompt_tokens, const float* style, uint64_t noise_seed,
                                       float noise_temperature, uint32_t steps, float cfg_rate,
                                       float* wav_out, float* mel_out, uint32_t* generated_out,
                                       uint32_t flags) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(s_infer && prompt_cond && prompt_mel && style && wav_out,
            "s_infer, prompt_cond, prompt_mel, style and wav_out must not be NULL");
    require(codes > 0 && codes <= (1u << 20) && prompt_tokens > 0 && prompt_tokens <= (1u << 20),
            "codes and prompt_tokens must be in [1, 2^20]");
    require(steps > 0 && steps <= 1000, "steps must be in [1, 1000]");
    require(cfg_rate >= 0.0f, "cfg_rate must be >= 0");
    const int gen = ctx->eng->acoustic_device(s_infer, (int)codes, prompt_cond, prompt_mel,
                                              (int)prompt_tokens, style, noise_seed, noise_temperature,
                                              (int)steps, cfg_rate, wav_out, mel_out);
    if (generated_out) *generated_out = (uint32_t)gen;
    if (flags & MIT2CFM_FLAG_SYNC) ctx->eng->sync();
  });
}

// ---- GPT mel-code decoder
mit2cfm_status mit2cfm_gpt_layers(mit2cfm_ctx* ctx, uint32_t* layers) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(layers != nullptr, "layers must not be NULL");
    *layers = ctx->eng->has_gpt() ? (uint32_t)ctx->eng->gpt().layers() : 0u;
  });
}

mit2cfm_status mit2cfm_gpt_kv_greedy(mit2cfm_ctx* ctx, const float* prefix, uint32_t prefix_tokens,
                                     uint32_t steps, int32_t hf_generate_positions,
                                     uint32_t* predicted_tokens, uint32_t* n_predicted,
                                     uint32_t* input_tokens, uint32_t* n_input, int32_t* first_stop_step,
                                     float* last_logits, double* timings_ms) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(prefix_tokens == 0 || prefix != nullptr, "prefix must not be NULL");
    require(prefix_tokens <= (1u << 16), "prefix_tokens must be <= 65536");
    require(steps <= (uint32_t)mit2hip::GptDecoder::kPositions, "steps must be <= 1818");
    require(steps == 0 || (predicted_tokens && n_predicted), "predicted_tokens/n_predicted must not be NULL");
    require(input_tokens && n_input && first_stop_step, "input_tokens/n_input/first_stop_step must not be NULL");
    mit2hip::GptDecoder::Greedy g;
    ctx->eng->gpt().kv_greedy(prefix, (int)prefix_tokens, (int)steps, hf_generate_positions != 0, g);
    if (n_predicted) *n_predicted = (uint32_t)g.predicted.size();
    if (!g.predicted.empty()) std::memcpy(predicted_tokens, g.predicted.data(), g.predicted.size() * 4);
    *n_input = (uint32_t)g.input_tokens.size();
    std::memcpy(input_tokens, g.input_tokens.data(), g.input_tokens.size() * 4);
    *first_stop_step = g.first_stop_step;
    if (last_logits && !g.last_logits.empty())
      std::memcpy(last_logits, g.last_logits.data(), g.last_logits.size() * sizeof(float));
    if (timings_ms) {
      timings_ms[0] = g.prefill_ms;
      timings_ms[1] = g.decode_ms;
    }
  });
}

mit2cfm_status mit2cfm_gpt_kv_sample(mit2cfm_ctx* ctx, const float* prefix, uint32_t prefix_tokens,
                                     uint32_t steps, int32_t hf_generate_positions,
                                     const mit2cfm_gpt_sampling* sampling, const uint32_t* history_prefix,
                                     uint32_t history_prefix_count, uint32_t* predicted_tokens,
                                     uint32_t* n_predicted, uint32_t* input_tokens, uint32_t* n_input,
                                     int32_t* first_stop_step, float* last_logits,
                                     float* last_processed_logits, double* timings_ms) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(sampling != nullptr, "sampling must not be NULL");
    require(history_prefix_count == 0 || history_prefix != nullptr,
            "history_prefix must not be NULL when history_prefix_count > 0");
    require(history_prefix_count <= mit2hip::GptDecoder::kMaxHistory, "history_prefix_count must be <= 8192");
    require(prefix_tokens == 0 || prefix != nullptr, "prefix must not be NULL");
    require(prefix_tokens <= (1u << 16), "prefix_tokens must be <= 65536");
    require(steps <= (uint32_t)mit2hip::GptDecoder::kPositions, "steps must be <= 1818");
    require(steps == 0 || (predicted_tokens && n_predicted), "predicted_tokens/n_predicted must not be NULL");
    require(input_tokens && n_input && first_stop_step, "input_tokens/n_input/first_stop_step must not be NULL");
    mit2hip::GptDecoder::Sampling smp;
    smp.seed = sampling->seed;
    smp.temperature = sampling->temperature;
    smp.top_k = sampling->top_k;
    smp.top_p = sampling->top_p;
    smp.repetition_penalty = sampling->repetition_penalty;
    smp.history = history_prefix;
    smp.n_history = history_prefix_count;
    mit2hip::GptDecoder::Greedy g;
    ctx->eng->gpt().kv_sample(prefix, (int)prefix_tokens, (int)steps, hf_generate_positions != 0, smp, g);
    if (n_predicted) *n_predicted = (uint32_t)g.predicted.size();
    if (!g.predicted.empty()) std::memcpy(predicted_tokens, g.predicted.data(), g.predicted.size() * 4);
    *n_input = (uint32_t)g.input_tokens.size();
    std::memcpy(input_tokens, g.input_tokens.data(), g.input_tokens.size() * 4);
    *first_stop_step = g.first_stop_step;
    if (last_logits && !g.last_logits.empty())
      std::memcpy(last_logits, g.last_logits.data(), g.last_logits.size() * sizeof(float));
    if (last_processed_logits && !g.last_processed_logits.empty())
      std::memcpy(last_processed_logits, g.last_processed_logits.data(), g.last_processed_logits.size() * sizeof(float));
    if (timings_ms) {
      timings_ms[0] = g.prefill_ms;
      timings_ms[1] = g.decode_ms;
    }
  });
}

mit2cfm_status mit2cfm_gpt_cached_decode(mit2cfm_ctx* ctx, const float* rows, uint32_t prefix_tokens,
                                         float* ln_f, float* final_norm, float* logits, uint32_t* argmax) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(rows != nullptr, "rows must not be NULL");
    require(prefix_tokens < (1u << 16), "prefix_tokens must be < 65536");
    const uint32_t a = ctx->eng->gpt().cached_decode(rows, (int)prefix_tokens, ln_f, final_norm, logits);
    if (argmax) *argmax = a;
  });
}

mit2cfm_status mit2cfm_gpt_profile_launch(mit2cfm_ctx* ctx, int32_t kernel, uint32_t count,
                                          double* bytes_per_launch, const char** name) {
  if (!ctx) return fail(nullptr, MIT2CFM_E_ARG, "ctx must not be NULL");
  return guarded(ctx, [&] {
    require(kernel >= 0 && kernel <= 5, "kernel must be 0..5");
    require(count <= 100000, "count must be <= 100000");
    double b = 0;
    const char* nm = ctx->eng->gpt().profile_launch(kernel, 0, &b);
    if (count) ctx->eng->gpt().profile_launch(kernel, (int)count, nullptr);
    if (bytes_per_launch) *bytes_per_launch = b;
    if (name) *name = nm;
  });
}
