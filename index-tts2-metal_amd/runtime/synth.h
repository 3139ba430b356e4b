// synth.h -- seeded synthetic inputs and weights for the DiT-CFM decoder.
//
// The normal generator is the reference's splitmix64 + Box-Muller
// (runtime/impl/tokenizer_tests.cpp:2102-2140, make_deterministic_normal_noise),
// so C++, Python and the oracle regenerate identical bytes from a seed.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace mit2 {

uint64_t splitmix64_next(uint64_t& state);
float splitmix64_uniform_open01(uint64_t& state);
// tokens*channels normals N(0, temperature^2), pairs (r cos a, r sin a).
std::vector<float> make_deterministic_normal_noise(uint32_t tokens, uint32_t channels,
                                                   uint64_t seed, float temperature);

struct SynthSpec {
  std::string name;             // full tensor name
  std::vector<int64_t> shape;   // PyTorch shape
  std::string dtype;            // "f16" (weights) or "f32" (freqs)
};

// Every tensor the DiT-CFM estimator reads (prefix s2mel.net.cfm.estimator.),
// sorted by name.
const std::vector<SynthSpec>& estimator_tensor_specs();

// Payload of spec i from seed base_seed + i, rounded to f16; *.freqs are the
// closed form exp(-ln(10000) * k / 128) in f32.  stddev > 0: N(0, stddev)
// for every tensor.  stddev == 0: activation-preserving scales (matrices
// N(0, 1/sqrt(fan_in)), norm weights and weight-norm gains 1 + N(0, 0.02),
// other vectors N(0, 0.02)).
std::vector<uint8_t> synth_tensor_bytes(size_t i, uint64_t base_seed, float stddev);

// The s2mel length regulator's 20 tensors (prefix s2mel.net.length_regulator.),
// sorted by name, all f16: N(0, stddev) from base_seed + i; the GroupNorm
// weights are 1 + N(0, stddev).
const std::vector<SynthSpec>& length_regulator_tensor_specs();
std::vector<uint8_t> synth_lr_tensor_bytes(size_t i, uint64_t base_seed, float stddev);

// The BigVGAN vocoder's 783 tensors (prefix bigvgan.), sorted by name.
// weight_v and biases N(0, stddev) f16 from base_seed + i; weight_g =
// g (1 + N(0, stddev)) f16 with g = 1 for conv_pre and the upsamplers, 0.1
// for conv_post and 0.6 for the resblock convs (so the residual stack
// neither grows nor vanishes and the waveform stays inside the clamp); the
// activations' filters are the 12-tap Kaiser-windowed sinc low-pass of the
// alias-free activation (f32); SnakeBeta's log alpha and log beta are
// N(0, 0.1) (f32).
const std::vector<SynthSpec>& bigvgan_tensor_specs();
std::vector<uint8_t> synth_bigvgan_tensor_bytes(size_t i, uint64_t base_seed, float stddev);

// The GPT mel-code decoder's tensors (24 GPT-2 layers, ln_f, final_norm,
// mel_head, mel and mel-position embeddings), sorted by name, all f16,
// checkpoint layouts (Conv1D weights [in][out]): N(0, stddev) from
// base_seed + i; the LayerNorm weights are 1 + N(0, stddev).
const std::vector<SynthSpec>& gpt_tensor_specs();
std::vector<uint8_t> synth_gpt_tensor_bytes(size_t i, uint64_t base_seed, float stddev);

// Kaiser-windowed sinc low-pass (cutoff 0.25, half-width 0.3, 12 taps, unit
// DC gain): the filter of BigVGAN's alias-free activation for ratio 2.
std::vector<float> kaiser_sinc_filter12();

}  // namespace mit2
