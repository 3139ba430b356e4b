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

}  // namespace mit2
