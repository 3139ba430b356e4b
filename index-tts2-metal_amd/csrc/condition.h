// condition.h -- kernels of the condition and noise producer that feeds the
// DiT-CFM decode: the s2mel length regulator's element-wise stages (its
// GEMMs run on gemm.hip) and the seeded normal-noise generator.
#pragma once

#include "device_common.h"

namespace mit2hip {

// dst[t] = src[min(floor(t * scale), in_tokens - 1)] for t < out_tokens,
// 512-wide f16 rows (cpu_nearest_interpolate, tokenizer_tests.cpp:3127, with
// scale = (float)in_tokens / (float)out_tokens formed by the caller); also
// zeroes row out_tokens of dst, the padding row of the zero-padded k = 3 conv.
// For split operand pairs, src_lo / dst_lo (both nonzero) are the element
// offsets of the lo rows, which move the same way.
hipError_t launch_nearest_rows(const half_t* src, int in_tokens, int out_tokens, float scale,
                               half_t* dst, size_t src_lo, size_t dst_lo, hipStream_t s);

// out = f16(in), n values; with lo_off nonzero also the lo half of each split
// pair at out + lo_off (GemmArgs::split).
hipError_t launch_f32_to_f16(const float* in, half_t* out, size_t n, size_t lo_off, hipStream_t s);

// GroupNorm with one group over rows x 512 values, then Mish:
// out[r][c] = f16(mish((y[r][c] - mean) * rstd * gamma[c] + beta[c])) for
// r < rows (cpu_groupnorm1 + cpu_mish, tokenizer_tests.cpp:3874-3904), the
// mean and rstd = 1/sqrt(var + eps) reduced in double from the per-row,
// per-32-column partial sums and sums of squares the producing GEMM wrote
// ([rows][16] each).  With out_lo nonzero also the lo half of the split pair
// at out + out_lo.
hipError_t launch_gn_mish(const float* sum_parts, const float* ssq_parts, float eps, const float* y,
                          const float* gamma, const float* beta, int rows, half_t* out, size_t out_lo,
                          hipStream_t s);

// make_deterministic_normal_noise (tokenizer_tests.cpp:2121-2140) on the GPU:
// out[n] for n = tokens * channels values.  splitmix64 is a counter: value
// pair j draws its two uniforms from states seed + (2j+1) g and seed + (2j+2) g
// (g the splitmix64 increment), so every pair is computed independently and
// the uniforms are bit-identical to the sequential generator.
hipError_t launch_normal_noise(size_t n, uint64_t seed, float temperature, float* out,
                               hipStream_t s);

}  // namespace mit2hip
