// vocoder.h -- the BigVGAN vocoder (mel -> waveform) on the GPU: the consumer
// of the DiT-CFM mel (runtime/impl/dit_cfm_bigvgan.cpp:3606-4512).
//
// Every conv, including the transposed-conv upsamplers, is one implicit-GEMM
// launch of gemm.hip (A_CONVP: any kernel size and dilation, zero padding);
// the anti-aliased SnakeBeta activation is one fused kernel (upsample x2,
// snake, low-pass downsample x2) that writes the next conv's f16 operand.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "device_common.h"

namespace mit2hip {

class Vocoder {
 public:
  // Tensors named "bigvgan.*" (fp32 on the host, any layout the checkpoint
  // has); throws std::invalid_argument when one is missing or misshaped.
  Vocoder(const std::unordered_map<std::string, std::vector<float>>& t, hipStream_t stream);
  // From the vocoder section of a device image (see append_image).
  Vocoder(const uint8_t* image, size_t bytes, hipStream_t stream);
  // Appends the prepared weights (arena bytes and layout) to an image.
  void append_image(std::vector<uint8_t>& out) const;
  ~Vocoder();
  Vocoder(const Vocoder&) = delete;
  Vocoder& operator=(const Vocoder&) = delete;

  // Arithmetic of the convs: f32 = true (default) runs them on split f16
  // operand pairs (fp32-level products, as the reference's fp32 vocoder),
  // false on plain f16 operands.
  void set_f32(bool on);
  bool f32() const;

  // True when any "bigvgan.*" tensor is present (then all of them must be).
  static bool present(const std::unordered_map<std::string, std::vector<float>>& t);
  size_t weight_bytes() const;

  // run_bigvgan_vocoder (dit_cfm_bigvgan.cpp:4058/4196): mel [tokens][80]
  // fp32 -> wav [256 * tokens] fp32, DEVICE pointers, enqueued on the stream.
  void vocode_device(const float* mel, int tokens, float* wav);

  // One reference stage on HOST pointers (synchronous), for parity tests:
  //  0 conv_pre           in [T][80]   -> out [T][1536]
  //  1 upsampler `index`  in [T][Cin]  -> out [s T][Cout]
  //  2 activation `index` (resblock j, activation a: index = 6 j + a; 108 =
  //    activation_post)   in [T][C]    -> out [T][C]
  //  3 resblock `index`   in [T][C]    -> out [T][C]
  //  4 resblock group `index` (upsampler stage 0..5) in [T][C] -> out [T][C]
  //  5 post               in [T][24]   -> out [T]
  //  6 body               in [T][80]   -> out [256 T][24]
  // Returns the number of output floats written.
  size_t stage_host(int stage, int index, const float* in, int tokens, float* out);
  // Output floats of a stage for `tokens` input rows (0 for a bad stage/index).
  static size_t stage_out_floats(int stage, int index, int tokens);
  static size_t stage_in_floats(int stage, int index, int tokens);

 public:
  struct Conv;  // (defined in vocoder.hip)
  struct Act;

 private:
  struct Impl;
  Impl* d_;
};

}  // namespace mit2hip
