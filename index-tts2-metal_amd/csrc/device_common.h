// device_common.h -- shared types and helpers for the gfx950 (CDNA4) kernels
// of the DiT-CFM decoder.
//
// Conventions used by every kernel in this directory:
//  * activations are token-major row-major; row m = branch * T + t;
//  * GEMM operands are f16 with fp32 accumulation on the matrix cores
//    (v_mfma_f32_16x16x32_f16, 64-lane wavefronts);
//  * the residual streams (transformer x/h, WaveNet x/out) stay fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mit2hip {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Word 3 of a raw buffer resource on gfx9-family GPUs (gfx950): 32-bit data,
// no swizzle, byte offsets checked against word 2 (the byte range), so a
// load past the range returns zeros without a memory access.
constexpr int kBufferRsrcWord3 = 0x00020000;

typedef __attribute__((address_space(3))) void lds_ptr_t;

// Buffer resources and direct buffer -> LDS loads.  The resource type and
// the builtins exist only for the GPU target; the host pass (which parses
// kernel bodies but never runs them) sees inert stand-ins, without which it
// would drop the kernels' launch stubs.
#if defined(__HIP_DEVICE_COMPILE__)
typedef __amdgpu_buffer_rsrc_t buffer_rsrc_t;
__device__ __forceinline__ buffer_rsrc_t make_buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kBufferRsrcWord3);
}
// Each lane's 16 (or 4) bytes at base + voffset + soffset land at
// M0 + 16*lane (4*lane), M0 = lds (wave-uniform); soffset is wave-uniform.
__device__ __forceinline__ void buffer_load_lds16(buffer_rsrc_t r, lds_ptr_t* lds, int voffset, int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voffset, soffset, 0, 0);
}
__device__ __forceinline__ void buffer_load_lds4(buffer_rsrc_t r, lds_ptr_t* lds, int voffset, int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 4, voffset, soffset, 0, 0);
}
// Register loads and stores through a resource: one 32-bit byte offset per
// lane; a store past the resource's byte range is dropped.
__device__ __forceinline__ float buffer_load_f32(buffer_rsrc_t r, int voffset) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voffset, 0, 0));
}
__device__ __forceinline__ void buffer_store_f32(buffer_rsrc_t r, int voffset, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voffset, 0, 0);
}
__device__ __forceinline__ void buffer_store_f16(buffer_rsrc_t r, int voffset, half_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, voffset, 0, 0);
}
#else
struct buffer_rsrc_t { const void* base; };
__device__ inline buffer_rsrc_t make_buffer_rsrc(const void* base, int) { return buffer_rsrc_t{base}; }
__device__ inline void buffer_load_lds16(buffer_rsrc_t, lds_ptr_t*, int, int) {}
__device__ inline void buffer_load_lds4(buffer_rsrc_t, lds_ptr_t*, int, int) {}
__device__ inline float buffer_load_f32(buffer_rsrc_t, int) { return 0.0f; }
__device__ inline void buffer_store_f32(buffer_rsrc_t, int, float) {}
__device__ inline void buffer_store_f16(buffer_rsrc_t, int, half_t) {}
#endif

// Padded operand widths (every GEMM K is a multiple of 128 so that K stages
// of 64/128/256 divide it and concatenated operands switch source on a stage
// boundary).
constexpr int kMelPad = 128;   // f16 mel rows: 80 values + 48 zeros
constexpr int kMcWidth = 896;  // merge-constant rows: [prompt 128 | content 512 | style 192 | 0 x 64]
constexpr int kMcContent = 128;
constexpr int kMcStyle = 640;

// D(16x16, fp32) += A(16x32, f16) * B(32x16, f16).
// Lane l supplies A row (l % 16) and B column (l % 16), each with the eight
// K-slots of lane group l / 16.  D element (row 4*(l/16)+i, col l%16) is in
// component i of lane l.
__device__ __forceinline__ floatx4 mfma16x16x32(const half8& a, const half8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// The GEMM epilogues' activations (the decode's gated WaveNet conv and the
// SwiGLU feed-forward, whose outputs are stored as f16) use the hardware
// exponential and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each)
// instead of an IEEE division and libm's tanhf: the epilogue of the k=5 conv
// GEMM runs 5% faster and w1|w3's 3%.
__device__ __forceinline__ float fast_rcp(float v) { return __builtin_amdgcn_rcpf(v); }
__device__ __forceinline__ float sigmoid_f(float v) { return fast_rcp(1.0f + __expf(-v)); }
__device__ __forceinline__ float silu_fast(float v) { return v * fast_rcp(1.0f + __expf(-v)); }

// tanh with the reference kernel's saturation (|a| > 20 -> +-1), as
// 1 - 2 / (e^(2a) + 1): the absolute error is a few 1e-8 (near 0 the
// rounding of e^(2a) to fp32 dominates), below the f16 rounding of the
// gated product it feeds.
__device__ __forceinline__ float tanh_sat(float a) {
  if (a > 20.0f) return 1.0f;
  if (a < -20.0f) return -1.0f;
  return 1.0f - 2.0f * fast_rcp(__expf(2.0f * a) + 1.0f);
}

// Most row sequences a product can name for row-tile skipping (8 requests
// with their cond and null branches).
constexpr int kMaxRowSeq = 16;

// The needed rows of a padded batch: nb sequences of T rows, of which the
// first need[b] rows of sequence b are needed (nb = 0: every row).
struct RowSkip {
  int T = 0;
  int nb = 0;
  int need[kMaxRowSeq] = {};
};

// Reflect index for padding (k-tap conv, reflect mode).  Any integer maps into
// [0, T) by repeated mirroring at 0 and T-1; a one-token sequence maps to 0.
__device__ __forceinline__ int reflect_index(int src, int T) {
  if (T <= 1) return 0;
  while (src < 0 || src >= T) {
    if (src < 0) src = -src;
    if (src >= T) src = 2 * T - 2 - src;
  }
  return src;
}

}  // namespace mit2hip
