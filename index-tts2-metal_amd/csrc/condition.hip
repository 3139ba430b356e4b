// condition.hip -- element-wise kernels of the condition and noise producer
// (the s2mel length regulator, gpt.cpp:5271-5340, and the seeded noise of
// tokenizer_tests.cpp:2102-2140).  All of them are HBM-bound row passes.
#include "condition.h"

#include "gemm.h"

namespace mit2hip {

// f16 operand of an fp32 tensor: hi = f16(v); with lo_off, also the lo half
// of the split pair at out + lo_off (GemmArgs::split).
__global__ void f32_to_f16_kernel(const float* __restrict__ in, half_t* __restrict__ out, size_t n,
                                  size_t lo_off) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (lo_off) {
    half_t h, l;
    split_f16(in[i], h, l);
    out[i] = h;
    out[lo_off + i] = l;
  } else {
    out[i] = (half_t)in[i];
  }
}

hipError_t launch_f32_to_f16(const float* in, half_t* out, size_t n, size_t lo_off, hipStream_t s) {
  if (n == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, out, n,
                     lo_off);
  return hipGetLastError();
}

// One wave per output row: 64 lanes x 8 halves = the 512 channels.  With
// split operands (dst_lo nonzero) the lo rows move the same way.
__global__ __launch_bounds__(256) void nearest_rows_kernel(const half_t* __restrict__ src,
                                                           int in_tokens, int out_tokens,
                                                           float scale,
                                                           half_t* __restrict__ dst,
                                                           size_t src_lo, size_t dst_lo) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t > out_tokens) return;
  half8 v, vl;
  if (t == out_tokens) {
    for (int i = 0; i < 8; ++i) v[i] = vl[i] = (half_t)0.0f;
  } else {
    int s = (int)floorf((float)t * scale);
    if (s >= in_tokens) s = in_tokens - 1;
    v = *reinterpret_cast<const half8*>(src + (size_t)s * 512 + lane * 8);
    if (dst_lo) vl = *reinterpret_cast<const half8*>(src + src_lo + (size_t)s * 512 + lane * 8);
  }
  *reinterpret_cast<half8*>(dst + (size_t)t * 512 + lane * 8) = v;
  if (dst_lo) *reinterpret_cast<half8*>(dst + dst_lo + (size_t)t * 512 + lane * 8) = vl;
}

hipError_t launch_nearest_rows(const half_t* src, int in_tokens, int out_tokens, float scale,
                               half_t* dst, size_t src_lo, size_t dst_lo, hipStream_t s) {
  if (in_tokens <= 0 || out_tokens <= 0 || (src_lo == 0) != (dst_lo == 0)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(nearest_rows_kernel, dim3((out_tokens + 1 + 3) / 4), dim3(256), 0, s, src,
                     in_tokens, out_tokens, scale, dst, src_lo, dst_lo);
  return hipGetLastError();
}

// Mish as x * tanh(softplus(x)) = x * n / (n + 2) with n = e^x (e^x + 2):
// one exponential and one division.  Past x = 15 the ratio rounds to 1 in
// fp32 (and e^x would overflow further on), so x is returned there.
__device__ __forceinline__ float mish_f(float x) {
  if (x > 15.0f) return x;
  const float e = expf(x);
  const float n = e * (e + 2.0f);
  return x * (n / (n + 2.0f));
}

// GroupNorm (one group over rows x 512 values) + Mish, statistics included.
// Every workgroup first reduces all of the producing GEMM's per-row partial
// sums and sums of squares in double, in one fixed order (a strided share per
// thread, a wave reduction, the 16 wave sums in order), so all of them hold
// the same mean and 1/std; then it normalises its own 4 rows, 2 values per
// thread.
constexpr int kGnRowsPerBlock = 4;
__global__ __launch_bounds__(1024) void gn_mish_kernel(const float* __restrict__ sum_parts,
                                                       const float* __restrict__ ssq_parts,
                                                       int nparts, double count, float eps,
                                                       const float* __restrict__ y,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, int rows,
                                                       half_t* __restrict__ out, size_t out_lo) {
  __shared__ double w1[16], w2[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  double a = 0.0, b = 0.0;
  // The thread's share, 16 loads issued before the adds that use them (one
  // at a time, each add waited for its own load: a chain of L2 round trips);
  // the adds keep the share's order.  Buffer loads past nparts return zero,
  // so the loads need no branch (a branch around each made it wait again).
  constexpr int kU = 16;
  const buffer_rsrc_t rs = make_buffer_rsrc(sum_parts, nparts * 4);
  const buffer_rsrc_t rq = make_buffer_rsrc(ssq_parts, nparts * 4);
  for (int i0 = tid; i0 < nparts; i0 += 1024 * kU) {
    float va[kU], vb[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = i0 + u * 1024;
      va[u] = buffer_load_f32(rs, i * 4);
      vb[u] = buffer_load_f32(rq, i * 4);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (i0 + u * 1024 < nparts) {
        a += (double)va[u];
        b += (double)vb[u];
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    a += __shfl_xor(a, off, 64);
    b += __shfl_xor(b, off, 64);
  }
  if (lane == 0) {
    w1[wave] = a;
    w2[wave] = b;
  }
  __syncthreads();
  double s1 = 0.0, s2 = 0.0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    s1 += w1[w];
    s2 += w2[w];
  }
  const double mean_d = s1 / count;
  double var = s2 / count - mean_d * mean_d;
  if (var < 0.0) var = 0.0;
  const float mean = (float)mean_d;
  const float rstd = (float)(1.0 / sqrt(var + (double)eps));

  const int r = blockIdx.x * kGnRowsPerBlock + (tid >> 8);
  if (r >= rows) return;
  const int c = (tid & 255) * 2;
  const float2 v = *reinterpret_cast<const float2*>(y + (size_t)r * 512 + c);
  half_t o0, o1, l0, l1;
  split_f16(mish_f((v.x - mean) * rstd * gamma[c] + beta[c]), o0, l0);
  split_f16(mish_f((v.y - mean) * rstd * gamma[c + 1] + beta[c + 1]), o1, l1);
  *reinterpret_cast<half2v*>(out + (size_t)r * 512 + c) = half2v{o0, o1};
  if (out_lo) *reinterpret_cast<half2v*>(out + out_lo + (size_t)r * 512 + c) = half2v{l0, l1};
}

hipError_t launch_gn_mish(const float* sum_parts, const float* ssq_parts, float eps, const float* y,
                          const float* gamma, const float* beta, int rows, half_t* out, size_t out_lo,
                          hipStream_t s) {
  if (rows <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gn_mish_kernel, dim3((rows + kGnRowsPerBlock - 1) / kGnRowsPerBlock), dim3(1024), 0,
                     s, sum_parts, ssq_parts, rows * 16, (double)rows * 512.0, eps, y, gamma, beta, rows,
                     out, out_lo);
  return hipGetLastError();
}

// splitmix64 output for the state reached after `steps` increments of seed.
__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t steps) {
  uint64_t z = seed + steps * 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Uniform in (0, 1) from the top 53 bits, as splitmix64_uniform_open01
// (tokenizer_tests.cpp:2109-2119) forms it, then rounded to float.
__device__ __forceinline__ float uniform_open01(uint64_t bits64) {
  constexpr double scale = 1.0 / 9007199254740992.0;  // 2^-53
  double v = ((double)(bits64 >> 11) + 0.5) * scale;
  if (v <= 0.0) v = scale;
  else if (v >= 1.0) v = 1.0 - scale;
  return (float)v;
}

__global__ __launch_bounds__(256) void normal_noise_kernel(size_t n, uint64_t seed,
                                                           float temperature,
                                                           float* __restrict__ out) {
  const size_t pair = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t i = 2 * pair;
  if (i >= n) return;
  const float u1 = uniform_open01(splitmix64_at(seed, 2 * (uint64_t)pair + 1));
  const float u2 = uniform_open01(splitmix64_at(seed, 2 * (uint64_t)pair + 2));
  constexpr float two_pi = 6.2831853071795864769f;
  const float radius = sqrtf(-2.0f * logf(u1));
  const float angle = two_pi * u2;
  out[i] = radius * cosf(angle) * temperature;
  if (i + 1 < n) out[i + 1] = radius * sinf(angle) * temperature;
}

hipError_t launch_normal_noise(size_t n, uint64_t seed, float temperature, float* out,
                               hipStream_t s) {
  if (n == 0) return hipErrorInvalidValue;
  const size_t pairs = (n + 1) / 2;
  hipLaunchKernelGGL(normal_noise_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s,
                     n, seed, temperature, out);
  return hipGetLastError();
}

}  // namespace mit2hip
