// rowops.hip -- bandwidth-bound row kernels of the DiT-CFM decoder (gfx950).
//
// Reference counterparts (kernels.metal unless noted): adaptive RMSNorm
// :755-792, adaptive LayerNorm :702-753, input merge :898-931, CFM Euler
// update :794-818, timestep embedding :1812-1829, GEMV :1084-1119, copies
// :150-159.  Each row kernel gives one 64-lane wavefront a 512-wide row
// (8 consecutive floats per lane, two 16-byte loads), so every access is
// fully coalesced and the row reductions are two-level shuffles.
#include "rowops.h"

namespace mit2hip {

// ---------------------------------------------------------------- norms
__global__ __launch_bounds__(256) void adarms_kernel(const float* __restrict__ x,
                                                     const float* __restrict__ gamma,
                                                     const float* __restrict__ aw,
                                                     const float* __restrict__ ab,
                                                     half_t* __restrict__ out, int rows) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)row * 512) + lane * 2;
  const float4 a = xr[0], b = xr[1];
  float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
  ss = warp_sum(ss);
  const float inv = 1.0f / sqrtf(ss / 512.0f + 1e-5f);
  half8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = lane * 8 + i;
    o[i] = (half_t)(aw[c] * (v[i] * inv * gamma[c]) + ab[c]);
  }
  *reinterpret_cast<half8*>(out + (size_t)row * 512 + lane * 8) = o;
}

__global__ __launch_bounds__(256) void adaln_kernel(const float* __restrict__ x,
                                                    const float* __restrict__ shift,
                                                    const float* __restrict__ scale,
                                                    half_t* __restrict__ out, int rows) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)row * 512) + lane * 2;
  const float4 a = xr[0], b = xr[1];
  float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += v[i];
  const float mean = warp_sum(s) / 512.0f;
  float var = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float d = v[i] - mean;
    var += d * d;
  }
  var = warp_sum(var) / 512.0f;
  const float inv = 1.0f / sqrtf(var + 1e-6f);
  half8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = lane * 8 + i;
    o[i] = (half_t)(((v[i] - mean) * inv) * (1.0f + scale[c]) + shift[c]);
  }
  *reinterpret_cast<half8*>(out + (size_t)row * 512 + lane * 8) = o;
}

__global__ __launch_bounds__(256) void norm_prep_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ aw,
                                                        const float* __restrict__ gamma,
                                                        half_t* __restrict__ n16,
                                                        float* __restrict__ ssq, int rows) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)row * 512) + lane * 2;
  const float4 a = xr[0], b = xr[1];
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  float ss = 0.f;
  half8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = lane * 8 + i;
    ss += v[i] * v[i];
    o[i] = (half_t)(v[i] * (aw[c] * gamma[c]));
  }
  *reinterpret_cast<half8*>(n16 + (size_t)row * 512 + lane * 8) = o;
  // four lanes hold one 32-column block
  ss += __shfl_xor(ss, 1, kWave);
  ss += __shfl_xor(ss, 2, kWave);
  if ((lane & 3) == 0) ssq[(size_t)row * 16 + (lane >> 2)] = ss;
}

hipError_t launch_norm_prep(const float* x, const float* aw, const float* gamma, half_t* n16,
                            float* ssq, int rows, hipStream_t s) {
  hipLaunchKernelGGL(norm_prep_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, aw, gamma, n16,
                     ssq, rows);
  return hipGetLastError();
}

// One wavefront per output column n: the f16 weight row stays in registers
// (8 values per lane) across the S steps.
__global__ __launch_bounds__(256) void norm_bias_kernel(const float* __restrict__ ab, int ab_ld,
                                                        int S, const half_t* __restrict__ W, int N,
                                                        float* __restrict__ out, int out_ld) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const half8 w = *reinterpret_cast<const half8*>(W + (size_t)n * 512 + lane * 8);
  // Four steps' rows requested together (a step's loads each waited for the
  // previous step's sum); rows past S are clamped to the last and not stored.
  constexpr int kSteps = 4;
  for (int s0 = 0; s0 < S; s0 += kSteps) {
    float4 a[kSteps], b[kSteps];
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const float4* ar = reinterpret_cast<const float4*>(ab + (size_t)min(s0 + u, S - 1) * ab_ld) + lane * 2;
      a[u] = ar[0];
      b[u] = ar[1];
    }
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      if (s0 + u >= S) break;
      float acc = a[u].x * (float)w[0] + a[u].y * (float)w[1] + a[u].z * (float)w[2] + a[u].w * (float)w[3] +
                  b[u].x * (float)w[4] + b[u].y * (float)w[5] + b[u].z * (float)w[6] + b[u].w * (float)w[7];
      acc = warp_sum(acc);
      if (lane == 0) out[(size_t)(s0 + u) * out_ld + n] = acc;
    }
  }
}

hipError_t launch_norm_bias(const float* ab, int ab_ld, int S, const half_t* W, int N, float* out,
                            int out_ld, hipStream_t s) {
  if (S <= 0 || ab_ld % 4 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(norm_bias_kernel, dim3((N + 3) / 4), dim3(256), 0, s, ab, ab_ld, S, W, N, out,
                     out_ld);
  return hipGetLastError();
}

hipError_t launch_adarms(const float* x, const float* gamma, const float* aw, const float* ab,
                         half_t* out16, int rows, hipStream_t s) {
  hipLaunchKernelGGL(adarms_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, gamma, aw, ab, out16,
                     rows);
  return hipGetLastError();
}

hipError_t launch_adaln(const float* x, const float* shift, const float* scale, half_t* out16,
                        int rows, hipStream_t s) {
  hipLaunchKernelGGL(adaln_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, shift, scale, out16,
                     rows);
  return hipGetLastError();
}

// ---------------------------------------------------------------- set-up
// One 256-thread block per (branch, token) row.
__global__ __launch_bounds__(256) void decode_prep_kernel(
    const float* __restrict__ x0, const float* __restrict__ prompt, const float* __restrict__ cond,
    const float* __restrict__ style, const uint32_t* __restrict__ P, int T, int cfg_on,
    float* __restrict__ x_cur, half_t* __restrict__ xmel16, half_t* __restrict__ cond16,
    half_t* __restrict__ mc16) {
  const int t = blockIdx.x;
  const int b = blockIdx.y;
  const int r = cfg_on ? (b >> 1) : b;
  const bool is_cond = cfg_on ? ((b & 1) == 0) : true;
  const uint32_t Pr = P[r];
  const size_t row = (size_t)b * T + t;
  const size_t rrow = (size_t)r * T + t;
  for (int j = threadIdx.x; j < kMelPad; j += blockDim.x) {
    float xv = 0.0f;
    if (j < 80 && (uint32_t)t >= Pr) xv = x0[rrow * 80 + j];
    if (j < 80 && is_cond) x_cur[rrow * 80 + j] = xv;
    xmel16[row * kMelPad + j] = (half_t)xv;
  }
  for (int j = threadIdx.x; j < 512; j += blockDim.x)
    cond16[row * 512 + j] = (half_t)(is_cond ? cond[rrow * 512 + j] : 0.0f);
  // prompt_x: the prompt frames on the first P rows of the cond branch.
  for (int j = threadIdx.x; j < kMcContent; j += blockDim.x) {
    float pv = 0.0f;
    if (is_cond && j < 80 && (uint32_t)t < Pr) pv = prompt[((size_t)r * T + t) * 80 + j];
    mc16[row * kMcWidth + j] = (half_t)pv;
  }
  for (int j = threadIdx.x; j < kMcWidth - kMcStyle; j += blockDim.x)
    mc16[row * kMcWidth + kMcStyle + j] =
        (half_t)(is_cond && j < 192 ? style[(size_t)r * 192 + j] : 0.0f);
}

hipError_t launch_decode_prep(const float* x0, const float* prompt, const float* cond,
                              const float* style, const uint32_t* P, int nreq, int T, int cfg_on,
                              float* x_cur, half_t* xmel16, half_t* cond16, half_t* mc16,
                              hipStream_t s) {
  const int B = cfg_on ? 2 * nreq : nreq;
  hipLaunchKernelGGL(decode_prep_kernel, dim3(T, B), dim3(256), 0, s, x0, prompt, cond, style, P,
                     T, cfg_on, x_cur, xmel16, cond16, mc16);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void step_prep_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ prompt_x,
                                                        const float* __restrict__ cond,
                                                        const float* __restrict__ style, int T,
                                                        half_t* __restrict__ xmel16,
                                                        half_t* __restrict__ cond16,
                                                        half_t* __restrict__ mc16) {
  const int t = blockIdx.x;
  const int b = blockIdx.y;
  const size_t row = (size_t)b * T + t;
  for (int j = threadIdx.x; j < kMelPad; j += blockDim.x) {
    xmel16[row * kMelPad + j] = (half_t)(j < 80 ? x[row * 80 + j] : 0.0f);
    mc16[row * kMcWidth + j] = (half_t)(j < 80 ? prompt_x[row * 80 + j] : 0.0f);
  }
  for (int j = threadIdx.x; j < 512; j += blockDim.x) cond16[row * 512 + j] = (half_t)cond[row * 512 + j];
  for (int j = threadIdx.x; j < kMcWidth - kMcStyle; j += blockDim.x)
    mc16[row * kMcWidth + kMcStyle + j] = (half_t)(j < 192 ? style[(size_t)b * 192 + j] : 0.0f);
}

hipError_t launch_step_prep(const float* x, const float* prompt_x, const float* cond,
                            const float* style, int B, int T, half_t* xmel16, half_t* cond16,
                            half_t* mc16, hipStream_t s) {
  hipLaunchKernelGGL(step_prep_kernel, dim3(T, B), dim3(256), 0, s, x, prompt_x, cond, style, T,
                     xmel16, cond16, mc16);
  return hipGetLastError();
}

// ---------------------------------------------------------------- conv2 (+ Euler)
// One wavefront computes a 16-token x 80-channel block of conv2 (five 16-wide
// MFMA column blocks, K = 512) for one or two branches.
__device__ __forceinline__ void conv2_block(const half_t* __restrict__ y16, size_t row0, int nvalid,
                                            const half_t* __restrict__ w2, int lr, int lg,
                                            floatx4 acc[5]) {
#pragma unroll
  for (int nb = 0; nb < 5; ++nb) acc[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int ks = 0; ks < 16; ++ks) {
    half8 a = {};
    if (lr < nvalid) a = *reinterpret_cast<const half8*>(y16 + (row0 + lr) * 512 + ks * 32 + lg * 8);
#pragma unroll
    for (int nb = 0; nb < 5; ++nb) {
      const half8 bw =
          *reinterpret_cast<const half8*>(w2 + (size_t)(nb * 16 + lr) * 512 + ks * 32 + lg * 8);
      acc[nb] = mfma16x16x32(a, bw, acc[nb]);
    }
  }
}

// conv2 + CFG blend + Euler update.  One workgroup per 16-token block of
// one request: wave w computes the partial product over K = [128 w, 128 w +
// 128) for both branches (five 16-wide MFMA column blocks each), the
// partials meet in LDS, and the 256 threads apply the update to the
// 16 x 80 block.
__global__ __launch_bounds__(256) void conv2_euler_kernel(
    const half_t* __restrict__ y16, const half_t* __restrict__ w2, const float* __restrict__ b2,
    const uint32_t* __restrict__ P, int T, int cfg_on, float cfg, float dt,
    float* __restrict__ x_cur, half_t* __restrict__ xmel16, float* __restrict__ vtrace) {
  // red[wave][branch][block nb][lane][i]: partial of token 4*(lane/16)+i, channel 16*nb + lane%16
  __shared__ float red[4][2][5][64][4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * 16;
  const int r = blockIdx.y;
  const int nvalid = min(16, T - t0);
  const int bc = cfg_on ? 2 * r : r;
  const int nbr = cfg_on ? 2 : 1;
  // Every operand this lane needs is requested up front (the weights once for
  // both branches, the rows clamped to the last valid one), then the
  // products run; loaded where they were used, each K step waited for its
  // own loads.
  half8 bw[4][5], av[2][4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int k = wave * 128 + ks * 32 + lg * 8;
#pragma unroll
    for (int nb = 0; nb < 5; ++nb) bw[ks][nb] = *reinterpret_cast<const half8*>(w2 + (size_t)(nb * 16 + lr) * 512 + k);
#pragma unroll
    for (int br = 0; br < 2; ++br) {
      const size_t row = (size_t)(bc + (br < nbr ? br : 0)) * T + t0 + min(lr, nvalid - 1);
      av[br][ks] = *reinterpret_cast<const half8*>(y16 + row * 512 + k);
    }
  }
#pragma unroll
  for (int br = 0; br < 2; ++br) {
    if (br >= nbr) break;
    floatx4 acc[5];
#pragma unroll
    for (int nb = 0; nb < 5; ++nb) acc[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      half8 a = av[br][ks];
      if (lr >= nvalid) a = half8{};
#pragma unroll
      for (int nb = 0; nb < 5; ++nb) acc[nb] = mfma16x16x32(a, bw[ks][nb], acc[nb]);
    }
#pragma unroll
    for (int nb = 0; nb < 5; ++nb)
      *reinterpret_cast<floatx4*>(&red[wave][br][nb][lane][0]) = acc[nb];
  }
  // The update's state (5 values per thread) is read before any of it is written.
  constexpr int kPer = 16 * 80 / 256;
  float xo[kPer], bo[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int idx = threadIdx.x + 256 * u;
    const int tok = idx / 80;
    const int n = idx - tok * 80;
    const int t = min(t0 + tok, T - 1);
    xo[u] = x_cur[((size_t)r * T + t) * 80 + n];
    bo[u] = b2[n];
  }
  __syncthreads();
  const uint32_t Pr = P[r];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int idx = threadIdx.x + 256 * u;
    const int tok = idx / 80;
    const int n = idx - tok * 80;
    const int t = t0 + tok;
    if (t >= T) continue;
    const int nb = n >> 4, ln = (tok >> 2) * 16 + (n & 15), i = tok & 3;
    const float bias = bo[u];
    float v = bias;
#pragma unroll
    for (int w = 0; w < 4; ++w) v += red[w][0][nb][ln][i];
    if (cfg_on) {
      float u = bias;
#pragma unroll
      for (int w = 0; w < 4; ++w) u += red[w][1][nb][ln][i];
      v = (1.0f + cfg) * v - cfg * u;
    }
    const size_t xi = ((size_t)r * T + t) * 80 + n;
    if (vtrace) vtrace[xi] = v;
    float xn = xo[u] + dt * v;
    if ((uint32_t)t < Pr) xn = 0.0f;
    x_cur[xi] = xn;
    xmel16[((size_t)bc * T + t) * kMelPad + n] = (half_t)xn;
    if (cfg_on) xmel16[((size_t)(bc + 1) * T + t) * kMelPad + n] = (half_t)xn;
  }
}

hipError_t launch_conv2_euler(const half_t* y16, const half_t* w2, const float* b2,
                              const uint32_t* P, int nreq, int T, int cfg_on, float cfg, float dt,
                              float* x_cur, half_t* xmel16, float* vtrace, hipStream_t s) {
  hipLaunchKernelGGL(conv2_euler_kernel, dim3((T + 15) / 16, nreq), dim3(256), 0, s, y16, w2, b2, P,
                     T, cfg_on, cfg, dt, x_cur, xmel16, vtrace);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void conv2_rows_kernel(const half_t* __restrict__ y16,
                                                         const half_t* __restrict__ w2,
                                                         const float* __restrict__ b2, int rows,
                                                         float* __restrict__ dphi) {
  const int lane = threadIdx.x & 63;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 16;
  if (m0 >= rows) return;
  const int nvalid = min(16, rows - m0);
  floatx4 acc[5];
  conv2_block(y16, (size_t)m0, nvalid, w2, lr, lg, acc);
#pragma unroll
  for (int nb = 0; nb < 5; ++nb) {
    const int n = nb * 16 + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + lg * 4 + i;
      if (m < rows) dphi[(size_t)m * 80 + n] = acc[nb][i] + b2[n];
    }
  }
}

hipError_t launch_conv2_rows(const half_t* y16, const half_t* w2, const float* b2, int rows,
                             float* dphi, hipStream_t s) {
  hipLaunchKernelGGL(conv2_rows_kernel, dim3((rows + 63) / 64), dim3(256), 0, s, y16, w2, b2, rows,
                     dphi);
  return hipGetLastError();
}

// ---------------------------------------------------------------- t-tables
__global__ void timestep_embedding_kernel(const float* __restrict__ tvals,
                                          const float* __restrict__ freqs, int S,
                                          float* __restrict__ temb) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= S * 128) return;
  const int s = i / 128, f = i % 128;
  const float arg = 1000.0f * tvals[s] * freqs[f];
  temb[s * 256 + f] = cosf(arg);
  temb[s * 256 + 128 + f] = sinf(arg);
}

hipError_t launch_timestep_embedding(const float* tvals, const float* freqs, int S, float* temb,
                                     hipStream_t s) {
  hipLaunchKernelGGL(timestep_embedding_kernel, dim3((S * 128 + 255) / 256), dim3(256), 0, s, tvals,
                     freqs, S, temb);
  return hipGetLastError();
}

// One wavefront per output feature n; lanes split K (coalesced W row reads);
// the row stays in registers across the S inputs.
__global__ __launch_bounds__(256) void linear_small_kernel(const float* __restrict__ in, int S,
                                                           int K, const float* __restrict__ W,
                                                           const float* __restrict__ bias, int N,
                                                           int silu_in, int silu_out,
                                                           float* __restrict__ out, int ldout) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  float w[8];
  const int kper = K / 64;  // K is a multiple of 64 and at most 512
  // Loads through buffer resources, issued with no branch around them (a load
  // inside a branch waited for the one before it): a position past the
  // operand reads zero; one past its row (j >= K / 64) is loaded and not
  // summed.  Four steps' inputs are requested together, so a step costs a
  // quarter of an L2 round trip instead of a whole one.  The host keeps N K
  // and S K below 2^29.
  const buffer_rsrc_t rW = make_buffer_rsrc(W, N * K * 4);
  const buffer_rsrc_t rI = make_buffer_rsrc(in, S * K * 4);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float wv = buffer_load_f32(rW, (n * K + j * 64 + lane) * 4);
    w[j] = j < kper ? wv : 0.0f;
  }
  constexpr int kSteps = 4;
  for (int s0 = 0; s0 < S; s0 += kSteps) {
    float xs[kSteps][8];
#pragma unroll
    for (int u = 0; u < kSteps; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        xs[u][j] = buffer_load_f32(rI, ((s0 + u) * K + j * 64 + lane) * 4);
#if defined(__HIP_DEVICE_COMPILE__)
        __asm__("" : "+v"(xs[u][j]));  // keep the load out of the branches below
#endif
      }
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const int st = s0 + u;
      if (st >= S) break;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j < kper) {
          float xv = xs[u][j];
          if (silu_in) xv = xv / (1.0f + expf(-xv));
          acc += w[j] * xv;
        }
      }
      acc = warp_sum(acc);
      if (lane == 0) {
        float v = acc + (bias ? bias[n] : 0.0f);
        if (silu_out) v = v / (1.0f + expf(-v));
        out[(size_t)st * ldout + n] = v;
      }
    }
  }
}

hipError_t launch_linear_small(const float* in, int S, int K, const float* W, const float* bias,
                               int N, int silu_in, int silu_out, float* out, int ldout,
                               hipStream_t s) {
  if (K % 64 != 0 || K > 512 || S <= 0 || (size_t)N * K >= (size_t(1) << 29) ||
      ((size_t)S + 4) * K >= (size_t(1) << 29))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(linear_small_kernel, dim3((N + 3) / 4), dim3(256), 0, s, in, S, K, W, bias, N,
                     silu_in, silu_out, out, ldout);
  return hipGetLastError();
}

__global__ void copy_f32_kernel(const float* __restrict__ src, float* __restrict__ dst, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t j = i; j < n; j += stride) dst[j] = src[j];
}

hipError_t launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(copy_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, n);
  return hipGetLastError();
}

__global__ void zero_kernel(uint4* __restrict__ p, size_t n16, unsigned char* __restrict__ tail,
                            size_t ntail) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t j = i; j < n16; j += stride) p[j] = make_uint4(0, 0, 0, 0);
  if (i < ntail) tail[i] = 0;
}

hipError_t launch_zero(void* p, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  const size_t n16 = bytes / 16;
  const size_t ntail = bytes - n16 * 16;
  size_t blocks = (n16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                     reinterpret_cast<uint4*>(p), n16,
                     reinterpret_cast<unsigned char*>(p) + n16 * 16, ntail);
  return hipGetLastError();
}

}  // namespace mit2hip
