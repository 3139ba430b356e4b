// attention.hip -- flash-style masked multi-head attention over mel frames
// (gfx950), head_dim 64, 8 heads.
//
// Replaces the reference's Metal attention (kernels.metal:2625-2807, launched
// from runtime/metal_context.mm:4895-4925) whose CPU definition is
// cpu_attention_single_head_masked (runtime/impl/tokenizer_tests.cpp:3960):
// softmax over unmasked keys of (q.k)/8, then the weighted sum of V.
//
// Layout: Q, K are [B][8][Tpad][64] f16 (Q already scaled by 1/8 and both
// RoPE-rotated by the QKV GEMM epilogue); V is stored transposed,
// Vt [B][8][64][Tpad].  Output O is token-major [B*T][512] f16, heads
// concatenated in head order.
//
// One workgroup = 4 wavefronts = 64 queries of one (branch, head).  Each
// wavefront owns 16 queries and walks the keys in tiles of 64 staged in LDS:
//   S^T(64 keys x 16 queries) = K . Q^T      8 MFMA 16x16x32
//   online softmax per query (column): the 4 lanes sharing a query exchange
//   max / sum with two xor-shuffles
//   O(16 x 64) += P . V                      8 MFMA 16x16x32
// Computing S transposed puts each query's probabilities in the lane that
// the P.V MFMA expects as its A-operand row, so P never leaves registers.
// A query whose keys are all masked produces zeros.
#include "device_common.h"

namespace mit2hip {

constexpr int kAttnTile = 64;
constexpr int kAttnLds = 72;  // halves per LDS row (64 + 8 pad)

__global__ __launch_bounds__(256) void attention_kernel(const half_t* __restrict__ Q,
                                                        const half_t* __restrict__ K,
                                                        const half_t* __restrict__ Vt,
                                                        const uint32_t* __restrict__ mask,
                                                        half_t* __restrict__ O, int T, int Tpad) {
  __shared__ __attribute__((aligned(16))) half_t Ks[kAttnTile * kAttnLds];
  __shared__ __attribute__((aligned(16))) half_t Vs[64 * kAttnLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int b = blockIdx.z;
  const int h = blockIdx.y;
  const int q0 = blockIdx.x * 64 + wave * 16;
  const size_t head = (size_t)b * 8 + h;
  const half_t* Qh = Q + head * Tpad * 64;
  const half_t* Kh = K + head * Tpad * 64;
  const half_t* Vh = Vt + head * 64 * Tpad;
  const uint32_t* mrow = mask + (size_t)b * T;

  // B operand of S^T = K.Q^T: this lane's query row, d-slots of lane group lg.
  const half8 qf0 = *reinterpret_cast<const half8*>(Qh + (size_t)(q0 + lr) * 64 + lg * 8);
  const half8 qf1 = *reinterpret_cast<const half8*>(Qh + (size_t)(q0 + lr) * 64 + 32 + lg * 8);

  floatx4 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max for query lr (identical in the 4 lanes of the query)
  float l_run = 0.0f;       // running denominator

  const int ntiles = Tpad / kAttnTile;
  for (int kt = 0; kt < ntiles; ++kt) {
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * 256;
      const int row = c >> 3;
      const int ch = c & 7;
      *reinterpret_cast<half8*>(&Ks[row * kAttnLds + ch * 8]) =
          *reinterpret_cast<const half8*>(Kh + (size_t)(kt * kAttnTile + row) * 64 + ch * 8);
      // V^T columns past T are padding: zero them so 0-probability keys add 0.
      half8 vv = *reinterpret_cast<const half8*>(Vh + (size_t)row * Tpad + kt * kAttnTile + ch * 8);
      const int kbase = kt * kAttnTile + ch * 8;
      if (kbase + 8 > T) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (kbase + e >= T) vv[e] = (half_t)0.0f;
      }
      *reinterpret_cast<half8*>(&Vs[row * kAttnLds + ch * 8]) = vv;
    }
    __syncthreads();

    // Scores: s[kb][i] = S[key = kt*64 + kb*16 + 4*lg + i][query = q0 + lr]
    floatx4 s[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const half8 kf0 = *reinterpret_cast<const half8*>(&Ks[(kb * 16 + lr) * kAttnLds + lg * 8]);
      const half8 kf1 =
          *reinterpret_cast<const half8*>(&Ks[(kb * 16 + lr) * kAttnLds + 32 + lg * 8]);
      floatx4 z = {0.f, 0.f, 0.f, 0.f};
      z = mfma16x16x32(kf0, qf0, z);
      s[kb] = mfma16x16x32(kf1, qf1, z);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt * kAttnTile + kb * 16 + lg * 4 + i;
        const bool valid = key < T && mrow[key] != 0;
        const float v = valid ? s[kb][i] : -INFINITY;
        s[kb][i] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    const float m_new = fmaxf(m_run, tmax);
    // All keys so far masked: keep everything at zero.
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = __expf(m_run - m_use);  // m_run = -inf -> 0
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = __expf(s[kb][i] - m_use);  // masked -> exp(-inf) = 0
        s[kb][i] = pv;
        psum += pv;
      }
    }
    psum += __shfl_xor(psum, 16, kWave);
    psum += __shfl_xor(psum, 32, kWave);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // Rescale O rows: lane holds O[query 4*lg + i][d]; fetch that query's alpha.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ai = __shfl(alpha, lg * 4 + i, kWave);
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db][i] *= ai;
    }

    // O += P . V over two 32-key chunks.  K-slot j of lane group lg maps to
    // key 32c + 4*lg + j (j < 4) and 32c + 16 + 4*lg + (j - 4) (j >= 4), the
    // keys this lane's P values belong to; V^T is read with the same map.
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      half8 pa;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pa[j] = (half_t)s[2 * c][j];
        pa[4 + j] = (half_t)s[2 * c + 1][j];
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const half_t* vrow = &Vs[(db * 16 + lr) * kAttnLds + c * 32 + lg * 4];
        const half4 v0 = *reinterpret_cast<const half4*>(vrow);
        const half4 v1 = *reinterpret_cast<const half4*>(vrow + 16);
        half8 vb;
        vb[0] = v0[0]; vb[1] = v0[1]; vb[2] = v0[2]; vb[3] = v0[3];
        vb[4] = v1[0]; vb[5] = v1[1]; vb[6] = v1[2]; vb[7] = v1[3];
        o[db] = mfma16x16x32(pa, vb, o[db]);
      }
    }
  }

  // Normalise and store: lane holds O[query q0 + 4*lg + i][d = 16*db + lr].
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = q0 + lg * 4 + i;
    const float li = __shfl(l_run, lg * 4 + i, kWave);
    if (q >= T) continue;
    const float inv = li > 0.0f ? 1.0f / li : 0.0f;
    half_t* dst = O + ((size_t)b * T + q) * 512 + h * 64;
#pragma unroll
    for (int db = 0; db < 4; ++db) dst[db * 16 + lr] = (half_t)(o[db][i] * inv);
  }
}

hipError_t launch_attention(const half_t* Q, const half_t* K, const half_t* Vt,
                            const uint32_t* mask, half_t* O, int B, int T, int Tpad,
                            hipStream_t stream) {
  if (B <= 0 || T <= 0 || Tpad < T || Tpad % kAttnTile != 0) return hipErrorInvalidValue;
  dim3 grid((T + 63) / 64, 8, B);
  hipLaunchKernelGGL(attention_kernel, grid, dim3(256), 0, stream, Q, K, Vt, mask, O, T, Tpad);
  return hipGetLastError();
}

}  // namespace mit2hip
