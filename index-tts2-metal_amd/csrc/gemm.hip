// gemm.hip -- f16 MFMA GEMM (gfx950) with the decoder's fused epilogues.
//
// Replaces the reference's MPS GEMM dispatch (runtime/metal_context.mm:328-378)
// and the kernels fused around it (bias pre-fill kernels.metal:227, residual
// add :161, SwiGLU :131, WaveNet gate :411, res/skip update :436, RoPE :2390).
//
// Tiling: a 256-thread workgroup (4 wavefronts in a 2x2 grid) owns a BM x BN
// output tile; K advances 32 at a time.  Global -> register prefetch of tile
// k+1 overlaps the MFMAs of tile k, and LDS is double buffered so there is a
// single barrier per K step.  LDS rows are padded to 40 halves (80 bytes) so
// the 16 lanes of each 128-bit fragment read hit 64 distinct banks.
#include "gemm.h"

namespace mit2hip {

constexpr int kBK = 32;
constexpr int kLdsStride = kBK + 8;  // halves per LDS row

template <int BM, int BN, int AM, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  constexpr int MI = BM / 32;  // 16-row MFMA blocks per wave (2 waves along M)
  constexpr int NI = BN / 32;  // 16-col MFMA blocks per wave (2 waves along N)
  constexpr int A_CHUNKS = BM * 4 / 256;
  constexpr int B_CHUNKS = BN * 4 / 256;
  static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) half_t As[2][BM * kLdsStride];
  __shared__ __attribute__((aligned(16))) half_t Bs[2][BN * kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int n0 = blockIdx.x * BN;
  const int m0 = blockIdx.y * BM;
  const int KT = p.K / kBK;

  half8 ra[A_CHUNKS];
  half8 rb[B_CHUNKS];

  auto load_tiles = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + i * 256;
      const int r = c >> 2;
      const int kc = c & 3;
      const int m = m0 + r;
      half8 v = {};
      if (m < p.M) {
        const half_t* src;
        if constexpr (AM == A_PLAIN) {
          src = p.A + (size_t)m * p.lda + k0 + kc * 8;
        } else if constexpr (AM == A_CONCAT) {
          src = (k0 < p.K1) ? p.A + (size_t)m * p.lda + k0 + kc * 8
                            : p.A2 + (size_t)m * p.lda2 + (k0 - p.K1) + kc * 8;
        } else {
          const int tap = k0 / p.conv_c;
          const int c0 = k0 - tap * p.conv_c;
          const int b = m / p.T;
          const int t = m - b * p.T;
          const int s = reflect_index(t + tap - 2, p.T);
          src = p.A + (size_t)(b * p.T + s) * p.lda + c0 + kc * 8;
        }
        v = *reinterpret_cast<const half8*>(src);
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + i * 256;
      const int r = c >> 2;
      const int kc = c & 3;
      rb[i] = *reinterpret_cast<const half8*>(p.W + (size_t)(n0 + r) * p.ldw + k0 + kc * 8);
    }
  };

  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<half8*>(&As[buf][(c >> 2) * kLdsStride + (c & 3) * 8]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<half8*>(&Bs[buf][(c >> 2) * kLdsStride + (c & 3) * 8]) = rb[i];
    }
  };

  floatx4 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load_tiles(kt + 1);
    half8 af[MI];
    half8 bf[NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
      af[i] = *reinterpret_cast<const half8*>(
          &As[buf][(wm * (BM / 2) + i * 16 + lr) * kLdsStride + lg * 8]);
#pragma unroll
    for (int j = 0; j < NI; ++j)
      bf[j] = *reinterpret_cast<const half8*>(
          &Bs[buf][(wn * (BN / 2) + j * 16 + lr) * kLdsStride + lg * 8]);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
    if (kt + 1 < KT) store_tiles(buf ^ 1);
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
  const int row_base = m0 + wm * (BM / 2) + lg * 4;
  const int col_base = n0 + wn * (BN / 2);

  if constexpr (EPI == EPI_F32 || EPI == EPI_F16 || EPI == EPI_DUAL || EPI == EPI_RESSKIP ||
                EPI == EPI_FINALSKIP) {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = row_base + i * 16 + r;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int n = col_base + j * 16 + lr;
          float v = acc[i][j][r];
          if (p.bias) v += p.bias[n];
          if constexpr (EPI == EPI_F32) {
            if (p.res) v = p.res[(size_t)m * p.ldres + n] + v;
            p.C32[(size_t)m * p.ldc32 + n] = v;
            if (p.C16) p.C16[(size_t)m * p.ldc16 + n] = (half_t)v;
          } else if constexpr (EPI == EPI_F16) {
            p.C16[(size_t)m * p.ldc16 + n] = (half_t)v;
          } else if constexpr (EPI == EPI_DUAL) {
            const int half_n = p.N >> 1;
            if (n < half_n) {
              p.C32[(size_t)m * p.ldc32 + n] = v;
              p.C16[(size_t)m * p.ldc16 + n] = (half_t)v;
            } else {
              p.C32b[(size_t)m * p.ldc32b + (n - half_n)] = v;
            }
          } else if constexpr (EPI == EPI_RESSKIP) {
            // v is the res_skip conv output (bias included).
            const float mk = p.mask[m] ? 1.0f : 0.0f;
            if (n < 512) {
              float* xs = p.C32 + (size_t)m * p.ldc32 + n;
              const float xn = (*xs + v) * mk;
              *xs = xn;
              p.C16[(size_t)m * p.ldc16 + n] = (half_t)xn;
            } else {
              float* os = p.C32b + (size_t)m * p.ldc32b + (n - 512);
              *os = p.flag ? (*os + v) : v;
            }
          } else {  // EPI_FINALSKIP: out = (out + rs) * mask; final_in = out + rp
            const float mk = p.mask[m] ? 1.0f : 0.0f;
            const float o = (p.C32b[(size_t)m * p.ldc32b + n] + v) * mk;
            p.C32[(size_t)m * p.ldc32 + n] = o + p.rp[(size_t)m * 512 + n];
          }
        }
      }
    }
  } else {
    // Paired epilogues: MFMA blocks (2q, 2q+1) of a wave hold, in the same
    // lane, the two operands for output channel c = 16*group + lr.
    static_assert(NI % 2 == 0, "paired epilogue needs an even block count");
#pragma unroll
    for (int q = 0; q < NI / 2; ++q) {
      const int ce = col_base + q * 32;  // GEMM column of the even block start
      const int group = ce >> 5;
      const float be = p.bias ? p.bias[ce + lr] : 0.0f;
      const float bo = p.bias ? p.bias[ce + 16 + lr] : 0.0f;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = row_base + i * 16 + r;
          if (m >= p.M) continue;
          const float ve = acc[i][2 * q][r] + be;
          const float vo = acc[i][2 * q + 1][r] + bo;
          if constexpr (EPI == EPI_SWIGLU) {
            const int c = group * 16 + lr;
            p.C16[(size_t)m * p.ldc16 + c] = (half_t)((ve / (1.0f + __expf(-ve))) * vo);
          } else if constexpr (EPI == EPI_GATE) {
            const int c = group * 16 + lr;
            const float a = ve + p.cond[c];
            const float b = vo + p.cond[512 + c];
            p.C16[(size_t)m * p.ldc16 + c] = (half_t)(tanh_sat(a) * sigmoid_f(b));
          } else {  // EPI_QKV
            const int o = group * 32 + 2 * lr;  // original column of the even element
            const int sec = o >> 9;             // 0 = q, 1 = k, 2 = v
            const int hh = (o & 511) >> 6;
            const int d = o & 63;
            const int b = m / p.T;
            const int t = m - b * p.T;
            const size_t head = (size_t)b * 8 + hh;
            if (sec < 2) {
              const float2 cs = p.rope[t * 32 + (d >> 1)];
              float re = ve * cs.x - vo * cs.y;
              float ro = vo * cs.x + ve * cs.y;
              if (sec == 0) {
                re *= 0.125f;  // 1/sqrt(64): a power of two, so the scaling is exact
                ro *= 0.125f;
              }
              half_t* dst = (sec == 0 ? p.q : p.k) + (head * p.Tpad + t) * 64 + d;
              half2v pr = {(half_t)re, (half_t)ro};
              *reinterpret_cast<half2v*>(dst) = pr;
            } else {
              half_t* dst = p.vt + (head * 64 + d) * p.Tpad + t;
              dst[0] = (half_t)ve;
              dst[p.Tpad] = (half_t)vo;
            }
          }
        }
      }
    }
  }
}

template <int BM, int BN, int AM, int EPI>
static hipError_t launch_tile(const GemmArgs& a, hipStream_t s) {
  dim3 grid(a.N / BN, (a.M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, AM, EPI>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int AM, int EPI>
static hipError_t launch_am_epi(const GemmArgs& a, hipStream_t s) {
  // 64x64 tiles keep >= 200 workgroups in flight at M = 1720 for N = 512;
  // wider N gets 64x128 (fewer A re-reads).
  if (a.N % 128 == 0 && a.N >= 1024) return launch_tile<64, 128, AM, EPI>(a, s);
  return launch_tile<64, 64, AM, EPI>(a, s);
}

template <int AM>
static hipError_t launch_am(const GemmArgs& a, EpiMode epi, hipStream_t s) {
  switch (epi) {
    case EPI_F32: return launch_am_epi<AM, EPI_F32>(a, s);
    case EPI_F16: return launch_am_epi<AM, EPI_F16>(a, s);
    case EPI_SWIGLU: return launch_am_epi<AM, EPI_SWIGLU>(a, s);
    case EPI_GATE: return launch_am_epi<AM, EPI_GATE>(a, s);
    case EPI_QKV: return launch_am_epi<AM, EPI_QKV>(a, s);
    case EPI_RESSKIP: return launch_am_epi<AM, EPI_RESSKIP>(a, s);
    case EPI_FINALSKIP: return launch_am_epi<AM, EPI_FINALSKIP>(a, s);
    case EPI_DUAL: return launch_am_epi<AM, EPI_DUAL>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm(const GemmArgs& a, AMode amode, EpiMode epi, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.K % kBK != 0 || a.N % 64 != 0 || !a.A || !a.W)
    return hipErrorInvalidValue;
  if (amode == A_CONCAT && (a.K1 % kBK != 0 || a.K1 <= 0 || a.K1 >= a.K || !a.A2))
    return hipErrorInvalidValue;
  if (amode == A_CONV5 && (a.T <= 0 || a.conv_c % kBK != 0 || a.K != 5 * a.conv_c))
    return hipErrorInvalidValue;
  switch (amode) {
    case A_PLAIN: return launch_am<A_PLAIN>(a, epi, stream);
    case A_CONCAT: return launch_am<A_CONCAT>(a, epi, stream);
    case A_CONV5: return launch_am<A_CONV5>(a, epi, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mit2hip
