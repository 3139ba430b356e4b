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
// One workgroup = 4 wavefronts = 64 queries of one (branch, head).  Keys are
// consumed in tiles of 64: the K tile, the V^T tile and the tile's key-mask
// words are copied global -> LDS with direct loads into a ring of NBUF
// buffers, so NBUF-1 tiles are in flight while one is computed.  Per wavefront
// (16 queries) and tile:
//   S^T(64 keys x 16 queries) = K . Q^T        8 MFMA 16x16x32
//   running max per query: two xor-shuffles (the 4 lanes sharing a query)
//   O^T(64 d x 16 queries) += V^T . P^T        8 MFMA 16x16x32
// Computing both products transposed leaves every query's probabilities,
// running denominator and 64 outputs in the lanes of that query, so the
// rescale by exp(m_old - m_new) and the denominator are lane-local and only
// the max crosses lanes.  A query whose keys are all masked produces zeros.
#include <type_traits>

#include "device_common.h"

namespace mit2hip {

constexpr int kAttnBuffers = 2;  // K/V^T tile buffers per key group (1 in flight)
constexpr int kAttnSplitMaxTpad = 2048;  // longest padded sequence that splits its keys

typedef __attribute__((address_space(3))) void attn_lds_t;

template <int N>
__device__ __forceinline__ void attn_wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void attn_wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (0 << 8));
}

// 16-byte slot of chunk c in a 128-byte LDS row r (8 slots): conflict-free
// ds_read_b128 for 16 consecutive rows at one chunk.
__device__ __forceinline__ int attn_slot(int r, int c) { return c ^ ((r >> 1) & 7); }

template <int I, int N, typename F>
__device__ __forceinline__ void attn_static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    attn_static_for<I + 1, N>(f);
  }
}

template <int NBUF, int SPLIT>
__global__ __launch_bounds__(256 * SPLIT) void attention_kernel(const half_t* __restrict__ Q,
                                                        const half_t* __restrict__ K,
                                                        const half_t* __restrict__ Vt,
                                                        const uint32_t* __restrict__ mask,
                                                        half_t* __restrict__ O, int T, int Tpad) {
  static_assert(NBUF >= 2 && NBUF <= 4, "2..4 tile buffers");
  static_assert(SPLIT == 1 || SPLIT == 2 || SPLIT == 4, "key split");
  // One __shared__ object per buffer (K, V^T, and one mask copy per wave);
  // each key group g has its own region inside every buffer.
  constexpr int KV = 64 * 64 * SPLIT;
  __shared__ __attribute__((aligned(1024))) half_t sK0[KV];
  __shared__ __attribute__((aligned(1024))) half_t sK1[KV];
  __shared__ __attribute__((aligned(1024))) half_t sK2[NBUF > 2 ? KV : 8];
  __shared__ __attribute__((aligned(1024))) half_t sK3[NBUF > 3 ? KV : 8];
  __shared__ __attribute__((aligned(1024))) half_t sV0[KV];
  __shared__ __attribute__((aligned(1024))) half_t sV1[KV];
  __shared__ __attribute__((aligned(1024))) half_t sV2[NBUF > 2 ? KV : 8];
  __shared__ __attribute__((aligned(1024))) half_t sV3[NBUF > 3 ? KV : 8];
  __shared__ __attribute__((aligned(1024))) uint32_t sM0[4 * 64 * SPLIT];
  __shared__ __attribute__((aligned(1024))) uint32_t sM1[4 * 64 * SPLIT];
  __shared__ __attribute__((aligned(1024))) uint32_t sM2[NBUF > 2 ? 4 * 64 * SPLIT : 4];
  __shared__ __attribute__((aligned(1024))) uint32_t sM3[NBUF > 3 ? 4 * 64 * SPLIT : 4];
  // (m, l, O) of key group 1 for the two-group merge: 4 waves x 64 lanes x
  // 18 floats.  With four groups, groups 1..3 park in the K0 / V0 / K1 tile
  // buffers instead (each holds 32 KB then), which are free after the loop.
  __shared__ __attribute__((aligned(1024))) float sPark[SPLIT == 2 ? 4 * 64 * 18 : 4];
  auto bufK = [&](auto st) -> half_t* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sK0; else if constexpr (s == 1) return sK1;
    else if constexpr (s == 2) return sK2; else return sK3;
  };
  auto bufV = [&](auto st) -> half_t* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sV0; else if constexpr (s == 1) return sV1;
    else if constexpr (s == 2) return sV2; else return sV3;
  };
  auto bufM = [&](auto st) -> uint32_t* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sM0; else if constexpr (s == 1) return sM1;
    else if constexpr (s == 2) return sM2; else return sM3;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = (tid >> 6) & 3;  // query block of this wave within the workgroup
  const int grp = tid >> 8;         // key group (SPLIT groups share the 64 queries)
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
  const int ntiles = Tpad / 64;
  // Key group grp walks tiles [grp*tpg, grp*tpg + tpg); tiles past the end
  // are loaded clamped and contribute nothing (every key >= T is masked), so
  // all groups run the same iterations and meet at the same barriers.
  const int tpg = (ntiles + SPLIT - 1) / SPLIT;
  const int tbase = grp * tpg;

  // Each wave moves 2 KB of K, 2 KB of V^T and its own 256-byte mask copy:
  // 5 direct loads per wave per tile.
  auto issue = [&](auto st, int j) {
    const int kt = min(tbase + j, ntiles - 1);
    half_t* sk = bufK(st) + grp * 64 * 64;
    half_t* sv = bufV(st) + grp * 64 * 64;
    uint32_t* sm = bufM(st) + grp * 256;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int qq0 = (wave * 2 + j) * 64;
      const int q = qq0 + lane;
      const int row = q >> 3;
      const int c = attn_slot(row, q & 7);
      __builtin_amdgcn_global_load_lds((const void*)(Kh + (size_t)(kt * 64 + row) * 64 + c * 8),
                                       (attn_lds_t*)(sk + qq0 * 8), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(Vh + (size_t)row * Tpad + kt * 64 + c * 8),
                                       (attn_lds_t*)(sv + qq0 * 8), 16, 0, 0);
    }
    const int key = min(kt * 64 + lane, T - 1);  // keys >= T are rejected at use
    __builtin_amdgcn_global_load_lds((const void*)(mrow + key), (attn_lds_t*)(sm + wave * 64), 4, 0,
                                     0);
  };

  // B operand of S^T = K.Q^T: this lane's query row, d-slots of lane group lg.
  const half8 qf0 = *reinterpret_cast<const half8*>(Qh + (size_t)(q0 + lr) * 64 + lg * 8);
  const half8 qf1 = *reinterpret_cast<const half8*>(Qh + (size_t)(q0 + lr) * 64 + 32 + lg * 8);

  floatx4 o[4];  // o[db][i] = O[query q0+lr][d = 16*db + 4*lg + i] (unnormalised)
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max of query lr (same in its 4 lanes)
  float l_run = 0.0f;       // this lane's share of the running denominator

  auto compute = [&](auto st, int j) {
    const int kt = tbase + j;  // unclamped: a tile past the end has every key >= T
    const half_t* sk = bufK(st) + grp * 64 * 64;
    const half_t* sv = bufV(st) + grp * 64 * 64;
    const uint32_t* sm = bufM(st) + grp * 256 + wave * 64;
    // Scores: sc[kb][i] = S[key kt*64 + kb*16 + 4*lg + i][query q0 + lr]
    floatx4 sc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int row = kb * 16 + lr;
      const half8 kf0 = *reinterpret_cast<const half8*>(sk + row * 64 + attn_slot(row, lg) * 8);
      const half8 kf1 = *reinterpret_cast<const half8*>(sk + row * 64 + attn_slot(row, 4 + lg) * 8);
      floatx4 z = {0.f, 0.f, 0.f, 0.f};
      z = mfma16x16x32(kf0, qf0, z);
      sc[kb] = mfma16x16x32(kf1, qf1, z);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const uint4 mk = *reinterpret_cast<const uint4*>(sm + kb * 16 + lg * 4);
      const uint32_t mv[4] = {mk.x, mk.y, mk.z, mk.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt * 64 + kb * 16 + lg * 4 + i;
        const bool valid = (key < T) & (mv[i] != 0u);
        const float v = valid ? sc[kb][i] : -INFINITY;
        sc[kb][i] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;  // all keys so far masked
    const float alpha = __expf(m_run - m_use);                  // m_run = -inf -> 0
    float psum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = __expf(sc[kb][i] - m_use);  // masked -> 0
        sc[kb][i] = pv;
        psum += pv;
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] *= alpha;
    // O^T += V^T . P^T over two 32-key chunks.  K-slot j of lane group lg is
    // key 32c + 4*lg + j (j < 4) or 32c + 16 + 4*lg + (j - 4) (j >= 4): the
    // keys this lane's probabilities belong to; V^T rows are read with the
    // same map.
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      half8 pb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pb[j] = (half_t)sc[2 * c][j];
        pb[4 + j] = (half_t)sc[2 * c + 1][j];
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int row = db * 16 + lr;
        const int k0 = c * 32 + lg * 4;       // keys k0..k0+3 and k0+16..k0+19
        const half4 v0 = *reinterpret_cast<const half4*>(
            sv + row * 64 + attn_slot(row, k0 >> 3) * 8 + (k0 & 7));
        const half4 v1 = *reinterpret_cast<const half4*>(
            sv + row * 64 + attn_slot(row, (k0 + 16) >> 3) * 8 + (k0 & 7));
        half8 va;
        va[0] = v0[0]; va[1] = v0[1]; va[2] = v0[2]; va[3] = v0[3];
        va[4] = v1[0]; va[5] = v1[1]; va[6] = v1[2]; va[7] = v1[3];
        o[db] = mfma16x16x32(va, pb, o[db]);
      }
    }
  };

  // NBUF-buffer pipeline.  The steady-state body is branch-free (the issue
  // past the last tile repeats the last tile into a buffer that is not read
  // again), so the compiler keeps only the explicit vmcnt waits; the last
  // ntiles % NBUF tiles are already resident when the loop exits.
  attn_static_for<0, NBUF - 1>([&](auto st) { issue(st, min((int)decltype(st)::value, tpg - 1)); });
  attn_wait_vmcnt<5 * (NBUF - 1)>();  // the Q fragments (issued before the prologue) have landed
  int kt0 = 0;
  for (; kt0 + NBUF <= tpg; kt0 += NBUF) {
    attn_static_for<0, NBUF>([&](auto st) {
      constexpr int s = decltype(st)::value;
      attn_wait_lgkmcnt0();
      __builtin_amdgcn_s_barrier();
      issue(std::integral_constant<int, (s + NBUF - 1) % NBUF>{}, min(kt0 + s + NBUF - 1, tpg - 1));
      attn_wait_vmcnt<5 * (NBUF - 1)>();
      __builtin_amdgcn_s_barrier();
      compute(st, kt0 + s);
    });
  }
  attn_wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  attn_static_for<0, NBUF - 1>([&](auto st) {
    if (kt0 + (int)decltype(st)::value < tpg) compute(st, kt0 + decltype(st)::value);
  });

  // Denominator: sum of the 4 lane shares of the query.
  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
  if constexpr (SPLIT > 1) {
    // Merge the key groups: groups 1.. park (m, l, O) in LDS; group 0
    // rescales every part to the common max.
    auto park_of = [&](int g) -> float* {
      if constexpr (SPLIT == 2) {
        return sPark + (wave * 64 + lane) * 18;
      } else {
        float* base = reinterpret_cast<float*>(g == 1 ? sK0 : g == 2 ? sV0 : sK1);
        return base + (wave * 64 + lane) * 18;
      }
    };
    if constexpr (SPLIT == 4) {
      // every wave's last tile reads are done before tile buffers are reused
      attn_wait_lgkmcnt0();
      __syncthreads();
    }
    if (grp > 0) {
      float* p = park_of(grp);
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[db * 4 + i] = o[db][i];
      p[16] = m_run;
      p[17] = l_run;
    }
    attn_wait_lgkmcnt0();  // the parked values are in LDS before any wave passes the barrier
    __builtin_amdgcn_s_barrier();
    if (grp > 0) return;
    float mstar = m_run;
#pragma unroll
    for (int g = 1; g < SPLIT; ++g) mstar = fmaxf(mstar, park_of(g)[16]);
    const float mref = mstar == -INFINITY ? 0.0f : mstar;
    const float w0 = __expf(m_run - mref);
    l_run *= w0;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] *= w0;
#pragma unroll
    for (int g = 1; g < SPLIT; ++g) {
      const float* p = park_of(g);
      const float wg = __expf(p[16] - mref);
      l_run += wg * p[17];
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[db][i] += wg * p[db * 4 + i];
    }
  }
  const int q = q0 + lr;
  if (q < T) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    half_t* dst = O + ((size_t)b * T + q) * 512 + h * 64 + lg * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      half4 v;
      v[0] = (half_t)(o[db][0] * inv);
      v[1] = (half_t)(o[db][1] * inv);
      v[2] = (half_t)(o[db][2] * inv);
      v[3] = (half_t)(o[db][3] * inv);
      *reinterpret_cast<half4*>(dst + db * 16) = v;
    }
  }
}

hipError_t launch_attention(const half_t* Q, const half_t* K, const half_t* Vt,
                            const uint32_t* mask, half_t* O, int B, int T, int Tpad,
                            hipStream_t stream) {
  if (B <= 0 || T <= 0 || Tpad < T || Tpad % 64 != 0) return hipErrorInvalidValue;
  dim3 grid((T + 63) / 64, 8, B);
  // Short and medium sequences give few query tiles and leave most SIMDs with
  // one wave: split the keys of each workgroup over two wave groups (a
  // four-group split, also built, measured slower at T = 860 on MI355X).
  // The choice depends on the sequence length only, never on the batch, so a
  // request's output does not depend on what it is batched with.
  if (Tpad <= kAttnSplitMaxTpad)
    hipLaunchKernelGGL((attention_kernel<kAttnBuffers, 2>), grid, dim3(512), 0, stream, Q, K, Vt,
                       mask, O, T, Tpad);
  else
    hipLaunchKernelGGL((attention_kernel<kAttnBuffers, 1>), grid, dim3(256), 0, stream, Q, K, Vt,
                       mask, O, T, Tpad);
  return hipGetLastError();
}

}  // namespace mit2hip
