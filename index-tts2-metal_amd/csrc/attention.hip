// attention.hip -- flash-style masked multi-head attention over mel frames
// (gfx950), head_dim 64, 8 heads.
//
// Replaces the reference's Metal attention (kernels.metal:2625-2807, launched
// from runtime/metal_context.mm:4895-4925) whose CPU definition is
// cpu_attention_single_head_masked (runtime/impl/tokenizer_tests.cpp:3960):
// softmax over unmasked keys of (q.k)/8, then the weighted sum of V.
//
// Layout: Q, K are [B][8][Tpad][64] f16 (Q already scaled by log2(e)/8 and
// both RoPE-rotated by the QKV GEMM epilogue); V is stored transposed,
// Vt [B][8][64][Tpad].  The key mask arrives as kbias [B][Tpad] fp32 (0 for
// a valid key, -inf for a masked or padding key; key_bias_kernel builds it
// once per mask, followed by B int words: each branch's key count, one past
// its last valid key).  Output O is token-major [B*T][512] f16, heads
// concatenated in head order.  The BRANCH_KEYS variant stops each branch
// after the tile holding its last valid key.  The tiles it skips are fully
// masked (they would add exact zeros), but the two key groups then split the
// branch's own tile count, so the partial sums associate as they would for
// that branch decoded at its own padded length: the two variants agree to
// rounding, not bit for bit.
//
// Keys are consumed in tiles of 64: the K tile, the V^T tile and the tile's
// bias words are copied global -> LDS with direct loads into a ring of NBUF
// buffers, so NBUF-1 tiles are in flight while one is computed.  Per
// wavefront (32 queries) and tile:
//   S^T(64 keys x 32 queries) = K . Q^T        16 MFMA 16x16x32
//   running max per query: two xor-shuffles (the 4 lanes sharing a query)
//   O^T(64 d x 32 queries) += V^T . P^T        16 MFMA 16x16x32
//   denominator (ones row) . P^T                4 MFMA 16x16x32
// Computing the products transposed leaves every query's probabilities,
// denominator and 64 outputs in the lanes of that query, so the rescale is
// lane-local and only the max crosses lanes.  A query whose keys are all
// masked produces zeros, as the reference Metal kernel does.
#include <type_traits>

#include "device_common.h"

namespace mit2hip {


template <int N>
__device__ __forceinline__ void attn_wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ void attn_wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (0 << 8));
}

template <int I, int N, typename F>
__device__ __forceinline__ void attn_static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    attn_static_for<I + 1, N>(f);
  }
}

// ---------------------------------------------------------------------------
// One wavefront = 32 queries (two 16-query MFMA blocks),
// so every K and V^T fragment read from LDS feeds two MFMAs.  A workgroup is
// G key groups x 2 query waves = 64 queries of one (branch, head); group g
// walks its own share of the key tiles with its own LDS ring, and the groups
// merge (m, l, O) at the end.
//
// Softmax arithmetic per score is what bounds this kernel (the matrix cores
// have slack), so it is kept to a share of a max, an exp2 and a share of
// the f16 pack:
//  * scores are in log2 units (the QKV epilogue scales q by log2(e) / 8),
//    and the QK^T accumulators start at minus the running max, so the
//    matrix cores return s2 - m directly;
//  * the key mask is an additive per-key bias, 0 for a valid key and -inf
//    for a masked or padding key (built once per mask by key_bias_kernel),
//    added only on the tiles that hold a masked key (a ballot over the
//    tile's bias words);
//  * the running max m moves only when a tile's max exceeds it by more than
//    8: probabilities exp2(s2 - m) then stay <= 2^8, well inside f16, and the
//    O rescale is skipped for the whole wave in the common case;
//  * the denominator is a fifth MFMA block whose A operand is a row of ones:
//    l = sum of the f16 probabilities the PV product used, accumulated in
//    fp32 by the matrix core.
//
// Key order inside a 64-key tile.  S^T block kb (16 keys) loads K row
//   krow(kb, r) = 32 (kb >> 1) + 8 (r >> 2) + 4 (kb & 1) + (r & 3)
// into MFMA row r, so the 4 scores a lane holds for blocks 2c and 2c+1 belong
// to the 8 consecutive keys 32 c + 8 lg + (0..7): exactly the K-slots the
// lane supplies to O^T += V^T . P^T, whose V^T fragment is then one 16-byte
// LDS read.  The permutation only reorders the keys within a tile.
//
// LDS swizzles (16-byte slot of chunk c in a 128-byte row r): K rows are read
// in the permuted order, V^T rows in natural order, each with its own key.
__device__ __forceinline__ int attn_kslot(int r, int c) { return c ^ ((r & 3) | (((r >> 3) & 1) << 2)); }
__device__ __forceinline__ int attn_vslot(int r, int c) { return c ^ (r & 7); }

constexpr float kLazyMax = 8.0f;  // log2 headroom before the running max moves

template <int NBUF, int G, int QB, int NQW, bool BRANCH_KEYS, bool QSKIP>
__global__ __launch_bounds__(64 * NQW * G) void attention_kernel(const half_t* __restrict__ Q,
                                                                const half_t* __restrict__ K,
                                                                const half_t* __restrict__ Vt,
                                                                const float* __restrict__ kbias,
                                                                half_t* __restrict__ O, int T, int Tpad) {
  static_assert(NBUF >= 2 && NBUF <= 3, "2..3 tile buffers");
  static_assert(G == 1 || G == 2 || G == 4, "key groups");
  static_assert(QB == 1 || QB == 2, "16-query blocks per wave");
  static_assert(NQW == 1 || NQW == 2 || NQW == 4, "query waves per group");
  static_assert(NQW * QB <= 4, "the merge parks at most 64 queries per group");
  constexpr int TILE = 64 * 64;      // halves in one K or V^T tile
  constexpr int QWG = 16 * QB * NQW; // queries per workgroup
  constexpr int NW = NQW * G;        // waves per workgroup
  __shared__ __attribute__((aligned(1024))) half_t sK0[G * TILE];
  __shared__ __attribute__((aligned(1024))) half_t sK1[G * TILE];
  __shared__ __attribute__((aligned(1024))) half_t sK2[NBUF > 2 ? G * TILE : 8];
  __shared__ __attribute__((aligned(1024))) half_t sV0[G * TILE];
  __shared__ __attribute__((aligned(1024))) half_t sV1[G * TILE];
  __shared__ __attribute__((aligned(1024))) half_t sV2[NBUF > 2 ? G * TILE : 8];
  // key-bias words of the tile, one copy per wave (so each wave's own vmcnt covers it)
  __shared__ __attribute__((aligned(1024))) float sB0[NW * 64];
  __shared__ __attribute__((aligned(1024))) float sB1[NW * 64];
  __shared__ __attribute__((aligned(1024))) float sB2[NBUF > 2 ? NW * 64 : 4];
  auto bufK = [&](auto st) -> half_t* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sK0; else if constexpr (s == 1) return sK1; else return sK2;
  };
  auto bufV = [&](auto st) -> half_t* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sV0; else if constexpr (s == 1) return sV1; else return sV2;
  };
  auto bufB = [&](auto st) -> float* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sB0; else if constexpr (s == 1) return sB1; else return sB2;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int qw = wv % NQW;  // query wave within the group
  const int grp = wv / NQW; // key group
  const int lr = lane & 15;
  const int lg = lane >> 4;
  // Workgroups are dealt to the 8 XCDs round-robin; XCD i runs head i of
  // every branch, so a head's K and V^T tiles are fetched into one XCD's L2
  // and every query block of that head hits there.
  const int nqb = (T + QWG - 1) / QWG;
  const int h = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int b = slot / nqb;
  const int q0 = (slot - b * nqb) * QWG + qw * 16 * QB;
  const size_t head = (size_t)b * 8 + h;
  const half_t* Qh = Q + head * Tpad * 64;
  const half_t* Kh = K + head * Tpad * 64;
  const half_t* Vh = Vt + head * 64 * Tpad;
  const float* brow = kbias + (size_t)b * Tpad;
  // Key tiles: every tile, or with BRANCH_KEYS only this branch's tiles up
  // to its last valid key (the tiles after it are fully masked), at least
  // one.  The groups below split whichever count this is.
  int ntiles = Tpad / 64;
  if constexpr (BRANCH_KEYS) {
    const int nk = reinterpret_cast<const int*>(kbias + (size_t)(gridDim.x / (8 * nqb)) * Tpad)[b];
    ntiles = max(1, min(ntiles, (nk + 63) / 64));
    // QSKIP (padded batches whose padded rows are left unspecified): query
    // rows from two past the branch's last valid key on are not needed --
    // the two rows after it are, because the WaveNet's k=5 conv at the last
    // valid rows reads them -- so a workgroup holding none of them leaves.
    if constexpr (QSKIP) {
      if ((slot - b * nqb) * QWG >= min(nk + 2, T)) return;
    }
  }
  // Group grp walks tiles [grp*tpg, grp*tpg + tpg).  A tile index past the
  // end loads the last tile again (clamped) and is not computed, so every
  // group runs the same iterations and meets at the same barriers.
  const int tpg = (ntiles + G - 1) / G;
  const int tbase = grp * tpg;

  // Per tile the NQW waves of a group split its K and V^T tiles (8 KB each,
  // 8 / NQW direct loads of 1 KB per wave and tile), and each wave loads its
  // own copy of the 64 bias words.  The loads go through buffer resources
  // over this head's K and V^T and this branch's bias row: a lane's byte
  // offset within a tile is fixed for the whole loop, and the tile's offset
  // is a scalar, so issuing a tile costs no vector instructions.
  constexpr int kPer = 8 / NQW;
  constexpr int kLoads = 2 * kPer + 1;
  const buffer_rsrc_t rK = make_buffer_rsrc(Kh, Tpad * 64 * 2);
  const buffer_rsrc_t rV = make_buffer_rsrc(Vh, Tpad * 64 * 2);
  const buffer_rsrc_t rB = make_buffer_rsrc(brow, Tpad * 4);
  int voK[kPer], voV[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int q = (qw * kPer + u) * 64 + lane;  // this lane's 16-byte slot of the tile
    const int row = q >> 3;
    voK[u] = (row * 64 + attn_kslot(row, q & 7) * 8) * 2;
    voV[u] = (row * Tpad + attn_vslot(row, q & 7) * 8) * 2;
  }
  auto issue = [&](auto st, int j) {
    const int kt = min(tbase + j, ntiles - 1);
    half_t* sk = bufK(st) + grp * TILE;
    half_t* sv = bufV(st) + grp * TILE;
    float* sb = bufB(st) + wv * 64;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int s0 = (qw * kPer + u) * 64;  // first 16-byte slot of this load
      buffer_load_lds16(rK, (lds_ptr_t*)(sk + s0 * 8), voK[u], kt * 8192);
      buffer_load_lds16(rV, (lds_ptr_t*)(sv + s0 * 8), voV[u], kt * 128);
    }
    buffer_load_lds4(rB, (lds_ptr_t*)sb, lane * 4, kt * 256);
  };

  // B operands of S^T = K.Q^T: query rows q0 + 16 qb + lr, d-slots of lane group lg.
  half8 qf[QB][2];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const half_t* qp = Qh + (size_t)(q0 + 16 * qb + lr) * 64 + lg * 8;
    qf[qb][0] = *reinterpret_cast<const half8*>(qp);
    qf[qb][1] = *reinterpret_cast<const half8*>(qp + 32);
  }
  // A operand of the denominator block: row 0 all ones, rows 1..15 zero.
  half8 ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = lr == 0 ? (half_t)1.0f : (half_t)0.0f;

  floatx4 o[4][QB];  // o[db][qb][i] = O[query q0+16qb+lr][d = 16 db + 4 lg + i] (unnormalised)
  floatx4 o5[QB];    // o5[qb][0] in lane group 0: the running denominator of query q0+16qb+lr
  float m_run[QB];   // running max (log2 units), same in a query's 4 lanes
  // The QK^T accumulators start at -m_use (m_use = m_run, or 0 while no key
  // of the query is valid yet), so the matrix cores return the scores
  // already shifted by the running max; thr is how far a shifted score may
  // rise before the max moves (-inf while m_run is -inf: any valid key moves it).
  float negm[QB];
  float thr[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    o5[qb] = floatx4{0.f, 0.f, 0.f, 0.f};
    m_run[qb] = -INFINITY;
    negm[qb] = 0.0f;
    thr[qb] = -INFINITY;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db][qb] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](auto st, int j) {
    const int kt = tbase + j;
    // A tile past the end (its group's share is short) would contribute
    // exp2(-inf) = 0 to every sum and leave the maxima alone: skip it.
    if (kt >= ntiles) return;
    const half_t* sk = bufK(st) + grp * TILE;
    const half_t* sv = bufV(st) + grp * TILE;
    const float* sb = bufB(st) + wv * 64;
    // Whether any key of the tile is masked (one bias word per lane; the
    // same answer in every lane, so the bias pass below is a uniform branch
    // that only tiles holding a masked or padding key take).
    const bool masked = __any(sb[lane] != 0.0f);
    // sc[kb][qb][i] = S[key kt*64 + 32 (kb>>1) + 8 lg + 4 (kb&1) + i][query q0 + 16 qb + lr]
    //                 - m_use[query]   (log2 units: q carries log2(e) / 8)
    floatx4 sc[4][QB];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int row = 32 * (kb >> 1) + 8 * (lr >> 2) + 4 * (kb & 1) + (lr & 3);
      const half8 kf0 = *reinterpret_cast<const half8*>(sk + row * 64 + attn_kslot(row, lg) * 8);
      const half8 kf1 = *reinterpret_cast<const half8*>(sk + row * 64 + attn_kslot(row, 4 + lg) * 8);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const floatx4 z = mfma16x16x32(kf0, qf[qb][0], floatx4{negm[qb], negm[qb], negm[qb], negm[qb]});
        sc[kb][qb] = mfma16x16x32(kf1, qf[qb][1], z);
      }
    }
    if (masked) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const float4 bb = *reinterpret_cast<const float4*>(sb + 32 * (kb >> 1) + 8 * lg + 4 * (kb & 1));
        const float bv[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[kb][qb][i] += bv[i];
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      // NaN-propagating maximum (v_maximum3_f32): no canonicalising pass over
      // the matrix-core results, three inputs per instruction
      float lmax = __builtin_elementwise_maximum(sc[0][qb][0], sc[0][qb][1]);
#pragma unroll
      for (int e = 2; e < 16; e += 2)
        lmax = __builtin_elementwise_maximum(
            __builtin_elementwise_maximum(lmax, sc[e >> 2][qb][e & 3]), sc[e >> 2][qb][(e & 3) + 1]);
      if (__any(lmax > thr[qb])) {
        float tmax = fmaxf(lmax, __shfl_xor(lmax, 16, kWave));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
        const bool need = tmax > thr[qb];
        const float delta = need ? tmax : 0.0f;  // the max's move, in the shifted frame
        // o and l are all zero while m_run is -inf: alpha 0 keeps them so
        // (exp2(-delta) could overflow for a very negative first max)
        const float alpha = m_run[qb] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(-delta);
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db][qb] *= alpha;
        o5[qb] *= alpha;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[kb][qb][i] -= delta;
        if (need) {
          m_run[qb] = (m_run[qb] == -INFINITY ? 0.0f : m_run[qb]) + tmax;
          thr[qb] = kLazyMax;
          negm[qb] = -m_run[qb];
        }
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[kb][qb][i] = __builtin_amdgcn_exp2f(sc[kb][qb][i]);
    }
    // O^T += V^T . P^T over two 32-key chunks; K-slot j of lane group lg is
    // key 32 c + 8 lg + j in both operands.  The ones block sums P.
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      half8 pb[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pb[qb][i] = (half_t)sc[2 * c][qb][i];
          pb[qb][4 + i] = (half_t)sc[2 * c + 1][qb][i];
        }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int row = db * 16 + lr;
        const half8 va = *reinterpret_cast<const half8*>(sv + row * 64 + attn_vslot(row, 4 * c + lg) * 8);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o[db][qb] = mfma16x16x32(va, pb[qb], o[db][qb]);
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) o5[qb] = mfma16x16x32(ones, pb[qb], o5[qb]);
    }
  };

  attn_static_for<0, NBUF - 1>([&](auto st) { issue(st, min((int)decltype(st)::value, tpg - 1)); });
  attn_wait_vmcnt<kLoads * (NBUF - 1)>();  // the Q fragments (issued before the prologue) have landed
  int kt0 = 0;
  for (; kt0 + NBUF <= tpg; kt0 += NBUF) {
    attn_static_for<0, NBUF>([&](auto st) {
      constexpr int s = decltype(st)::value;
      attn_wait_vmcnt<kLoads * (NBUF - 2)>();  // this wave's share of tile kt0+s has landed
      attn_wait_lgkmcnt0();                    // its reads of tile kt0+s-1 have returned
      __builtin_amdgcn_s_barrier();            // ... for every wave
      issue(std::integral_constant<int, (s + NBUF - 1) % NBUF>{}, min(kt0 + s + NBUF - 1, tpg - 1));
      compute(st, kt0 + s);
    });
  }
  attn_wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  attn_static_for<0, NBUF - 1>([&](auto st) {
    if (kt0 + (int)decltype(st)::value < tpg) compute(st, kt0 + decltype(st)::value);
  });

  // Denominator of each query: component 0 of the ones block in lane group 0.
  float l_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) l_run[qb] = __shfl(o5[qb][0], lr, kWave);
  if constexpr (G > 1) {
    // Groups 1.. park (m, l, O) in the tile buffers, free once every wave is
    // past its last tile: group g's O values (NQW*QB*4 KB) in sK0 (g = 1, 2;
    // sK0 holds G x 8 KB) or sK1 (g = 3), its (m, l) pairs in sV0.  Group 0
    // then rescales every part to the common max.
    constexpr int kParkO = NQW * QB * 64 * 16;  // floats of O parked per group
    auto park_o = [&](int g) -> float* {
      float* base = reinterpret_cast<float*>(g <= 2 ? sK0 : sK1);
      return base + ((g - 1) & 1) * kParkO + (qw * 64 + lane) * (16 * QB);
    };
    auto park_ml = [&](int g) -> float* {
      return reinterpret_cast<float*>(sV0) + (((g - 1) * NQW + qw) * 64 + lane) * (2 * QB);
    };
    attn_wait_lgkmcnt0();
    __syncthreads();
    if (grp > 0) {
      float* po = park_o(grp);
      float* pm = park_ml(grp);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
          *reinterpret_cast<floatx4*>(po + qb * 16 + db * 4) = o[db][qb];
        pm[qb * 2] = m_run[qb];
        pm[qb * 2 + 1] = l_run[qb];
      }
    }
    attn_wait_lgkmcnt0();
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mstar = m_run[qb];
#pragma unroll
      for (int g = 1; g < G; ++g) mstar = fmaxf(mstar, park_ml(g)[qb * 2]);
      const float mref = mstar == -INFINITY ? 0.0f : mstar;
      const float w0 = __builtin_amdgcn_exp2f(m_run[qb] - mref);
      l_run[qb] *= w0;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db][qb] *= w0;
#pragma unroll
      for (int g = 1; g < G; ++g) {
        const float* po = park_o(g) + qb * 16;
        const float* pm = park_ml(g) + qb * 2;
        const float wg = __builtin_amdgcn_exp2f(pm[0] - mref);
        l_run[qb] += wg * pm[1];
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db][qb] += wg * *reinterpret_cast<const floatx4*>(po + db * 4);
      }
    }
  }
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int q = q0 + 16 * qb + lr;
    if (q < T) {
      const float inv = l_run[qb] > 0.0f ? 1.0f / l_run[qb] : 0.0f;
      half_t* dst = O + ((size_t)b * T + q) * 512 + h * 64 + lg * 4;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        half4 v;
        v[0] = (half_t)(o[db][qb][0] * inv);
        v[1] = (half_t)(o[db][qb][1] * inv);
        v[2] = (half_t)(o[db][qb][2] * inv);
        v[3] = (half_t)(o[db][qb][3] * inv);
        *reinterpret_cast<half4*>(dst + db * 16) = v;
      }
    }
  }
}

// kbias[b][t] = 0 for a valid key (t < T, mask != 0), -inf otherwise, for
// t < Tpad: the additive key mask of attention_kernel (log2 units).
// One block per branch b: its Tpad bias words, and after all B rows of them
// the branch's key count (one past its last valid key; 0 if none).
__global__ __launch_bounds__(256) void key_bias_kernel(const uint32_t* __restrict__ mask, int T, int Tpad,
                                                       float* __restrict__ kbias, int* __restrict__ nkeys) {
  const int b = blockIdx.x;
  int last = 0;
  for (int t = threadIdx.x; t < Tpad; t += 256) {
    const bool valid = t < T && mask[(size_t)b * T + t] != 0u;
    kbias[(size_t)b * Tpad + t] = valid ? 0.0f : -INFINITY;
    if (valid) last = t + 1;
  }
  __shared__ int wmax[4];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) last = max(last, __shfl_xor(last, off, kWave));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = last;
  __syncthreads();
  if (threadIdx.x == 0) nkeys[b] = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
}

hipError_t launch_key_bias(const uint32_t* mask, int B, int T, int Tpad, float* kbias,
                           hipStream_t stream) {
  if (B <= 0 || T <= 0 || Tpad < T || Tpad % 64 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(key_bias_kernel, dim3(B), dim3(256), 0, stream, mask, T, Tpad, kbias,
                     reinterpret_cast<int*>(kbias + (size_t)B * Tpad));
  return hipGetLastError();
}

template <int NBUF, int G, int QB, int NQW>
static void launch_attention_shape(const half_t* Q, const half_t* K, const half_t* Vt,
                                   const float* kbias, half_t* O, int B, int T, int Tpad,
                                   hipStream_t stream, bool branch_keys, bool qskip) {
  constexpr int qwg = 16 * QB * NQW;
  const dim3 grid((T + qwg - 1) / qwg * 8 * B), block(64 * G * NQW);
  if (qskip)
    hipLaunchKernelGGL((attention_kernel<NBUF, G, QB, NQW, true, true>), grid, block, 0, stream, Q, K,
                       Vt, kbias, O, T, Tpad);
  else if (branch_keys)
    hipLaunchKernelGGL((attention_kernel<NBUF, G, QB, NQW, true, false>), grid, block, 0, stream, Q, K,
                       Vt, kbias, O, T, Tpad);
  else
    hipLaunchKernelGGL((attention_kernel<NBUF, G, QB, NQW, false, false>), grid, block, 0, stream, Q,
                       K, Vt, kbias, O, T, Tpad);
}

hipError_t launch_attention(const half_t* Q, const half_t* K, const half_t* Vt,
                            const float* kbias, half_t* O, int B, int T, int Tpad,
                            hipStream_t stream, bool branch_keys, bool qskip) {
  if (B <= 0 || T <= 0 || Tpad < T || Tpad % 64 != 0) return hipErrorInvalidValue;
  // Shapes swept on MI355X (B = 2, us per launch, head-per-XCD mapping):
  //   T = 128 / 300:  32 queries x 2 key groups, 16-query waves, 2 buffers   3.5 / 4.9
  //   T = 860:        64 queries x 2 key groups, 16-query waves, 2 buffers   8.5 (3 buffers: 8.6)
  //   T = 1348:       64 queries x 2 key groups, 16-query waves, 2 buffers  17.5 (3 buffers: 21.4)
  //   T = 3000:       64 queries x 2 key groups, 16-query waves, 2 buffers  52-54
  // 32-query waves (two 16-query blocks per wave) are slower at every length
  // (T = 860 / 1348 / 3000: 10.4 / 20.9 / 59-68).  Every shape splits the
  // keys into the same two groups, so the result is bit-identical whichever
  // is chosen; the choice depends on the padded length only, never on the
  // batch.
  if (Tpad <= 512)
    launch_attention_shape<2, 2, 1, 2>(Q, K, Vt, kbias, O, B, T, Tpad, stream, branch_keys, qskip);
  else
    launch_attention_shape<2, 2, 1, 4>(Q, K, Vt, kbias, O, B, T, Tpad, stream, branch_keys, qskip);
  return hipGetLastError();
}

}  // namespace mit2hip
