// gemm.hip -- f16 MFMA GEMM (gfx950) with the decoder's fused epilogues.
//
// Replaces the reference's MPS GEMM dispatch (runtime/metal_context.mm:328-378)
// and the kernels fused around it (bias pre-fill kernels.metal:227, residual
// add :161, SwiGLU :131, WaveNet gate :411, res/skip update :436, RoPE :2390,
// reflect-pad + im2col :175-225 for the k=5 conv).
//
// Pipeline.  A 256-thread workgroup (4 wavefronts, 2x2) owns a BM x BN tile.
// K is consumed in stages of SK halves; NST stages live in a ring of LDS
// buffers, each its own __shared__ object.  Operands move global -> LDS with
// gfx950's direct loads (global_load_lds_dwordx4: each lane's 16 bytes land
// at M0 + 16*lane), so NST-1 stages (tens of KB per CU) are in flight while
// the current one feeds the MFMAs, with no register staging.  Because every
// stage buffer is a distinct LDS object the compiler can tell the in-flight
// DMA from the buffer being read and keeps only the explicit vmcnt waits.
//
// LDS layout.  A stage row is SK halves = CPR 16-byte slots; the slot holding
// global chunk c of row r is c ^ key(r) (key = r & 15, or (r >> 1) & 7 for
// 8-slot rows), so the 16 lanes of a ds_read_b128 that read 16 consecutive
// rows at one chunk hit 64 distinct banks.
//
// Tile -> workgroup map.  Workgroups are dealt to the 8 XCDs round-robin; the
// map gives each XCD a rectangle of tiles (Xm x Xn split of the tile grid,
// chosen on the host to minimise A and W re-reads across XCDs) so that the
// operands a rectangle shares stay in that XCD's L2.
#include <algorithm>
#include <type_traits>

#include "gemm.h"

namespace mit2hip {

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt lgkmcnt(0): this wave's LDS reads have returned.
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (0 << 8));
}

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Issue order for one K step of the pipelined loop: each of ND fragment
// reads beside one MFMA (the next K step needs them first), then each of NV
// stage loads beside one, then the remaining MFMAs; reads or loads left over
// when the NM MFMAs run out follow in the same order.
template <int ND, int NV, int NM>
__device__ __forceinline__ void interleave() {
  static_for<0, (ND + NV > NM ? ND + NV : NM)>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if constexpr (i < ND) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);            // DS read
    else if constexpr (i < ND + NV) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // VMEM
    if constexpr (i < NM) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);            // MFMA
  });
}

struct TileMap {
  int nM, nN;  // tile grid (nM: the row tiles that are computed)
  int Xm, Xn;  // XCD rectangle grid, Xm * Xn == 8
  int per_xcd; // workgroups per XCD (grid = 8 * per_xcd)
  // Row-tile skipping: the computed row tiles are nseg runs; run s starts at
  // row tile seg_first[s] and holds computed tiles [seg_cum[s], seg_cum[s+1]).
  int nseg;
  int seg_first[kMaxRowSeq];
  int seg_cum[kMaxRowSeq];
  __device__ __forceinline__ bool map(int b, int& tm, int& tn) const {
    const int xcd = b & 7, slot = b >> 3;
    const int rx = xcd / Xn, ry = xcd - (xcd / Xn) * Xn;
    const int mlo = rx * nM / Xm, mhi = (rx + 1) * nM / Xm;
    const int nlo = ry * nN / Xn, nhi = (ry + 1) * nN / Xn;
    const int rn = nhi - nlo;
    if (rn <= 0 || slot >= (mhi - mlo) * rn) return false;
    tm = mlo + slot / rn;
    tn = nlo + slot % rn;
    if (nseg > 0) {
      // static indices only (the map stays in kernel-argument registers)
      int first = seg_first[0], cum = 0;
#pragma unroll
      for (int s = 1; s < kMaxRowSeq; ++s) {
        if (s < nseg && tm >= seg_cum[s]) {
          first = seg_first[s];
          cum = seg_cum[s];
        }
      }
      tm = first + (tm - cum);
    }
    return true;
  }
};

// Rotary rotation of the pair (x, y) by (cos, sin) = cs.  Each output is one
// fused multiply-add over one rounded product, written out so that every
// tile shape's instantiation rounds alike (left to the contraction pass, the
// choice of which product to fuse varied between instantiations).
__device__ inline float2 rope_rotate(float x, float y, float2 cs) {
  return make_float2(__builtin_fmaf(x, cs.x, -(y * cs.y)), __builtin_fmaf(y, cs.x, x * cs.y));
}

// f16 of v as computed in fp32.  The empty asm statement keeps v a register
// value, so the conversion is never merged with v's producing multiply or
// fused multiply-add into one mixed-precision instruction (v_fma_mix, which
// rounds once, straight to f16).  The compiler made that choice differently
// in different kernels, so a row's q and V bits depended on the kernel that
// computed them; with this every QKV kernel rounds twice, alike.  (Not
// volatile: a volatile statement also pinned the epilogue's RoPE loads in
// place, one dependent load at a time.)
__device__ inline half_t f16_of(float v) {
  __asm__("" : "+v"(v));
  return (half_t)v;
}

template <int BM, int BN, int SK, int NST, int AM, int EPI, int WM, int WN, int KG, int SP, int PIPE>
__global__ __launch_bounds__(64 * WM * WN * (PIPE ? 1 : KG)) void gemm_kernel(GemmArgs p, TileMap tmap) {
  // K split.  The product over K is summed in KG parts of equal length, added
  // in part order at the end (the same bits whichever form computes them).
  // PIPE = 0: part g is walked by its own group of WM x WN wavefronts with
  // its own LDS region.  PIPE = 1: one group of wavefronts walks all of K,
  // holding one accumulator set per part, with the pipelined main loop
  // below.
  constexpr int KW = PIPE ? 1 : KG;          // wavefront groups
  constexpr int NW = WM * WN;                // wavefronts per group, WM along M x WN along N
  constexpr int CPR = SK / 8;                // 16-byte slots per stage row
  constexpr int LA = BM * CPR / (64 * NW);   // DMA instructions per wave per stage (A)
  constexpr int LB = BN * CPR / (64 * NW);   // (W)
  constexpr int AS = SP >= 1 ? 2 : 1;        // copies of each A stage (split: hi, lo)
  constexpr int WS = SP == 2 ? 2 : 1;        // copies of each W stage
  constexpr bool kWin = AM == A_CONVW;       // A from the LDS window: only W is streamed
  constexpr int L = (kWin ? 0 : LA * AS) + LB * WS;  // DMA instructions per wave per stage
  constexpr int WTM = BM / WM;               // rows of a wave's sub-tile
  constexpr int WTN = BN / WN;               // columns of a wave's sub-tile
  constexpr int MI = WTM / 16;               // 16-row MFMA blocks per wave
  constexpr int NI = WTN / 16;               // 16-col MFMA blocks per wave
  static_assert(LA >= 1 && LB >= 1, "tile too small for the workgroup");
  static_assert(LA * 64 * NW == BM * CPR && LB * 64 * NW == BN * CPR, "uneven DMA split");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave sub-tile must be whole MFMA blocks");
  static_assert(L * (NST - 1 + PIPE) < 64, "too many loads in flight");
  static_assert(CPR == 8 || CPR >= 16, "stage width");
  static_assert(KG == 1 || ((KG == 2 || KG == 4) && EPI != EPI_QKV),
                "K groups: 2 or 4, and the QKV epilogue needs every wave");
  static_assert(!PIPE || ((KG == 1 || KG == 2) && (SP == 0 || KG == 1)),
                "pipelined loop: K in 1 or 2 parts; split operands with one part");
  static_assert(EPI != EPI_QKV || 512 % BN == 0, "a qkv tile must lie inside one of the q, k, v sections");
  static_assert(SP >= 0 && SP <= 2, "split mode");
  static_assert(!kWin || (!PIPE && KG == 1), "window convs: the one-group stage loop");

  // One __shared__ object per stage and operand, declared here so each kernel
  // instantiation owns its own objects (the per-object alias scopes are what
  // let the compiler keep only the explicit vmcnt waits).
  // With KG = 2 K groups, each group has its own region in every buffer;
  // split operands keep their lo halves after all the groups' hi halves.
  constexpr int kAStage = kWin ? 8 : AS * KW * BM * SK;  // halves of an A ring buffer
  constexpr int kBStage = WS * KW * BN * SK;
  constexpr int kA2 = NST > 2 ? kAStage : 8, kA3 = NST > 3 ? kAStage : 8, kA4 = NST > 4 ? kAStage : 8,
                kA5 = NST > 5 ? kAStage : 8, kA6 = NST > 6 ? kAStage : 8, kA7 = NST > 7 ? kAStage : 8;
  constexpr int kB2 = NST > 2 ? kBStage : 8, kB3 = NST > 3 ? kBStage : 8, kB4 = NST > 4 ? kBStage : 8,
                kB5 = NST > 5 ? kBStage : 8, kB6 = NST > 6 ? kBStage : 8, kB7 = NST > 7 ? kBStage : 8;
  // Unused buffers are 8 halves; with the window they are 16-byte aligned
  // (a 1024-byte slot each would not leave the window room).
  constexpr int kPad = kWin ? 16 : 1024;
#define MIT2_LDS_ALIGN(n) alignas((n) > 8 ? 1024 : kPad)
  __shared__ MIT2_LDS_ALIGN(kAStage) half_t sA0[kAStage];
  __shared__ MIT2_LDS_ALIGN(kAStage) half_t sA1[kAStage];
  __shared__ MIT2_LDS_ALIGN(kA2) half_t sA2[kA2];
  __shared__ MIT2_LDS_ALIGN(kA3) half_t sA3[kA3];
  __shared__ MIT2_LDS_ALIGN(kA4) half_t sA4[kA4];
  __shared__ MIT2_LDS_ALIGN(kA5) half_t sA5[kA5];
  __shared__ MIT2_LDS_ALIGN(kA6) half_t sA6[kA6];
  __shared__ MIT2_LDS_ALIGN(kA7) half_t sA7[kA7];
  // A_CONVW: the row block's input window (hi rows, then lo rows)
  constexpr int kWinH = kWin ? conv_window_halves(BM, BN, AS) : 8;
  __shared__ MIT2_LDS_ALIGN(kWinH) half_t sWin[kWinH];
  static_assert(!kWin || kWinH / (8 * 64 * NW) + L * (NST - 1) < 64, "too many loads in flight");
  __shared__ MIT2_LDS_ALIGN(kBStage) half_t sB0[kBStage];
  __shared__ MIT2_LDS_ALIGN(kBStage) half_t sB1[kBStage];
  __shared__ MIT2_LDS_ALIGN(kB2) half_t sB2[kB2];
  __shared__ MIT2_LDS_ALIGN(kB3) half_t sB3[kB3];
  __shared__ MIT2_LDS_ALIGN(kB4) half_t sB4[kB4];
  __shared__ MIT2_LDS_ALIGN(kB5) half_t sB5[kB5];
  __shared__ MIT2_LDS_ALIGN(kB6) half_t sB6[kB6];
  __shared__ MIT2_LDS_ALIGN(kB7) half_t sB7[kB7];
#undef MIT2_LDS_ALIGN
  constexpr int kALo = KW * BM * SK;  // offset of a stage's lo half in its buffer
  constexpr int kWLo = KW * BN * SK;
  static_assert(NST >= 2 && NST <= 8, "two to eight stages");
  const int kg = __builtin_amdgcn_readfirstlane(threadIdx.x / (64 * NW));  // K group of this wave
  auto bufA = [&](auto st) -> half_t* {
    constexpr int s = decltype(st)::value;
    half_t* b;
    if constexpr (s == 0) b = sA0; else if constexpr (s == 1) b = sA1;
    else if constexpr (s == 2) b = sA2; else if constexpr (s == 3) b = sA3;
    else if constexpr (s == 4) b = sA4; else if constexpr (s == 5) b = sA5;
    else if constexpr (s == 6) b = sA6; else b = sA7;
    return KW == 1 ? b : b + kg * BM * SK;
  };
  auto bufB = [&](auto st) -> half_t* {
    constexpr int s = decltype(st)::value;
    half_t* b;
    if constexpr (s == 0) b = sB0; else if constexpr (s == 1) b = sB1;
    else if constexpr (s == 2) b = sB2; else if constexpr (s == 3) b = sB3;
    else if constexpr (s == 4) b = sB4; else if constexpr (s == 5) b = sB5;
    else if constexpr (s == 6) b = sB6; else b = sB7;
    return KW == 1 ? b : b + kg * BN * SK;
  };

  int tile_m, tile_n;
  if (!tmap.map(blockIdx.x, tile_m, tile_n)) return;
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6) % NW;  // wave within its K group
  const int wm = wave / WN;
  const int wn = wave - wm * WN;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  // K group kg walks stages [kg * KT, kg * KT + KT) (the host makes K / SK a
  // multiple of KG, so both groups meet the same barriers).
  const int KT = p.K / SK / KW;
  const int kt_lo = kg * KT;

  // Output ownership.  The MFMA is issued with W as its first operand, so the
  // accumulator is C^T: lane (lr, lg) of block (i, j) holds the four
  // consecutive columns n = col_base + 16 j + 4 lg + r (r = 0..3) of row
  // m = row_base + 16 i + lr.  Every epilogue access is then a 16-byte
  // (fp32) or 8-byte (f16) vector per lane.
  const int row_base = m0 + wm * WTM + lr;
  const int col_base = n0 + wn * WTN + 4 * lg;
  // First of the four output columns this lane holds in block j: col_base +
  // 16 j, or with column-pair rows (GemmArgs::colperm) 8 consecutive columns
  // per block pair (2 q, 2 q + 1) starting at n0 + wn*WTN + 32 q + 8 lg.
  const bool perm = EPI == EPI_F32 && p.colperm;
  auto colj = [&](int j) { return perm ? col_base + 32 * (j >> 1) + 4 * lg + 4 * (j & 1) : col_base + 16 * j; };

  // Epilogue operands that do not depend on the product are fetched before
  // the K loop, so their latency hides behind it (PIPE = 1: after the loop,
  // so they do not hold registers beside its larger tiles).
  constexpr bool kPreA =
      EPI == EPI_F32 || EPI == EPI_RESSKIP || EPI == EPI_FINALSKIP || EPI == EPI_RESAVG;
  constexpr bool kPreB = EPI == EPI_FINALSKIP;
  // The WaveNet epilogues' row mask (one word per row) and the gate's
  // global conditioning (one float4 pair per column group) as well: fetched
  // in the epilogue, each load's wait also drained the stores before it.
  // The WaveNet epilogues' loads are unconditional (rows past M read row
  // M - 1, which no epilogue uses; the skip accumulator is read even when it
  // starts at zero, and the epilogue drops it): a load under a per-lane
  // branch made the compiler wait for it where the branches join, ahead of
  // the first K stages.
  constexpr bool kPreMask = EPI == EPI_RESSKIP || EPI == EPI_FINALSKIP;
  constexpr bool kPreCond = EPI == EPI_GATE;
  constexpr bool kPre = kPreA || kPreCond;
  float4 pre_a[kPreA ? MI : 1][kPreA ? NI : 1];
  float4 pre_b[kPreB ? MI : 1][kPreB ? NI : 1];
  uint32_t pre_mask[kPreMask ? MI : 1];
  float4 pre_ca[kPreCond ? NI / 2 : 1], pre_cb[kPreCond ? NI / 2 : 1];
  auto load_pre = [&]() {
    if constexpr (kPreMask) {
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int mc = min(row_base + 16 * i, p.M - 1);
        pre_mask[i] = p.mask[mc];
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int n = colj(j);
          if constexpr (EPI == EPI_RESSKIP) {
            // a tile lies wholly below or above column 512 (BN divides 512)
            const float* src = n < 512 ? p.C32 + (size_t)mc * p.ldc32 + n
                                       : p.C32b + (size_t)mc * p.ldc32b + (n - 512);
            pre_a[i][j] = *reinterpret_cast<const float4*>(src);
          } else {
            pre_a[i][j] = *reinterpret_cast<const float4*>(p.C32b + (size_t)mc * p.ldc32b + n);
            pre_b[i][j] = *reinterpret_cast<const float4*>(p.rp + (size_t)mc * 512 + n);
          }
        }
      }
      return;
    }
    if constexpr (kPreCond) {
      // channel block of the pair (2 q, 2 q + 1): c = 16 group + 4 lg, as in the epilogue
#pragma unroll
      for (int q = 0; q < NI / 2; ++q) {
        const int c = ((col_base + q * 32 - 4 * lg) >> 5) * 16 + 4 * lg;
        pre_ca[q] = *reinterpret_cast<const float4*>(p.cond + c);
        pre_cb[q] = *reinterpret_cast<const float4*>(p.cond + 512 + c);
      }
    }
    if constexpr (!kPreA) return;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = row_base + 16 * i;
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int n = colj(j);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m < p.M && kg == 0 && (p.n_store == 0 || n < p.n_store)) {
          if constexpr (EPI == EPI_F32 || EPI == EPI_RESAVG) {
            if (p.res) v = *reinterpret_cast<const float4*>(p.res + (size_t)m * p.ldres + n);
          }
        }
        pre_a[i][j] = v;
      }
    }
  };
  if constexpr (kPre && !PIPE) load_pre();

  // Consumer side of a folded AdaRMSNorm: the producer's kSsqParts partial
  // sums of squares of each of this lane's rows (K = 512 values) are fetched
  // ahead of the first K stages and reduced to rs once those are in flight.
  constexpr bool kNormIn = EPI == EPI_SWIGLU || EPI == EPI_QKV;
  float4 ssq_pre[kNormIn ? MI : 1][kSsqParts / 4];
  if constexpr (kNormIn) {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = row_base + 16 * i;
#pragma unroll
      for (int u = 0; u < kSsqParts / 4; ++u)
        ssq_pre[i][u] = (p.ssq_in && m < p.M && kg == 0)
                            ? reinterpret_cast<const float4*>(p.ssq_in + (size_t)m * kSsqParts)[u]
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  auto swz = [](int row) { return CPR >= 16 ? (row & 15) : ((row >> 1) & 7); };

  // A_CONV5: a K stage never straddles a tap (kConvC % SK == 0), so each of
  // this lane's load slots needs one of five source rows, fixed for the
  // kernel: they are computed once here (five named offsets per slot, never
  // an indexed table) and picked per stage with the wave-uniform tap.
  struct ConvRows {
    int r0, r1, r2, r3, r4;  // element offset of row reflect(t + tap - 2), tap 0..4
  };
  constexpr bool kConv = AM == A_CONV5 || AM == A_CONV3Z;
  ConvRows conv_rows[kConv ? LA : 1];
  if constexpr (AM == A_CONV3Z) {
    // k = 3 with zero padding: taps t-1, t, t+1; a tap outside the sequence
    // reads row M, which the caller keeps all zero.
    static_assert(kConvC % SK == 0, "a K stage must lie within one conv tap");
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int row = ((wave * LA + j) * 64 + lane) / CPR;
      const int m = min(m0 + row, p.M - 1);
      const int b = m / p.T;
      const int t = m - b * p.T;
      const int base = b * p.T;
      conv_rows[j].r0 = (t > 0 ? base + t - 1 : p.M) * p.lda;
      conv_rows[j].r1 = (base + t) * p.lda;
      conv_rows[j].r2 = (t + 1 < p.T ? base + t + 1 : p.M) * p.lda;
      conv_rows[j].r3 = conv_rows[j].r4 = 0;
    }
  }
  if constexpr (AM == A_CONV5) {
    static_assert(kConvC % SK == 0, "a K stage must lie within one conv tap");
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int row = ((wave * LA + j) * 64 + lane) / CPR;
      const int m = min(m0 + row, p.M - 1);
      const int b = m / p.T;
      const int t = m - b * p.T;
      const int base = b * p.T;
      conv_rows[j].r0 = (base + reflect_index(t - 2, p.T)) * p.lda;
      conv_rows[j].r1 = (base + reflect_index(t - 1, p.T)) * p.lda;
      conv_rows[j].r2 = (base + t) * p.lda;
      conv_rows[j].r3 = (base + reflect_index(t + 1, p.T)) * p.lda;
      conv_rows[j].r4 = (base + reflect_index(t + 2, p.T)) * p.lda;
    }
  }

  // A_CONVP: the token (and sequence start) of each load slot's row, fixed
  // for the kernel; the tap and channel of a 16-byte chunk follow from its K
  // position, so one loader covers every kernel size, dilation and width.
  int cp_t[AM == A_CONVP ? LA : 1], cp_base[AM == A_CONVP ? LA : 1];
  if constexpr (AM == A_CONVP) {
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int row = ((wave * LA + j) * 64 + lane) / CPR;
      const int m = min(m0 + row, p.M - 1);
      const int b = m / p.T;
      cp_base[j] = b * p.T;
      cp_t[j] = m - b * p.T;
    }
  }

  // A_CONVP: source of the 16-byte chunk at K position k0 + kc of load slot
  // j's row m; `lo` selects the lo half of a split operand (the resident
  // zero row serves both halves).
  // Branch-free (the corrections and the zero-row choice are selects: as
  // if / else on per-lane values they made divergent branches around every
  // load), with one 32-bit element offset (the host keeps M x lda below
  // 2^31) added to the chosen base.  The row offset is formed for every
  // lane (in wrapping arithmetic: a padding tap's row may lie outside the
  // tensor, and its offset is then replaced) and pinned by an empty asm
  // statement, so the compiler cannot move it back under a branch.  Both
  // halves of a split operand share it.
  struct ConvpSrc {
    const half_t* hi;
    const half_t* lo;
  };
  auto convp_src = [&](int j, int k0, int kc) -> ConvpSrc {
    const int k = k0 + kc;
    // tap = k / conv_c through a float reciprocal, corrected by one either way
    int tap = (int)((float)k * p.conv_inv_c);
    int c = k - tap * p.conv_c;
    const bool under = c < 0;
    tap = under ? tap - 1 : tap;
    c = under ? c + p.conv_c : c;
    const bool over = c >= p.conv_c;
    tap = over ? tap + 1 : tap;
    c = over ? c - p.conv_c : c;
    const int src = cp_t[j] + tap * p.conv_d - p.conv_pad;
    const bool ok = tap < p.conv_k && src >= 0 && src < p.T;
    uint32_t row_off = (uint32_t)(cp_base[j] + src) * (uint32_t)p.lda + (uint32_t)c;
    __asm__("" : "+v"(row_off));
    const int off = ok ? (int)row_off : c;
    return {(ok ? p.A : p.A_zero) + off, (ok ? p.A + p.a_lo : p.A_zero) + off};
  };

  // A_CONVW (one sequence, M = T): the block's output rows m0 .. m0+BM-1 read
  // the input rows m0 - conv_pad + w, w < BM + (conv_k-1) conv_d, whatever
  // their tap; those rows (zero outside [0, T)) are loaded into LDS once per
  // tile, win_cw halves per row (the last chunks zero), the lo halves of a
  // split pair after all the hi rows.  Only W then runs through the ring.
  // The fill is issued ahead of the ring's first stages, so the loop's first
  // wait (every load older than the stages left in flight) covers it.
  int win_cw = 8, win_lo = 0, win_row = 0, win_rc = 0;
  if constexpr (kWin) {
    win_cw = conv_window_chunks(p.conv_c) * 8;
    win_rc = (BM + (p.conv_k - 1) * p.conv_d) * (win_cw >> 3);  // chunks per half
    win_lo = win_rc * 8;
    win_row = (wm * WTM + lr) * win_cw;
  }
  auto fill_window = [&]() {
    constexpr int NT = 64 * NW;
    const int cc = p.conv_c >> 3, ccp = win_cw >> 3;
    const int total = AS * win_rc;
    const float inv = 1.0f / (float)ccp;
    const int row0 = m0 - p.conv_pad;
    // chunk s of the window, s < total rounded up to NT (the host keeps that
    // inside sWin; the chunks past total read zeros)
    for (int q0 = 0; q0 < total; q0 += NT) {
      const int sq = q0 + wave * 64 + lane;
      const int h = sq >= win_rc ? 1 : 0;
      const int sl = h ? sq - win_rc : sq;
      int w = (int)((float)sl * inv);  // row and chunk through a float reciprocal, corrected
      int c = sl - w * ccp;
      const bool under = c < 0;
      w = under ? w - 1 : w;
      c = under ? c + ccp : c;
      const bool over = c >= ccp;
      w = over ? w + 1 : w;
      c = over ? c - ccp : c;
      const int src = row0 + w;
      const bool ok = sq < total && c < cc && src >= 0 && src < p.T;
      uint32_t off = (uint32_t)src * (uint32_t)p.lda + (uint32_t)(c * 8);
      __asm__("" : "+v"(off));
      const half_t* g = ok ? p.A + (h ? p.a_lo : (size_t)0) + off : p.A_zero;
      __builtin_amdgcn_global_load_lds((const void*)g, (lds_ptr_t*)(sWin + (q0 + wave * 64) * 8), 16, 0, 0);
    }
  };
  // Window offset of the 8 K positions kb + 8 lg .. (one tap) of this lane:
  // the tap's row shift plus the channel, or the zero chunk for the padded
  // K positions.  The wave-uniform part (tap and channel of kb, by a scalar
  // multiply-high) is scalar work; a lane's 8 lg < 32 <= 2 conv_c moves it
  // at most one tap on.
  const int lg8 = lg * 8;
  auto win_off = [&](int kb) -> int {
    const int dcw = p.conv_d * win_cw;
    const int tb = (int)__umulhi((uint32_t)kb, p.conv_magic);
    const int cb = kb - tb * p.conv_c;
    const int off_a = tb * dcw + cb;             // K positions still in tap tb
    const int off_b = off_a + dcw - p.conv_c;    // ... moved on to tap tb + 1
    const bool ok_a = tb < p.conv_k, ok_b = tb + 1 < p.conv_k;
    const bool wrap = cb + lg8 >= p.conv_c;
    const int off = (wrap ? off_b : off_a) + lg8;
    return (wrap ? ok_b : ok_a) ? off : p.conv_c;
  };

  // Every other operand is read through a buffer resource: a lane's byte
  // offset (its row and swizzled 16-byte chunk) is fixed for the kernel and
  // the stage's column offset is a scalar, so issuing a stage costs no
  // vector instructions beyond the conv taps' row selects.  The host keeps
  // every span below 2^31 bytes (gemm_spans_fit).
  const int a_rows = AM == A_CONV3Z ? p.M + 1 : p.M;  // A_CONV3Z: row M is the zero row
  const buffer_rsrc_t rW = make_buffer_rsrc(p.W, (int)(((size_t)(p.N - 1) * p.ldw + p.K + p.w_lo) * 2));
  const buffer_rsrc_t rA =
      make_buffer_rsrc(p.A, AM == A_CONVP || AM == A_CONVW ? 0 : (int)(((size_t)a_rows * p.lda + p.a_lo) * 2));
  const buffer_rsrc_t rA2 =
      AM == A_CONCAT ? make_buffer_rsrc(p.A2, (int)(((size_t)p.M * p.lda2 + p.a_lo) * 2)) : rA;
  int voA[LA], voA2[AM == A_CONCAT ? LA : 1], voW[LB];
#pragma unroll
  for (int j = 0; j < LA; ++j) {
    const int q = (wave * LA + j) * 64 + lane;
    const int row = q / CPR;
    const int c = (q % CPR) ^ swz(row);
    const int m = min(m0 + row, p.M - 1);  // rows past M load a valid row; never stored
    if constexpr (kConv) {
      voA[j] = c * 16;  // + the tap's row, chosen per stage
    } else {
      voA[j] = (m * p.lda + c * 8) * 2;
      if constexpr (AM == A_CONCAT) voA2[j] = (m * p.lda2 + c * 8) * 2;
    }
  }
#pragma unroll
  for (int j = 0; j < LB; ++j) {
    const int q = (wave * LB + j) * 64 + lane;
    const int row = q / CPR;
    voW[j] = ((n0 + row) * p.ldw + ((q % CPR) ^ swz(row)) * 8) * 2;
  }

  // Stage kt >= KT (the ring running past the last stage) keeps the per-stage
  // load count, which the vmcnt waits rely on: it loads the last stage again
  // (an L2 hit) into a buffer that is not read again.  The clamp is a scalar
  // select, so the loop body stays branch-free.
  auto issue = [&](auto st, int kt) {
    half_t* sa = bufA(st);
    half_t* sb = bufB(st);
    const int k0 = ((kt < KT ? kt : KT - 1) + kt_lo) * SK;  // wave-uniform
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int q0 = (wave * LA + j) * 64;
      lds_ptr_t* dst = (lds_ptr_t*)(sa + q0 * 8);
      lds_ptr_t* dst_lo = (lds_ptr_t*)(sa + kALo + q0 * 8);
      if constexpr (kWin) {
        (void)dst;
        (void)dst_lo;
      } else if constexpr (AM == A_CONVP) {
        const int q = q0 + lane;
        const int c = (q % CPR) ^ swz(q / CPR);
        const ConvpSrc src = convp_src(j, k0, c * 8);
        __builtin_amdgcn_global_load_lds((const void*)src.hi, dst, 16, 0, 0);
        if constexpr (AS == 2) __builtin_amdgcn_global_load_lds((const void*)src.lo, dst_lo, 16, 0, 0);
      } else if constexpr (kConv) {
        // The tap's row offset by value selects on the wave-uniform tap: a
        // select of the members' addresses would put conv_rows in scratch
        // memory, and its loads would wait for the ring's DMA (one counter).
        const int tap = k0 / kConvC;  // a stage never straddles a tap
        const ConvRows cr = conv_rows[j];
        int ro = cr.r0;
        ro = tap == 1 ? cr.r1 : ro;
        ro = tap == 2 ? cr.r2 : ro;
        if constexpr (AM == A_CONV5) {
          ro = tap == 3 ? cr.r3 : ro;
          ro = tap == 4 ? cr.r4 : ro;
        }
        const int vo = ro * 2 + voA[j];
        const int so = (k0 - tap * kConvC) * 2;
        buffer_load_lds16(rA, dst, vo, so);
        if constexpr (AS == 2) buffer_load_lds16(rA, dst_lo, vo, so + (int)p.a_lo * 2);
      } else if constexpr (AM == A_CONCAT) {
        const bool first = k0 < p.K1;  // a stage never straddles K1
        const buffer_rsrc_t r = first ? rA : rA2;
        const int vo = first ? voA[j] : voA2[j];
        const int so = (first ? k0 : k0 - p.K1) * 2;
        buffer_load_lds16(r, dst, vo, so);
        if constexpr (AS == 2) buffer_load_lds16(r, dst_lo, vo, so + (int)p.a_lo * 2);
      } else {
        buffer_load_lds16(rA, dst, voA[j], k0 * 2);
        if constexpr (AS == 2) buffer_load_lds16(rA, dst_lo, voA[j], k0 * 2 + (int)p.a_lo * 2);
      }
    }
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const int q0 = (wave * LB + j) * 64;
      buffer_load_lds16(rW, (lds_ptr_t*)(sb + q0 * 8), voW[j], k0 * 2);
      if constexpr (WS == 2)
        buffer_load_lds16(rW, (lds_ptr_t*)(sb + kWLo + q0 * 8), voW[j], k0 * 2 + (int)p.w_lo * 2);
    }
  };

  floatx4 acc[MI][NI];
  floatx4 accx[SP ? MI : 1][SP ? NI : 1];  // split: the cross terms, scaled by kSplitScale
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (SP > 0) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) accx[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // Fragment reads.  Every fragment row of this lane has the same swizzle
  // (rows differ by multiples of 16), so a read's address is the stage
  // buffer plus one per-(operand, kk) lane offset plus a constant.  The lane
  // offsets (K group region included) are opaque to the optimizer: it would
  // otherwise split each sum into a chain of one-term address steps, and the
  // LDS lowering gives a load its buffer's alias scope only within a few
  // steps of the buffer.  A read without a scope may alias every ring buffer,
  // so the compiler would wait for all DMA in flight before it.
  int a_lane[SK / 32], b_lane[SK / 32];
#pragma unroll
  for (int kk = 0; kk < SK / 32; ++kk) {
    const int sw = ((kk * 4 + lg) ^ swz(lr)) << 3;
    a_lane[kk] = (KW == 1 ? 0 : kg * BM * SK) + (wm * WTM + lr) * SK + sw;
    b_lane[kk] = (KW == 1 ? 0 : kg * BN * SK) + (wn * WTN + lr) * SK + sw;
#if defined(__HIP_DEVICE_COMPILE__)
    __asm__("" : "+v"(a_lane[kk]), "+v"(b_lane[kk]));
#endif
  }
  auto compute = [&](auto st, int kt) {
    const half_t* sa = bufA(st) - (KW == 1 ? 0 : kg * BM * SK);
    const half_t* sb = bufB(st) - (KW == 1 ? 0 : kg * BN * SK);
#pragma unroll
    for (int kk = 0; kk < SK / 32; ++kk) {
      half8 af[MI];
      half8 bf[NI];
      int wo = 0;  // A_CONVW: this lane's window offset for K step kk
      if constexpr (kWin) {
        wo = win_row + win_off((kt + kt_lo) * SK + kk * 32);
#if defined(__HIP_DEVICE_COMPILE__)
        __asm__("" : "+v"(wo));
#endif
#pragma unroll
        for (int i = 0; i < MI; ++i) af[i] = *reinterpret_cast<const half8*>(sWin + wo + i * 16 * win_cw);
      } else {
#pragma unroll
        for (int i = 0; i < MI; ++i)
          af[i] = *reinterpret_cast<const half8*>(sa + a_lane[kk] + i * 16 * SK);
      }
#pragma unroll
      for (int j = 0; j < NI; ++j)
        bf[j] = *reinterpret_cast<const half8*>(sb + b_lane[kk] + j * 16 * SK);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = mfma16x16x32(bf[j], af[i], acc[i][j]);
      if constexpr (SP > 0) {
        half8 afl[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i)
          afl[i] = kWin ? *reinterpret_cast<const half8*>(sWin + win_lo + wo + i * 16 * win_cw)
                        : *reinterpret_cast<const half8*>(sa + kALo + a_lane[kk] + i * 16 * SK);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) accx[i][j] = mfma16x16x32(bf[j], afl[i], accx[i][j]);
      }
      if constexpr (SP == 2) {
        half8 bfl[NI];
#pragma unroll
        for (int j = 0; j < NI; ++j)
          bfl[j] = *reinterpret_cast<const half8*>(sb + kWLo + b_lane[kk] + j * 16 * SK);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) accx[i][j] = mfma16x16x32(bfl[j], af[i], accx[i][j]);
      }
    }
  };

  float rsv[kNormIn ? MI : 1];
  auto norm_in = [&]() {
    if constexpr (kNormIn) {
      // the partials (issued before the NST - 1 + PIPE first stages) have landed
      wait_vmcnt<L * (NST - 1 + PIPE)>();
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < kSsqParts / 4; ++u)
          ss += (ssq_pre[i][u].x + ssq_pre[i][u].y) + (ssq_pre[i][u].z + ssq_pre[i][u].w);
        rsv[i] = p.ssq_in ? 1.0f / sqrtf(ss / 512.0f + 1e-5f) : 1.0f;
      }
    }
  };
  int kt0 = 0;
  floatx4 acc1[PIPE && KG == 2 ? MI : 1][PIPE && KG == 2 ? NI : 1];  // PIPE: the second K part
  if constexpr (PIPE) {
    // Pipelined loop.  The fragments of a K step are read into one of two
    // register slots while the MFMAs of the previous step run, and the one
    // barrier of a stage sits before its last K step:
    //   step kk < KK-1: read step kk+1's fragments; MFMAs of step kk;
    //   last step:      wait for this wave's reads (the stage buffer is free)
    //                   and for its share of stage kt+1; barrier; refill this
    //                   stage's buffer with stage kt+NST; read step 0 of stage
    //                   kt+1; MFMAs of the last step.
    // So the MFMAs after the barrier need no LDS read, and a stage is in
    // flight for NST-1 stage times.  The MFMAs per output element are the
    // same instructions in the same K order as with PIPE = 0.
    constexpr int KK = SK / 32;
    static_assert(KK % 2 == 0, "two register slots alternate over an even number of K steps");
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) acc1[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    half8 fa[2][MI], fb[2][NI];
    half8 fal[SP >= 1 ? 2 : 1][SP >= 1 ? MI : 1], fbl[SP == 2 ? 2 : 1][SP == 2 ? NI : 1];  // split: lo halves
    auto frag_read = [&](auto st, auto kkc, auto slot) {
      constexpr int kk = decltype(kkc)::value;
      constexpr int sl = decltype(slot)::value;
      const half_t* sa = bufA(st);
      const half_t* sb = bufB(st);
#pragma unroll
      for (int i = 0; i < MI; ++i) fa[sl][i] = *reinterpret_cast<const half8*>(sa + a_lane[kk] + i * 16 * SK);
#pragma unroll
      for (int j = 0; j < NI; ++j) fb[sl][j] = *reinterpret_cast<const half8*>(sb + b_lane[kk] + j * 16 * SK);
      if constexpr (SP >= 1) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
          fal[sl][i] = *reinterpret_cast<const half8*>(sa + kALo + a_lane[kk] + i * 16 * SK);
      }
      if constexpr (SP == 2) {
#pragma unroll
        for (int j = 0; j < NI; ++j)
          fbl[sl][j] = *reinterpret_cast<const half8*>(sb + kWLo + b_lane[kk] + j * 16 * SK);
      }
    };
    // Per K step the same MFMAs in the same order as compute() above: the
    // hi.hi products into c, then (split operands) the cross terms into accx.
    auto mma = [&](floatx4 (&c)[MI][NI], auto slot) {
      constexpr int sl = decltype(slot)::value;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) c[i][j] = mfma16x16x32(fb[sl][j], fa[sl][i], c[i][j]);
      if constexpr (SP >= 1) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) accx[i][j] = mfma16x16x32(fb[sl][j], fal[sl][i], accx[i][j]);
      }
      if constexpr (SP == 2) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) accx[i][j] = mfma16x16x32(fbl[sl][j], fa[sl][i], accx[i][j]);
      }
    };
    constexpr int kFragReads = MI + NI + (SP >= 1 ? MI : 0) + (SP == 2 ? NI : 0);
    constexpr int kMfmas = MI * NI * (1 + SP);
    // Every ring buffer is filled before the loop: stage kt's buffer is
    // refilled at stage kt's barrier.
    static_for<0, NST>([&](auto st) { issue(st, (int)decltype(st)::value); });
    norm_in();
    wait_vmcnt<L * (NST - 1)>();  // this wave's share of stage 0 has landed
    __builtin_amdgcn_s_barrier();  // ... for every wave
    frag_read(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{},
              std::integral_constant<int, 0>{});
    // Branch-free loop bodies (a branch would make the compiler's wait
    // counts conservative where paths join): the host launches this form
    // only when each K part is a whole number of NST-stage rounds, so the
    // second part starts again at ring buffer 0.
    auto stage = [&](auto st, int kt, floatx4 (&c)[MI][NI]) {
      constexpr int s = decltype(st)::value;
      static_for<0, KK>([&](auto kkc) {
        constexpr int kk = decltype(kkc)::value;
        constexpr int cur = kk & 1;
        using Nxt = std::integral_constant<int, cur ^ 1>;
        if constexpr (kk + 1 < KK) {
          frag_read(st, std::integral_constant<int, kk + 1>{}, Nxt{});
          mma(c, std::integral_constant<int, cur>{});
          interleave<kFragReads, 0, kMfmas>();
        } else {
          wait_lgkmcnt0();               // this wave's reads of stage kt have returned
          wait_vmcnt<L * (NST - 2)>();   // its share of stage kt+1 has landed
          __builtin_amdgcn_s_barrier();  // ... for every wave
          issue(st, kt + NST);
          frag_read(std::integral_constant<int, (s + 1) % NST>{}, std::integral_constant<int, 0>{}, Nxt{});
          mma(c, std::integral_constant<int, cur>{});
          interleave<kFragReads, L, kMfmas>();
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the K steps in program order
      });
    };
    const int kpart = KT / KG;  // stages per K part, a multiple of NST
    for (; kt0 < kpart; kt0 += NST)
      static_for<0, NST>([&](auto st) { stage(st, kt0 + (int)decltype(st)::value, acc); });
    if constexpr (KG == 2) {
      for (; kt0 < KT; kt0 += NST)
        static_for<0, NST>([&](auto st) { stage(st, kt0 + (int)decltype(st)::value, acc1); });
    }
    if constexpr (kPre) load_pre();
  }
  // Pipeline, one barrier per stage.  At the top of stage kt this wave waits
  // for its own share of stage kt (NST-2 younger stages may stay in flight);
  // the barrier then says every wave's share has landed AND every wave has
  // finished reading stage kt-1, whose buffer is refilled with stage
  // kt+NST-1 before stage kt is computed.  The body is branch-free (an issue
  // past the last stage is a one-address load into a buffer that is not read
  // again), which keeps the compiler from adding waits of its own; the last
  // KT % NST stages are resident when the loop exits.
  if constexpr (!PIPE) {
    if constexpr (kWin) fill_window();
    static_for<0, NST - 1>([&](auto st) { issue(st, (int)decltype(st)::value); });
    norm_in();
    for (; kt0 + NST <= KT; kt0 += NST) {
      static_for<0, NST>([&](auto st) {
        constexpr int s = decltype(st)::value;
        wait_vmcnt<L * (NST - 2)>();   // this wave's share of stage kt0+s has landed
        wait_lgkmcnt0();               // this wave's reads of stage kt0+s-1 have returned
        __builtin_amdgcn_s_barrier();  // ... for every wave
        issue(std::integral_constant<int, (s + NST - 1) % NST>{}, kt0 + s + NST - 1);
        compute(st, kt0 + s);
      });
    }
  }
  wait_vmcnt<0>();  // the tail stages have landed; no DMA outstanding at exit
  __builtin_amdgcn_s_barrier();
  // Late prefetch: the small per-column epilogue operands are requested after
  // the K loop's last wait, so their latency overlaps the resident tail
  // stages' compute without holding registers through the K loop; the
  // folded-norm producer's aw and gamma are multiplied in the epilogue, so
  // nothing waits for them before the tail.  (Issued ahead of that wait, they
  // were covered by it; kept in a lambda or issued before the K loop, the
  // compiler moved the loop's accumulators between registers every stage.)
  float4 bv[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j)
    bv[j] = p.bias ? *reinterpret_cast<const float4*>(p.bias + colj(j)) : make_float4(0.f, 0.f, 0.f, 0.f);
  constexpr bool kColScale = EPI == EPI_F32 || EPI == EPI_F16 || EPI == EPI_RESAVG;
  float4 csv[kColScale ? NI : 1];
  if constexpr (kColScale) {
#pragma unroll
    for (int j = 0; j < NI; ++j)
      csv[j] = p.colscale ? *reinterpret_cast<const float4*>(p.colscale + colj(j))
                          : make_float4(1.f, 1.f, 1.f, 1.f);
  }
  constexpr bool kNormOut = EPI == EPI_F32;
  float4 nsa[kNormOut ? NI : 1], nsg[kNormOut ? NI : 1];
  if constexpr (kNormOut) {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      nsa[j] = p.C16s ? *reinterpret_cast<const float4*>(p.sc_a + colj(j)) : make_float4(0.f, 0.f, 0.f, 0.f);
      nsg[j] = p.C16s ? *reinterpret_cast<const float4*>(p.sc_g + colj(j)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  if constexpr (!PIPE) {
    static_for<0, NST - 1>([&](auto st) {
      if (kt0 + (int)decltype(st)::value < KT) compute(st, kt0 + (int)decltype(st)::value);
    });
  } else if constexpr (KG == 2) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) acc[i][j] += acc1[i][j];  // part 0 + part 1
  }
  if constexpr (SP > 0) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) acc[i][j] += accx[i][j] * kSplitInv;
  }

  // K groups: groups 1..KG-1 hand their partial tiles to group 0 through LDS
  // and leave; group 0 adds them in group order (a fixed order, so the sum is
  // deterministic) and runs the epilogue.  Each partial (BM x BN fp32) goes
  // into one of the idle ring buffers sB0, sA0, sB1 when those hold a tile,
  // else into a buffer of its own.
  if constexpr (KG > 1 && !PIPE) {
    constexpr int kTileBytes = BM * BN * 4;
    constexpr bool kRedInRing = kTileBytes <= KG * BN * SK * 2 &&
                                (KG < 3 || kTileBytes <= KG * BM * SK * 2) && (KG < 4 || NST >= 2);
    constexpr int kPart = NW * MI * NI * 64;  // floatx4 per partial tile
    __shared__ __attribute__((aligned(1024))) floatx4 red_own[kRedInRing ? 1 : (KG - 1) * kPart];
    auto red_buf = [&](int g) -> floatx4* {
      if constexpr (kRedInRing) {
        half_t* b = g == 1 ? sB0 : g == 2 ? sA0 : sB1;
        return reinterpret_cast<floatx4*>(b);
      } else {
        return red_own + (g - 1) * kPart;
      }
    };
    if constexpr (kRedInRing) {
      wait_lgkmcnt0();
      __syncthreads();  // every wave has finished reading the ring
    }
    if (kg > 0) {
      floatx4* red = red_buf(kg);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) red[((wave * MI + i) * NI + j) * 64 + lane] = acc[i][j];
    }
    wait_lgkmcnt0();
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int g = 1; g < KG; ++g) {
      const floatx4* red = red_buf(g);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] += red[((wave * MI + i) * NI + j) * 64 + lane];
    }
  }

  if constexpr (kColScale) {
    if (p.colscale) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] *= floatx4{csv[j].x, csv[j].y, csv[j].z, csv[j].w};
    }
  }

  // ---------------------------------------------------------------- epilogue
  auto st16 = [](half_t* dst, float a, float b, float c, float d) {
    half4 h;
    h[0] = (half_t)a; h[1] = (half_t)b; h[2] = (half_t)c; h[3] = (half_t)d;
    *reinterpret_cast<half4*>(dst) = h;
  };
  // f16 output of a split operand: hi at dst, lo at dst + p.c16_lo (when set).
  auto st16s = [&](half_t* dst, float a, float b, float c, float d) {
    if (!p.c16_lo) {
      st16(dst, a, b, c, d);
      return;
    }
    half_t hv[4], lv[4];
    split_f16(a, hv[0], lv[0]);
    split_f16(b, hv[1], lv[1]);
    split_f16(c, hv[2], lv[2]);
    split_f16(d, hv[3], lv[3]);
    const half4 h = {hv[0], hv[1], hv[2], hv[3]};
    const half4 l = {lv[0], lv[1], lv[2], lv[3]};
    *reinterpret_cast<half4*>(dst) = h;
    *reinterpret_cast<half4*>(dst + p.c16_lo) = l;
  };

  float4 nsc[kNormOut ? NI : 1];  // producer of a folded norm: aw * gamma per column
  if constexpr (kNormOut) {
#pragma unroll
    for (int j = 0; j < NI; ++j) nsc[j] = make_float4(nsa[j].x * nsg[j].x, nsa[j].y * nsg[j].y,
                                                      nsa[j].z * nsg[j].z, nsa[j].w * nsg[j].w);
  }
  if constexpr (EPI == EPI_F32 || EPI == EPI_F16 || EPI == EPI_DUAL || EPI == EPI_RESSKIP ||
                EPI == EPI_FINALSKIP || EPI == EPI_RESAVG) {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = row_base + 16 * i;
      const bool live = m < p.M;
      float ssq[(NI + 1) / 2];  // EPI_F32 with ssq_out: this lane's share per 32-column block
      float s1[(NI + 1) / 2];   // ... and with sum_out
#pragma unroll
      for (int q = 0; q < (NI + 1) / 2; ++q) ssq[q] = s1[q] = 0.0f;
      float4 pv = make_float4(0.f, 0.f, 0.f, 0.f);  // column pairs: the even block's outputs
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int n = colj(j);
        float4 v = make_float4(acc[i][j][0] + bv[j].x, acc[i][j][1] + bv[j].y,
                               acc[i][j][2] + bv[j].z, acc[i][j][3] + bv[j].w);
        if constexpr (EPI == EPI_RESAVG) {
          if (!live || (p.n_store && n >= p.n_store)) continue;
          const float4 r = pre_a[i][j];
          v = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
          if (p.C32) *reinterpret_cast<float4*>(p.C32 + (size_t)m * p.ldc32 + n) = v;
          float4* g = reinterpret_cast<float4*>(p.C32b + (size_t)m * p.ldc32b + n);
          const float4 g0 = p.flag ? *g : make_float4(0.f, 0.f, 0.f, 0.f);
          const float4 g1 = make_float4(g0.x + v.x / 3.0f, g0.y + v.y / 3.0f, g0.z + v.z / 3.0f,
                                        g0.w + v.w / 3.0f);
          *g = g1;
          if (p.C16) st16s(p.C16 + (size_t)m * p.ldc16 + n, g1.x, g1.y, g1.z, g1.w);
          continue;
        }
        if (p.n_store && n >= p.n_store) continue;  // zero-padded weight rows
        if constexpr (EPI == EPI_F32) {
          if (p.res) {
            const float4 r = pre_a[i][j];
            v = make_float4(r.x + v.x, r.y + v.y, r.z + v.z, r.w + v.w);
          }
          ssq[j / 2] += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
          s1[j / 2] += (v.x + v.y) + (v.z + v.w);
          if (!live) continue;
          if (p.C32) *reinterpret_cast<float4*>(p.C32 + (size_t)m * p.ldc32 + n) = v;
          if (perm) {
            // blocks j - 1 and j hold columns n - 4 .. n + 3: one 16-byte store each
            if ((j & 1) == 0) {
              pv = v;
            } else {
              const float4 pn = nsc[j - 1], cn = nsc[j];
              if (p.C16) {
                half8 h;
                h[0] = (half_t)pv.x; h[1] = (half_t)pv.y; h[2] = (half_t)pv.z; h[3] = (half_t)pv.w;
                h[4] = (half_t)v.x; h[5] = (half_t)v.y; h[6] = (half_t)v.z; h[7] = (half_t)v.w;
                *reinterpret_cast<half8*>(p.C16 + (size_t)m * p.ldc16 + n - 4) = h;
              }
              if (p.C16s) {
                half8 h;
                h[0] = (half_t)(pv.x * pn.x); h[1] = (half_t)(pv.y * pn.y);
                h[2] = (half_t)(pv.z * pn.z); h[3] = (half_t)(pv.w * pn.w);
                h[4] = (half_t)(v.x * cn.x); h[5] = (half_t)(v.y * cn.y);
                h[6] = (half_t)(v.z * cn.z); h[7] = (half_t)(v.w * cn.w);
                *reinterpret_cast<half8*>(p.C16s + (size_t)m * p.ldc16s + n - 4) = h;
              }
            }
            continue;
          }
          if (p.C16) st16(p.C16 + (size_t)m * p.ldc16 + n, v.x, v.y, v.z, v.w);
          if (p.C16s)
            st16(p.C16s + (size_t)m * p.ldc16s + n, v.x * nsc[j].x, v.y * nsc[j].y,
                 v.z * nsc[j].z, v.w * nsc[j].w);
          continue;
        }
        if (!live) continue;
        if constexpr (EPI == EPI_F16) {
          st16s(p.C16 + (size_t)m * p.ldc16 + n, v.x, v.y, v.z, v.w);
        } else if constexpr (EPI == EPI_DUAL) {
          const int half_n = p.N >> 1;
          if (n < half_n) {
            *reinterpret_cast<float4*>(p.C32 + (size_t)m * p.ldc32 + n) = v;
            st16(p.C16 + (size_t)m * p.ldc16 + n, v.x, v.y, v.z, v.w);
          } else {
            *reinterpret_cast<float4*>(p.C32b + (size_t)m * p.ldc32b + (n - half_n)) = v;
          }
        } else if constexpr (EPI == EPI_RESSKIP) {
          // v is the res_skip conv output (bias included).
          const float mk = pre_mask[i] ? 1.0f : 0.0f;
          // the skip accumulator starts at zero when flag is 0
          const float4 o = n < 512 || p.flag ? pre_a[i][j] : make_float4(0.f, 0.f, 0.f, 0.f);
          if (n < 512) {
            const float4 xn = make_float4((o.x + v.x) * mk, (o.y + v.y) * mk, (o.z + v.z) * mk,
                                          (o.w + v.w) * mk);
            *reinterpret_cast<float4*>(p.C32 + (size_t)m * p.ldc32 + n) = xn;
            st16(p.C16 + (size_t)m * p.ldc16 + n, xn.x, xn.y, xn.z, xn.w);
          } else {
            *reinterpret_cast<float4*>(p.C32b + (size_t)m * p.ldc32b + (n - 512)) =
                make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
          }
        } else {  // EPI_FINALSKIP: out = (out + rs) * mask; final_in = out + rp
          const float mk = pre_mask[i] ? 1.0f : 0.0f;
          const float4 o = pre_a[i][j];
          const float4 r = pre_b[i][j];
          *reinterpret_cast<float4*>(p.C32 + (size_t)m * p.ldc32 + n) =
              make_float4((o.x + v.x) * mk + r.x, (o.y + v.y) * mk + r.y, (o.z + v.z) * mk + r.z,
                          (o.w + v.w) * mk + r.w);
        }
      }
      if constexpr (EPI == EPI_F32) {
        if (p.ssq_out) {
          static_assert(WTN % 32 == 0, "a folded-norm producer covers whole 32-column blocks");
          // The four lanes of a row (lane groups lg) hold each 32-column block.
#pragma unroll
          for (int q = 0; q < NI / 2; ++q) {
            float t = ssq[q];
            t += __shfl_xor(t, 16, kWave);
            t += __shfl_xor(t, 32, kWave);
            if (live && lg == 0)
              p.ssq_out[(size_t)m * kSsqParts + ((n0 + wn * WTN + 32 * q) >> 5)] = t;
          }
        }
        if (p.sum_out) {
#pragma unroll
          for (int q = 0; q < NI / 2; ++q) {
            float t = s1[q];
            t += __shfl_xor(t, 16, kWave);
            t += __shfl_xor(t, 32, kWave);
            if (live && lg == 0)
              p.sum_out[(size_t)m * kSsqParts + ((n0 + wn * WTN + 32 * q) >> 5)] = t;
          }
        }
      }
    }
  } else {
    if constexpr (EPI == EPI_QKV) {
      if (n0 >= 1024) {
        // V tile = BN/64 heads x BM tokens.  Transpose through LDS so that
        // V^T[d][t] is written by consecutive lanes at consecutive t.
        static_assert(BN % 64 == 0, "a v tile must hold whole heads");
        // The staging tile [BN channels][BM rows] reuses ring buffers, free
        // once every wave is past its last MFMA: the first W stage buffer when
        // it is large enough, else 64 channels in each A stage buffer.
        static_assert(SK >= BM || (SK == 64 && BN <= 64 * NST), "no ring buffer holds the V^T staging tile");
        auto stg = [&](int c) -> half_t* {
          if constexpr (SK >= BM) {
            return sB0 + c * BM;
          } else {
            half_t* b = c < 64 ? sA0 : c < 128 ? sA1 : sA2;
            return b + (c & 63) * BM;
          }
        };
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        // Blocks (2q, 2q+1) of this wave hold the even / odd channels of one
        // 32-channel group (v rows are permuted like the q and k rows):
        // tile channel c = 32 g + 2 (4 lg + r) (+1 for the odd block).
#pragma unroll
        for (int q = 0; q < NI / 2; ++q) {
          const int g = (wn * WTN + 32 * q) >> 5;
          const float bev[4] = {bv[2 * q].x, bv[2 * q].y, bv[2 * q].z, bv[2 * q].w};
          const float bov[4] = {bv[2 * q + 1].x, bv[2 * q + 1].y, bv[2 * q + 1].z, bv[2 * q + 1].w};
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int rl = wm * WTM + i * 16 + lr;
              const int c = 32 * g + 2 * (4 * lg + r);
              stg(c)[rl] = f16_of(__builtin_fmaf(rsv[i], acc[i][2 * q][r], bev[r]));
              stg(c + 1)[rl] = f16_of(__builtin_fmaf(rsv[i], acc[i][2 * q + 1][r], bov[r]));
            }
        }
        wait_lgkmcnt0();  // this wave's stores have landed before the barrier releases readers
        __builtin_amdgcn_s_barrier();
        const int h0 = (n0 - 1024) >> 6;
#pragma unroll
        for (int rr = 0; rr < BM; rr += 64) {
          const int rl = rr + lane;
          const int m = m0 + rl;
          if (rl < BM && m < p.M) {
            const int b = m / p.T;
            const int t = m - b * p.T;
            for (int c = wave; c < BN; c += NW)
              p.vt[(((size_t)b * 8 + h0 + (c >> 6)) * 64 + (c & 63)) * p.Tpad + t] = stg(c)[rl];
          }
        }
        return;
      }
    }
    // Paired epilogues: blocks (2q, 2q+1) of a wave hold, in the same lane and
    // slot r, the two operands of output channel c = 16 group + 4 lg + r.
    static_assert(NI % 2 == 0, "paired epilogue needs an even block count");
#pragma unroll
    for (int q = 0; q < NI / 2; ++q) {
      const int ce = col_base + q * 32;  // GEMM column of this lane's even-block values
      const int group = (ce - 4 * lg) >> 5;
      const float4 be = bv[2 * q];
      const float4 bo = bv[2 * q + 1];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = row_base + 16 * i;
        if (m >= p.M) continue;
        float rs_row = 1.0f;  // rs of the row when the AdaRMSNorm is folded in
        if constexpr (kNormIn) rs_row = rsv[i];
        const float ve[4] = {__builtin_fmaf(rs_row, acc[i][2 * q][0], be.x),
                             __builtin_fmaf(rs_row, acc[i][2 * q][1], be.y),
                             __builtin_fmaf(rs_row, acc[i][2 * q][2], be.z),
                             __builtin_fmaf(rs_row, acc[i][2 * q][3], be.w)};
        const float vo[4] = {__builtin_fmaf(rs_row, acc[i][2 * q + 1][0], bo.x),
                             __builtin_fmaf(rs_row, acc[i][2 * q + 1][1], bo.y),
                             __builtin_fmaf(rs_row, acc[i][2 * q + 1][2], bo.z),
                             __builtin_fmaf(rs_row, acc[i][2 * q + 1][3], bo.w)};
        if constexpr (EPI == EPI_SWIGLU) {
          const int c = group * 16 + 4 * lg;
          float y[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = silu_fast(ve[r]) * vo[r];
          st16(p.C16 + (size_t)m * p.ldc16 + c, y[0], y[1], y[2], y[3]);
        } else if constexpr (EPI == EPI_GATE) {
          const int c = group * 16 + 4 * lg;
          const float4 ca = pre_ca[q];
          const float4 cb = pre_cb[q];
          const float cav[4] = {ca.x, ca.y, ca.z, ca.w};
          const float cbv[4] = {cb.x, cb.y, cb.z, cb.w};
          float y[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = tanh_sat(ve[r] + cav[r]) * sigmoid_f(vo[r] + cbv[r]);
          st16(p.C16 + (size_t)m * p.ldc16 + c, y[0], y[1], y[2], y[3]);
        } else {  // EPI_QKV, q and k sections (v tiles are written above)
          const int o = group * 32 + 8 * lg;  // original column of the first even element
          const int sec = o >> 9;             // 0 = q, 1 = k
          const int hh = (o & 511) >> 6;
          const int d0 = o & 63;
          const int b = m / p.T;
          const int t = m - b * p.T;
          const size_t head = (size_t)b * 8 + hh;
          const float2* cs = p.rope + t * 32 + (d0 >> 1);
          // q carries the softmax scale in log2 units, log2(e) / sqrt(64), so the
          // attention's scores come out of the matrix cores ready for exp2
          // (one rounding to f16 either way)
          const float sc = sec == 0 ? 0.125f * 1.4426950408889634f : 1.0f;
          half8 h;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float2 rot = rope_rotate(ve[r], vo[r], cs[r]);
            h[2 * r] = f16_of(rot.x * sc);
            h[2 * r + 1] = f16_of(rot.y * sc);
          }
          half_t* dst = (sec == 0 ? p.q : p.k) + (head * p.Tpad + t) * 64 + d0;
          *reinterpret_cast<half8*>(dst) = h;
        }
      }
    }
  }
}

// QKV product of long sequences (K = 512, N = 1536) with the row block kept
// resident.  A persistent grid of kQkvRowsGrid workgroups; workgroup r takes
// a contiguous range of the work items (row block, 128-column tile), ordered
// row block first, so it loads each 64 x 512 A block into LDS once and then
// streams only W's 128-row column tiles through a 4-stage ring that runs on
// from one item to the next (no per-tile fill or drain).  Eight wavefronts of
// 32 x 32.  The MFMAs run in the same K order as gemm_kernel's and the
// epilogue is its QKV epilogue (rs, bias, RoPE, the q scale, f16_of), so
// every output has the same bits as with the 64 x 64 / 64 x 128 tiles.  The
// row blocks are tm's computed row tiles (row skipping included); the
// workgroups of one XCD take neighbouring ranges.
constexpr int kQkvRowsGrid = 256;

__global__ __launch_bounds__(512) void qkv_rows_kernel(GemmArgs p, TileMap tm) {
  constexpr int BM = 64, BN = 128, K = 512, SK = 64, KT = K / SK, WN = 4, NW = 8, NSTW = 4;
  constexpr int WTM = 32, WTN = 32, MI = 2, NI = 2;
  constexpr int LAB = BM * (K / 8) / (64 * NW);  // 16-byte A loads per lane per row block
  constexpr int LB = BN * (SK / 8) / (64 * NW);  // 16-byte W loads per lane per stage
  constexpr int nN = 1536 / BN;
  __shared__ __attribute__((aligned(1024))) half_t sA[BM * K];
  __shared__ __attribute__((aligned(1024))) half_t sW0[BN * SK];
  __shared__ __attribute__((aligned(1024))) half_t sW1[BN * SK];
  __shared__ __attribute__((aligned(1024))) half_t sW2[BN * SK];
  __shared__ __attribute__((aligned(1024))) half_t sW3[BN * SK];
  __shared__ __attribute__((aligned(1024))) half_t sV[BN * BM];  // V^T staging [channel][row]
  auto bufW = [&](auto st) -> half_t* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sW0;
    else if constexpr (s == 1) return sW1;
    else if constexpr (s == 2) return sW2;
    else return sW3;
  };
  const int items = tm.nM * nN;
  const int bid = blockIdx.x;
  const int r8 = (bid & 7) * (kQkvRowsGrid / 8) + (bid >> 3);
  const int i0 = (int)((long)r8 * items / kQkvRowsGrid), i1 = (int)((long)(r8 + 1) * items / kQkvRowsGrid);
  if (i0 >= i1) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave - wm * WN;
  const int lr = lane & 15, lg = lane >> 4;
  const buffer_rsrc_t rA = make_buffer_rsrc(p.A, (int)((size_t)p.M * p.lda * 2));
  const buffer_rsrc_t rW = make_buffer_rsrc(p.W, (int)((size_t)p.N * p.ldw * 2));
  // W stage rows hold 8 slots, slot of chunk c at c ^ ((row >> 1) & 7); A
  // rows hold 64, chunk c at c ^ (row & 15) (16 consecutive rows read at one
  // chunk hit distinct banks either way).
  int voW[LB];
#pragma unroll
  for (int j = 0; j < LB; ++j) {
    const int q = (wave * LB + j) * 64 + lane;
    const int row = q >> 3;
    voW[j] = (row * p.ldw + (((q & 7) ^ ((row >> 1) & 7)) * 8)) * 2;
  }
  // A fragment offsets: K stage kt reads chunk 8 kt + 4 kk + lg of row
  // wm*32 + 16 i + lr, at slot (8 kt + 4 kk + lg) ^ lr = 8 (kt ^ (lr >> 3)) +
  // ((4 kk + lg) ^ (lr & 7)); the kt-parity part is a_off[kt & 1].
  const int h8 = lr >> 3;
  int a_off[2][2];
#pragma unroll
  for (int pp = 0; pp < 2; ++pp)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      a_off[pp][kk] = (wm * WTM + lr) * K + ((pp ^ h8) * 64) + (((kk * 4 + lg) ^ (lr & 7)) * 8);
  int b_off[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) b_off[kk] = (wn * WTN + lr) * SK + (((kk * 4 + lg) ^ ((lr >> 1) & 7)) * 8);
  __asm__("" : "+v"(a_off[0][0]), "+v"(a_off[0][1]), "+v"(a_off[1][0]), "+v"(a_off[1][1]), "+v"(b_off[0]),
          "+v"(b_off[1]));
  // head dims d0 .. d0 + 7 of this lane's q / k outputs (the same in every column tile)
  const int d0 = (wn * WTN + 8 * lg) & 63;
  float rsv[MI];
  float2 csv[MI][4];
  auto row_block = [&](int rc) {  // computed row tile -> row tile
    int first = tm.seg_first[0], cum = 0;
    if (tm.nseg == 0) return rc;
#pragma unroll
    for (int s = 1; s < kMaxRowSeq; ++s) {
      if (s < tm.nseg && rc >= tm.seg_cum[s]) {
        first = tm.seg_first[s];
        cum = tm.seg_cum[s];
      }
    }
    return first + (rc - cum);
  };
  // A block, rs and the rotary (cos, sin) of this lane's rows
  auto load_rows = [&](int rb) {
#pragma unroll
    for (int j = 0; j < LAB; ++j) {
      const int q = (wave * LAB + j) * 64 + lane;
      const int row = q >> 6;
      const int c = (q & 63) ^ (row & 15);
      const int m = min(rb * BM + row, p.M - 1);
      buffer_load_lds16(rA, (lds_ptr_t*)(sA + (wave * LAB + j) * 64 * 8), (m * p.lda + c * 8) * 2, 0);
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = rb * BM + wm * WTM + 16 * i + lr;
      float4 sp[kSsqParts / 4];
#pragma unroll
      for (int u = 0; u < kSsqParts / 4; ++u)
        sp[u] = (p.ssq_in && m < p.M) ? reinterpret_cast<const float4*>(p.ssq_in + (size_t)m * kSsqParts)[u]
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
      float ss = 0.0f;
#pragma unroll
      for (int u = 0; u < kSsqParts / 4; ++u) ss += (sp[u].x + sp[u].y) + (sp[u].z + sp[u].w);
      rsv[i] = p.ssq_in ? 1.0f / sqrtf(ss / 512.0f + 1e-5f) : 1.0f;
      const int mc = min(m, p.M - 1);
      const int t = mc - (mc / p.T) * p.T;
      const float2* cs = p.rope + t * 32 + (d0 >> 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) csv[i][r] = cs[r];
    }
  };
  // W stage kt of item's column tile into ring buffer st; past the range's
  // last item it re-reads that item's last stage (never used).
  auto issue = [&](auto st, int item, int kt) {
    if (item >= i1) {
      item = i1 - 1;
      kt = KT - 1;
    }
    const int cb = item % nN;
    half_t* sw = bufW(st);
#pragma unroll
    for (int j = 0; j < LB; ++j)
      buffer_load_lds16(rW, (lds_ptr_t*)(sw + (wave * LB + j) * 64 * 8), voW[j], (cb * BN * p.ldw + kt * SK) * 2);
  };
  floatx4 acc[MI][NI];
  int item = i0;
  int rc = item / nN;
  int rb = row_block(rc);
  load_rows(rb);
  static_for<0, NSTW - 1>([&](auto st) { issue(st, item, (int)decltype(st)::value); });
  while (true) {
    const int n0 = (item % nN) * BN;
    float4 bv[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j)
      bv[j] = p.bias ? *reinterpret_cast<const float4*>(p.bias + n0 + wn * WTN + 16 * j + 4 * lg)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    static_for<0, KT>([&](auto ktc) {
      constexpr int kt = decltype(ktc)::value;
      // stage kt has landed (vector memory operations complete in issue
      // order; at most NSTW - 2 stages stay in flight behind it)
      wait_vmcnt<LB * (NSTW - 2)>();
      wait_lgkmcnt0();
      __builtin_amdgcn_s_barrier();
      {
        // the buffer of stage kt - 1, free now that every wave is past it
        constexpr int kn = kt + NSTW - 1;
        issue(std::integral_constant<int, kn % NSTW>{}, kn < KT ? item : item + 1, kn < KT ? kn : kn - KT);
      }
      const half_t* sw = bufW(std::integral_constant<int, kt % NSTW>{});
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        half8 af[MI], bf[NI];
#pragma unroll
        for (int i = 0; i < MI; ++i)
          af[i] = *reinterpret_cast<const half8*>(sA + a_off[kt & 1][kk] + (kt - (kt & 1)) * 64 + i * 16 * K);
#pragma unroll
        for (int j = 0; j < NI; ++j) bf[j] = *reinterpret_cast<const half8*>(sw + b_off[kk] + j * 16 * SK);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) acc[i][j] = mfma16x16x32(bf[j], af[i], acc[i][j]);
      }
    });
    const int m0 = rb * BM;
    const float be[4] = {bv[0].x, bv[0].y, bv[0].z, bv[0].w};
    const float bo[4] = {bv[1].x, bv[1].y, bv[1].z, bv[1].w};
    if (n0 >= 1024) {
      // V: stage [128 channels][64 rows]; then consecutive lanes write consecutive t of V^T
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rl = wm * WTM + i * 16 + lr;
          const int c = 32 * wn + 2 * (4 * lg + r);
          sV[c * BM + rl] = f16_of(__builtin_fmaf(rsv[i], acc[i][0][r], be[r]));
          sV[(c + 1) * BM + rl] = f16_of(__builtin_fmaf(rsv[i], acc[i][1][r], bo[r]));
        }
      wait_lgkmcnt0();
      __builtin_amdgcn_s_barrier();
      const int h0 = (n0 - 1024) >> 6;
      const int m = m0 + lane;
      if (m < p.M) {
        const int b = m / p.T;
        const int t = m - b * p.T;
        for (int c = wave; c < BN; c += NW)
          p.vt[(((size_t)b * 8 + h0 + (c >> 6)) * 64 + (c & 63)) * p.Tpad + t] = sV[c * BM + lane];
      }
    } else {
      const int o = n0 + wn * WTN + 8 * lg;  // original column of the first even element
      const int sec = o >> 9;                 // 0 = q, 1 = k
      const int hh = (o & 511) >> 6;
      const float sc = sec == 0 ? 0.125f * 1.4426950408889634f : 1.0f;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = m0 + wm * WTM + 16 * i + lr;
        if (m >= p.M) continue;
        const float ve[4] = {__builtin_fmaf(rsv[i], acc[i][0][0], be[0]), __builtin_fmaf(rsv[i], acc[i][0][1], be[1]),
                             __builtin_fmaf(rsv[i], acc[i][0][2], be[2]), __builtin_fmaf(rsv[i], acc[i][0][3], be[3])};
        const float vo[4] = {__builtin_fmaf(rsv[i], acc[i][1][0], bo[0]), __builtin_fmaf(rsv[i], acc[i][1][1], bo[1]),
                             __builtin_fmaf(rsv[i], acc[i][1][2], bo[2]), __builtin_fmaf(rsv[i], acc[i][1][3], bo[3])};
        const int b = m / p.T;
        const int t = m - b * p.T;
        const size_t head = (size_t)b * 8 + hh;
        half8 h;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float2 rot = rope_rotate(ve[r], vo[r], csv[i][r]);
          h[2 * r] = f16_of(rot.x * sc);
          h[2 * r + 1] = f16_of(rot.y * sc);
        }
        half_t* dst = (sec == 0 ? p.q : p.k) + (head * p.Tpad + t) * 64 + d0;
        *reinterpret_cast<half8*>(dst) = h;
      }
    }
    ++item;
    if (item >= i1) break;
    if (item / nN != rc) {
      // next row block: every wave is done with sA (and sV) before it is refilled
      wait_lgkmcnt0();
      __builtin_amdgcn_s_barrier();
      rc = item / nN;
      rb = row_block(rc);
      load_rows(rb);
      wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
    }
  }
  wait_vmcnt<0>();  // the range's trailing stage loads have landed before the LDS is released
}

// Chooses the XCD rectangle split minimising the bytes the XCDs re-read:
// A (M x a_cols distinct values; a_cols < K for the k=5 conv, whose taps
// re-read the same rows) is read once per rectangle column, W (N x K) once
// per rectangle row.
static TileMap make_tile_map(const GemmArgs& a, int M, int N, int K, int a_cols, int BM, int BN) {
  TileMap t;
  t.nM = (M + BM - 1) / BM;
  t.nN = N / BN;
  t.nseg = 0;
  for (int s = 0; s < kMaxRowSeq; ++s) t.seg_first[s] = t.seg_cum[s] = 0;
  if (a.row_nb > 0) {
    // Row tiles [lo, hi] of each sequence's needed rows, merged where they
    // touch; sequences come in row order, so the runs do too.
    int lo = -1, hi = -1, total = 0;
    auto flush = [&]() {
      t.seg_first[t.nseg] = lo;
      t.seg_cum[t.nseg] = total;
      total += hi - lo + 1;
      ++t.nseg;
    };
    for (int b = 0; b < a.row_nb; ++b) {
      const int blo = b * a.row_T / BM, bhi = (b * a.row_T + a.row_need[b] - 1) / BM;
      if (lo >= 0 && blo <= hi + 1) {
        hi = std::max(hi, bhi);
      } else {
        if (lo >= 0) flush();
        lo = blo;
        hi = bhi;
      }
    }
    flush();
    t.nM = total;
    M = total * BM;
  }
  const double a_bytes = 2.0 * M * a_cols, w_bytes = 2.0 * N * K;
  const int opts[4][2] = {{8, 1}, {4, 2}, {2, 4}, {1, 8}};
  double best = 1e300;
  t.Xm = 8;
  t.Xn = 1;
  for (const auto& o : opts) {
    const int xm = o[0], xn = o[1];
    if (xm > t.nM || xn > t.nN) continue;
    const double cost = a_bytes * xn + w_bytes * xm;
    if (cost < best) {
      best = cost;
      t.Xm = xm;
      t.Xn = xn;
    }
  }
  if (t.Xm > t.nM || t.Xn > t.nN) {  // tiny grids: fall back to whatever fits
    t.Xm = t.nM >= 8 ? 8 : 1;
    t.Xn = 8 / t.Xm;
  }
  int mx = 0;
  for (int x = 0; x < 8; ++x) {
    const int rx = x / t.Xn, ry = x % t.Xn;
    const int rm = (rx + 1) * t.nM / t.Xm - rx * t.nM / t.Xm;
    const int rn = (ry + 1) * t.nN / t.Xn - ry * t.nN / t.Xn;
    mx = std::max(mx, rm * rn);
  }
  t.per_xcd = mx;
  return t;
}

template <int BM, int BN, int SK, int NST, int AM, int EPI, int WM = 2, int WN = 2, int KG = 1,
          int SP = 0, int PIPE = 0>
static hipError_t launch_tile(const GemmArgs& a, hipStream_t s) {
  if ((a.K / SK) % KG != 0) return hipErrorInvalidValue;  // both K parts need equal stage counts
  if (PIPE && (a.K / SK / KG) % NST != 0) return hipErrorInvalidValue;  // whole rounds per part
  const TileMap tm = make_tile_map(
      a, a.M, a.N, a.K, AM == A_CONV5 || AM == A_CONV3Z || AM == A_CONVP || AM == A_CONVW ? a.conv_c : a.K,
      BM, BN);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, SK, NST, AM, EPI, WM, WN, KG, SP, PIPE>), dim3(8 * tm.per_xcd),
                     dim3(64 * WM * WN * (PIPE ? 1 : KG)), 0, s,
                     a, tm);
  return hipGetLastError();
}

// Tile, stage and wavefront choice, swept at M = 1720 (B = 2, T = 860) on
// MI355X.  Two limits decide it: the L2 -> CU path delivers about 48 B/clk
// per CU whatever the load method or depth, so a K loop's time is its total
// operand bytes, 2MNK (1/BM + 1/BN), spread over the CUs; and a workgroup of
// four wavefronts alone on a CU cannot hide its LDS and MFMA latencies.
//  * wide outputs use big tiles with eight wavefronts (two per SIMD) and
//    about one tile per CU: w1|w3 (N = 3072) 128x192, 11.8 vs 15.4 us for
//    64x64; the k=5 conv (N = 1024, K = 2560) 64x128 with 64-wide stages,
//    16.5 us (17.2 with 128-wide stages, 21.3 with 64x64 tiles); res/skip
//    and conv1|res_projection (N = 1024) 64x128;
//  * N = 512 outputs and QKV keep 64x64 tiles with four wavefronts in a
//    3-stage ring (three workgroups per CU): larger tiles leave too few
//    tiles to cover the CUs.  The long-K ones (K >= 1024) add a second
//    group of four wavefronts that takes half of the K stages, and so does
//    the k=5 conv (a second group of eight).
// The K split depends on N and K only, never on M, so a request's result
// does not depend on the batch it is decoded with.
//
// Whether a BM x BN tiling leaves most CUs idle: then 32-row tiles with the
// same K split spread the product over more CUs (the per-CU operand rate,
// not the total, limits these K loops).  At M = 256 (a T = 128 CFG pair):
// the k=5 conv 10.5 vs 15.5 us, w1|w3 5.2 vs 8.7, w2 5.9 vs 7.0.  Only the
// tile shape changes, never the K split or the order of the MFMAs over K, so
// a row's result is the same bits whichever tiling the batch gets.
static bool few_tiles(const GemmArgs& a, int BM, int BN) {
  return (long)((a.M + BM - 1) / BM) * (a.N / BN) < 128;
}

// Large products (the padded multi-request and long-form decodes) take the
// pipelined loop (PIPE = 1) with bigger tiles once the tiling still gives
// every CU a tile: it computes the same MFMAs in the same K order as the
// tiles above, so the choice changes no bit of a row's result.  Swept at
// M = 1720 / 6000 / 21568 (B = 2 x T = 860 / 3000, B = 16 x T = 1348):
//  * k=5 conv (N = 1024, K = 2560): 192x128 tiles, eight wavefronts, a
//    4-stage ring: 36.0 vs 46.7 us at M = 6000, 139.5 vs 200.9 at 21568
//    (slower at 1720, where it leaves 184 CUs idle);
//  * long-K N = 512 products (w2 K = 1536): 192x128 at M = 21568, 46.4 vs
//    83.2 us; 128x128 at M = 6000, 17.0 vs 24.0 us.
// The short-K products (K = 512: w1|w3, QKV, wo, res/skip) stay on the
// tiles above, which the pipelined loop did not beat at any M.
// Row tiles a launch covers: ceil(M / BM), or with row skipping the merged
// runs of each sequence's needed rows, as make_tile_map lays them out.
static long row_tiles(const GemmArgs& a, int BM) {
  if (a.row_nb <= 0) return (a.M + BM - 1) / BM;
  long total = 0;
  int lo = -1, hi = -1;
  for (int b = 0; b < a.row_nb; ++b) {
    const int blo = b * a.row_T / BM, bhi = (b * a.row_T + a.row_need[b] - 1) / BM;
    if (lo >= 0 && blo <= hi + 1) {
      hi = std::max(hi, bhi);
    } else {
      if (lo >= 0) total += hi - lo + 1;
      lo = blo;
      hi = bhi;
    }
  }
  return total + hi - lo + 1;
}
static long tile_count(const GemmArgs& a, int BM, int BN) { return row_tiles(a, BM) * (a.N / BN); }

// Relative time of a pipelined tiling: its rounds of tiles over the 256 CUs
// (one workgroup per CU at these ring sizes) times the tile's area over the
// fraction of peak it reaches at large M (measured standalone at M = 21568).
// At the full padded batch this picks 192 x 128 for the conv (139.5 vs 149.7
// us measured against 128 x 128); with the padding skipped the needed row
// tiles leave 192 x 128 a last round mostly idle, and 128 x 128 wins.
static double pipe_cost(long tiles, int BM, int BN, double rate) {
  return (double)((tiles + 255) / 256) * BM * BN / rate;
}
template <int KG, int NST>
static bool pipe_fits(const GemmArgs& a) {
  return a.K % (64 * KG * NST) == 0;  // each K part a whole number of rounds of the ring
}

// Split-operand launches (fp32-level products, GemmArgs::split): everything
// but the vocoder runs 64 x 64 (or 32 x 64) tiles with one K group, so the
// doubled ring stays within the LDS.  The vocoder's convs (A split, weight-normed v exact
// in f16: SP = 1) take the pipelined loop once a stage's row tiles fill most
// of the chip, else the f16 tile choice (their rings double, still one or
// two workgroups per CU).  Swept at the 860-frame call (every candidate
// bit-equal to the 64 x 128 tile; us per launch, first conv of each pair
// at dilation 1 / 3 / 5 and the second at 1 alike):
//  * M = 3,440, N = 768 (after the first upsampler): 128 x 128, 3-stage
//    ring: k = 3 / 7 / 11 at 43.3-44.4 / 88.5-90.0 / 131.6-135.2 against
//    52.3 / 109.2-110.0 / 165.5-170.2 (192 x 128 tiles are too few there);
//  * M = 13,760, N = 384: 192 x 128 with a 2-stage ring at k = 3 / 7 (one
//    round of 216 tiles against 1.27 rounds of 128 x 128): 39.5-40.1 /
//    73.4-74.9 against 47.4 / 92.0-92.1; at k = 11 (K = 4224) the 2-stage
//    ring falls behind (199-201) and 128 x 128 with three stages wins:
//    137.6-142.7 against 169.7-172.6;
//  * M = 27,520, N = 192: 64 x 192 (4 x 2 wavefronts of 16 x 96), 3-stage
//    ring: k = 3 / 7 / 11 at 29.3 / 45.5 / 62.0 against 36.0 / 62.8-63.4 /
//    90.9-91.0;
//  * M = 55,040, N = 96 (K = 320 / 704 / 1088: a prime number of stages, so
//    the plain loop): 128 x 96 tiles of 4 x 1 wavefronts, k = 3 / 11 at
//    27.4 / 57.5 against 30.2-30.4 / 63.5-63.8 for 64 x 96 and 31.4 / 72.6
//    for 64 x 32 (64 x 96 below 256 tiles).  128- and 256-row tiles lose at
//    the 48- and 24-channel stages (one workgroup per CU).
// The transposed convs (SP = 2) found nothing faster.
// A_CONVW: the vocoder's narrower convs (24 to 192 channels), whose
// streamed form re-reads every input row once per tap, keep the row block's
// input window in LDS and stream only W (the same MFMAs in the same K order
// as the streamed form, so the same bits).  Tiles: the streamed form's for
// 24 and 96 channels; 128 x 64 (4 x 1 waves) for 48 channels at >= 256 row
// tiles; 64 x 192 with a 2-stage W ring for 192 channels (the window leaves
// no room for a third).  The window must fit its LDS buffer, and conv_c >= 24
// (a lane's K chunk is at most one tap past its K step's first position).
template <int BM, int BN, int NW, int SP>
static bool conv_window_fits(const GemmArgs& a) {
  constexpr long AS = SP >= 1 ? 2 : 1;
  const long chunks = AS * (BM + (long)(a.conv_k - 1) * a.conv_d) * conv_window_chunks(a.conv_c);
  const long nt = 64L * NW;
  return a.conv_c >= 24 && (chunks + nt - 1) / nt * nt * 8 <= conv_window_halves(BM, BN, (int)AS);
}

template <int EPI, int SP>
static bool launch_conv_window(const GemmArgs& a0, hipStream_t s, hipError_t& e) {
  GemmArgs a = a0;
  a.conv_magic = (uint32_t)(((uint64_t(1) << 32) + (uint64_t)a.conv_c - 1) / (uint64_t)a.conv_c);
  if ((uint64_t)a.K * (uint64_t)a.conv_c >= (uint64_t(1) << 32)) return false;
  if (a.N == 96) {
    if (tile_count(a, 128, 96) >= 256 && conv_window_fits<128, 96, 4, SP>(a)) {
      e = launch_tile<128, 96, 64, 3, A_CONVW, EPI, 4, 1, 1, SP>(a, s);
      return true;
    }
    if (conv_window_fits<64, 96, 4, SP>(a)) {
      e = launch_tile<64, 96, 64, 3, A_CONVW, EPI, 4, 1, 1, SP>(a, s);
      return true;
    }
  } else if (a.N == 192) {
    if constexpr (SP <= 1) {  // (a split W would not leave the window room)
      if (conv_window_fits<64, 192, 8, SP>(a)) {
        e = launch_tile<64, 192, 64, 2, A_CONVW, EPI, 4, 2, 1, SP>(a, s);
        return true;
      }
    }
  } else if (a.N == 64) {
    if (tile_count(a, 128, 64) >= 256 && conv_window_fits<128, 64, 4, SP>(a)) {
      e = launch_tile<128, 64, 64, 3, A_CONVW, EPI, 4, 1, 1, SP>(a, s);
      return true;
    }
    if (conv_window_fits<64, 64, 4, SP>(a)) {
      e = launch_tile<64, 64, 64, 3, A_CONVW, EPI, 2, 2, 1, SP>(a, s);
      return true;
    }
  } else if (a.N == 32 && conv_window_fits<64, 32, 4, SP>(a)) {
    e = launch_tile<64, 32, 64, 3, A_CONVW, EPI, 4, 1, 1, SP>(a, s);
    return true;
  }
  return false;
}

template <int AM, int EPI, int SP>
static hipError_t launch_split(const GemmArgs& a, hipStream_t s) {
  if constexpr (AM == A_CONVP) {
    if constexpr (SP >= 1 && (EPI == EPI_F32 || EPI == EPI_RESAVG)) {
      hipError_t e;
      if (a.conv_window && a.M == a.T && a.row_nb == 0 && launch_conv_window<EPI, SP>(a, s, e)) return e;
    }
    if constexpr (SP == 1) {
      if (a.N % 128 == 0 && a.row_nb == 0) {
        const long t128 = tile_count(a, 128, 128), t192 = tile_count(a, 192, 128);
        const long r128 = (t128 + 255) / 256, r192 = (t192 + 255) / 256;
        const int stages = a.K / 64;
        if (t192 >= 128 && r192 < r128 && a.K <= 2688 && stages % 2 == 0)
          return launch_tile<192, 128, 64, 2, AM, EPI, 4, 2, 1, SP, 1>(a, s);
        if (t128 >= 128 && stages % 3 == 0) return launch_tile<128, 128, 64, 3, AM, EPI, 4, 2, 1, SP, 1>(a, s);
      }
      if (a.N == 192 && a.row_nb == 0 && tile_count(a, 64, 192) >= 128 && (a.K / 64) % 3 == 0)
        return launch_tile<64, 192, 64, 3, AM, EPI, 4, 2, 1, SP, 1>(a, s);
      if (a.N == 96) {
        if (tile_count(a, 128, 96) >= 256) return launch_tile<128, 96, 64, 3, AM, EPI, 4, 1, 1, SP>(a, s);
        return launch_tile<64, 96, 64, 3, AM, EPI, 4, 1, 1, SP>(a, s);
      }
    }
    if (a.N % 128 == 0) return launch_tile<64, 128, 64, 3, AM, EPI, 2, 4, 1, SP>(a, s);
    if (a.N % 64 == 0) return launch_tile<64, 64, 64, 3, AM, EPI, 2, 2, 1, SP>(a, s);
    if (a.N % 32 == 0) return launch_tile<64, 32, 64, 3, AM, EPI, 4, 1, 1, SP>(a, s);
    return hipErrorInvalidValue;
  } else {
    // The condition producer's products (M = a few hundred rows): 32-row
    // tiles when 64 x 64 leaves most CUs idle.  Its k=3 convs at 602 rows
    // (N = 512, K = 1536, both operands split): 9.8 vs 13.7 us per launch.
    if (few_tiles(a, 64, 64)) return launch_tile<32, 64, 64, 3, AM, EPI, 2, 2, 1, SP>(a, s);
    return launch_tile<64, 64, 64, 3, AM, EPI, 2, 2, 1, SP>(a, s);
  }
}

template <int AM, int EPI>
static hipError_t launch_am_epi(const GemmArgs& a, hipStream_t s) {
  if constexpr (AM == A_CONVP) {
    // The vocoder's convs: M is long (thousands to hundreds of thousands of
    // samples), N is the channel count (zero-padded to the tile width).
    if constexpr (EPI == EPI_F32 || EPI == EPI_RESAVG) {
      hipError_t e;
      if (a.conv_window && a.M == a.T && a.row_nb == 0 && launch_conv_window<EPI, 0>(a, s, e)) return e;
    }
    if (a.N % 128 == 0) return launch_tile<64, 128, 64, 3, AM, EPI, 2, 4>(a, s);
    if (a.N % 64 == 0) return launch_tile<64, 64, 64, 3, AM, EPI, 2, 2>(a, s);
    if (a.N % 32 == 0) return launch_tile<64, 32, 64, 3, AM, EPI, 4, 1>(a, s);
    return hipErrorInvalidValue;
  }
  if constexpr (EPI == EPI_SWIGLU) {
    if (a.N % 192 == 0) {
      if (few_tiles(a, 128, 192) && a.N % 128 == 0) return launch_tile<32, 128, 64, 3, AM, EPI, 2, 2>(a, s);
      return launch_tile<128, 192, 64, 3, AM, EPI, 4, 2>(a, s);
    }
  }
  if constexpr (AM == A_CONV5) {
    // Two K groups (16 wavefronts, the partial tile reduced through the idle
    // ring): 17.1 vs 18.3 us.
    if (a.N % 128 == 0) {
      const long t192 = tile_count(a, 192, 128), t128 = tile_count(a, 128, 128);
      if (t192 >= 256 && pipe_fits<2, 4>(a)) {
        if (pipe_cost(t128, 128, 128, 0.302) < pipe_cost(t192, 192, 128, 0.324))
          return launch_tile<128, 128, 64, 4, AM, EPI, 2, 4, 2, 0, 1>(a, s);
        return launch_tile<192, 128, 64, 4, AM, EPI, 4, 2, 2, 0, 1>(a, s);
      }
      if (few_tiles(a, 64, 128)) return launch_tile<32, 64, 64, 3, AM, EPI, 2, 2, 2>(a, s);
      return launch_tile<64, 128, 64, 3, AM, EPI, 2, 4, 2>(a, s);
    }
  }
  if constexpr (EPI == EPI_QKV) {
    // Long sequences: the row-resident loop once there are four or more
    // items per workgroup (M = 21,568: 61.1-64.1 vs 74.2-77.1 us for 64 x 128
    // tiles, 84.8 for 64 x 64; M = 6,000: 22.8 vs 24.4; slower at M = 2,000,
    // 11.4 vs 10.4).  The same bits as the 64 x 64 tile.
    if (AM == A_PLAIN && a.K == 512 && a.N == 1536 && tile_count(a, 64, 128) >= 1024) {
      const TileMap tm = make_tile_map(a, a.M, a.N, a.K, a.K, 64, 128);
      hipLaunchKernelGGL(qkv_rows_kernel, dim3(kQkvRowsGrid), dim3(512), 0, s, a, tm);
      return hipGetLastError();
    }
  }
  if constexpr (EPI == EPI_RESSKIP || EPI == EPI_DUAL) {
    if (a.N % 128 == 0) {
      if (few_tiles(a, 64, 128)) return launch_tile<32, 64, 64, 3, AM, EPI, 2, 2>(a, s);
      return launch_tile<64, 128, 64, 3, AM, EPI, 2, 4>(a, s);
    }
  }
  if constexpr (EPI == EPI_F32) {
    // Long-K N = 512 products (w2 K = 1536, skip-in K = 1024) split K over
    // two wave groups: 9.4 vs 9.8 us and 7.25 vs 7.7 us.
    if (a.K >= 1024 && (a.K / 64) % 2 == 0) {
      if (a.N % 128 == 0 && pipe_fits<2, 4>(a)) {
        const long t192 = tile_count(a, 192, 128), t128 = tile_count(a, 128, 128);
        if (t192 >= 256 && pipe_cost(t192, 192, 128, 0.292) <= pipe_cost(t128, 128, 128, 0.257))
          return launch_tile<192, 128, 64, 4, AM, EPI, 4, 2, 2, 0, 1>(a, s);
        if (t128 >= 160) return launch_tile<128, 128, 64, 4, AM, EPI, 2, 4, 2, 0, 1>(a, s);
      }
      if (few_tiles(a, 64, 64)) return launch_tile<32, 64, 64, 3, AM, EPI, 2, 2, 2>(a, s);
      return launch_tile<64, 64, 64, 3, AM, EPI, 2, 2, 2>(a, s);
    }
  }
  if (few_tiles(a, 64, 64)) return launch_tile<32, 64, 64, 3, AM, EPI, 2, 2>(a, s);
  return launch_tile<64, 64, 64, 3, AM, EPI>(a, s);
}

// Every operand gemm_kernel reads through a buffer resource spans less than
// 2^31 bytes (buffer offsets are 32-bit).  The A_CONVP operand is read with
// global addresses instead, formed from a 32-bit element offset within each
// half of the pair: its M x lda halves stay below 2^31.
static bool gemm_spans_fit(const GemmArgs& a, AMode am) {
  constexpr size_t kMax = size_t(1) << 31;
  if (a.N <= 0 || a.M <= 0 || a.K <= 0 || a.ldw < 0 || a.lda < 0 || a.lda2 < 0) return false;
  const size_t w = ((size_t)(a.N - 1) * a.ldw + a.K + a.w_lo) * 2;
  const size_t rows = am == A_CONV3Z ? (size_t)a.M + 1 : (size_t)a.M;
  const size_t aa = am == A_CONVP || am == A_CONVW ? (size_t)a.M * a.lda : (rows * a.lda + a.a_lo) * 2;
  const size_t a2 = am == A_CONCAT ? ((size_t)a.M * a.lda2 + a.a_lo) * 2 : 0;
  return w < kMax && aa < kMax && a2 < kMax;
}

hipError_t launch_gemm(const GemmArgs& a, AMode amode, EpiMode epi, hipStream_t stream) {
  if (!gemm_spans_fit(a, amode)) return hipErrorInvalidValue;
  if (a.row_nb != 0) {
    if (a.row_nb < 0 || a.row_nb > kMaxRowSeq || a.row_T <= 0 || (long)a.row_nb * a.row_T != a.M)
      return hipErrorInvalidValue;
    for (int b = 0; b < a.row_nb; ++b)
      if (a.row_need[b] < 1 || a.row_need[b] > a.row_T) return hipErrorInvalidValue;
  }
  // Column-pair rows: EPI_F32 only, whole 32-column groups, every column stored.
  if (a.colperm && (epi != EPI_F32 || a.N % 32 != 0 || a.n_store != 0 || a.split != 0))
    return hipErrorInvalidValue;
  if (a.split != 0 || a.c16_lo != 0) {
    // Split operands: the condition producer's and the vocoder's GEMMs.
    if (a.split < 0 || a.split > 2 || (a.split >= 1 && a.a_lo == 0) || (a.split == 2 && a.w_lo == 0) ||
        a.M <= 0 || a.N <= 0 || !a.A || !a.W || a.K <= 0 || a.K % 64 != 0)
      return hipErrorInvalidValue;
    if (a.c16_lo != 0 && epi != EPI_F16 && epi != EPI_RESAVG) return hipErrorInvalidValue;
    if (amode == A_CONVP) {
      if (a.N % 32 != 0 || a.T <= 0 || a.M % a.T != 0 || a.conv_c <= 0 || a.conv_c % 8 != 0 ||
          a.lda < a.conv_c || a.conv_k <= 0 || a.conv_d <= 0 || a.conv_pad < 0 ||
          a.K < a.conv_k * a.conv_c || a.conv_inv_c != 1.0f / (float)a.conv_c || !a.A_zero ||
          a.n_store < 0 || a.n_store > a.N || a.n_store % 4 != 0)
        return hipErrorInvalidValue;
    } else {
      if (a.n_store != 0 || a.N % 64 != 0 || a.K % 128 != 0) return hipErrorInvalidValue;
      if (amode == A_CONV3Z && (a.T <= 0 || a.M % a.T != 0 || a.conv_c != kConvC || a.K != 3 * kConvC))
        return hipErrorInvalidValue;
    }
#define MIT2_SPLIT(AMV, EPV)                                                      \
  if (amode == AMV && epi == EPV) {                                               \
    if (a.split == 2) return launch_split<AMV, EPV, 2>(a, stream);                \
    if (a.split == 1) return launch_split<AMV, EPV, 1>(a, stream);                \
    return launch_split<AMV, EPV, 0>(a, stream);                                  \
  }
    MIT2_SPLIT(A_PLAIN, EPI_F16)
    MIT2_SPLIT(A_PLAIN, EPI_F32)
    MIT2_SPLIT(A_CONV3Z, EPI_F32)
    MIT2_SPLIT(A_CONVP, EPI_F32)
    MIT2_SPLIT(A_CONVP, EPI_F16)
    if (a.C32b) MIT2_SPLIT(A_CONVP, EPI_RESAVG)
#undef MIT2_SPLIT
    return hipErrorInvalidValue;
  }
  if (amode == A_CONVP) {
    if (a.M <= 0 || a.N <= 0 || a.N % 32 != 0 || a.K <= 0 || a.K % 64 != 0 || !a.A || !a.W ||
        a.T <= 0 || a.M % a.T != 0 || a.conv_c <= 0 || a.conv_c % 8 != 0 || a.lda < a.conv_c ||
        a.conv_k <= 0 || a.conv_d <= 0 || a.conv_pad < 0 || a.K < a.conv_k * a.conv_c ||
        a.conv_inv_c != 1.0f / (float)a.conv_c || !a.A_zero || a.n_store < 0 || a.n_store > a.N ||
        a.n_store % 4 != 0)
      return hipErrorInvalidValue;
    if (epi == EPI_F32) return launch_am_epi<A_CONVP, EPI_F32>(a, stream);
    if (epi == EPI_F16) return launch_am_epi<A_CONVP, EPI_F16>(a, stream);
    if (epi == EPI_RESAVG && a.C32b) return launch_am_epi<A_CONVP, EPI_RESAVG>(a, stream);
    return hipErrorInvalidValue;
  }
  if (a.n_store != 0 || epi == EPI_RESAVG) return hipErrorInvalidValue;
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.K % 128 != 0 || a.N % 64 != 0 || !a.A || !a.W)
    return hipErrorInvalidValue;
  if (amode == A_CONCAT && (a.K1 % 128 != 0 || a.K1 <= 0 || a.K1 >= a.K || !a.A2))
    return hipErrorInvalidValue;
  if (amode == A_CONV5 && (a.T <= 0 || a.conv_c != kConvC || a.K != 5 * kConvC))
    return hipErrorInvalidValue;
  if (amode == A_CONV3Z && (a.T <= 0 || a.M % a.T != 0 || a.conv_c != kConvC || a.K != 3 * kConvC))
    return hipErrorInvalidValue;
  if (amode == A_PLAIN) {
    switch (epi) {
      case EPI_F32: return launch_am_epi<A_PLAIN, EPI_F32>(a, stream);
      case EPI_F16: return launch_am_epi<A_PLAIN, EPI_F16>(a, stream);
      case EPI_SWIGLU: return launch_am_epi<A_PLAIN, EPI_SWIGLU>(a, stream);
      case EPI_QKV: return launch_am_epi<A_PLAIN, EPI_QKV>(a, stream);
      case EPI_RESSKIP: return launch_am_epi<A_PLAIN, EPI_RESSKIP>(a, stream);
      case EPI_FINALSKIP: return launch_am_epi<A_PLAIN, EPI_FINALSKIP>(a, stream);
      case EPI_DUAL: return launch_am_epi<A_PLAIN, EPI_DUAL>(a, stream);
      default: break;
    }
  } else if (amode == A_CONCAT) {
    if (epi == EPI_F32) return launch_am_epi<A_CONCAT, EPI_F32>(a, stream);
    if (epi == EPI_F16) return launch_am_epi<A_CONCAT, EPI_F16>(a, stream);
    if (epi == EPI_DUAL) return launch_am_epi<A_CONCAT, EPI_DUAL>(a, stream);
  } else if (amode == A_CONV5) {
    if (epi == EPI_GATE) return launch_am_epi<A_CONV5, EPI_GATE>(a, stream);
  } else if (amode == A_CONV3Z) {
    if (epi == EPI_F32) return launch_am_epi<A_CONV3Z, EPI_F32>(a, stream);
  }
  return hipErrorInvalidValue;  // combination not built
}

}  // namespace mit2hip
