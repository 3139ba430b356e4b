// gemm.h -- f16 MFMA GEMM with fused epilogues for the DiT-CFM decoder.
//
// C[M, N] = A[M, K] . W[N, K]^T, fp32 accumulation.  W is a resident f16
// weight whose rows may be permuted at upload so that an epilogue finds the
// two operands it combines (SwiGLU halves, WaveNet gate halves, RoPE pairs)
// in the same lane.  K must be a multiple of 128 and N a multiple of the tile
// width (weights are zero-padded at upload where the model's K is not).
#pragma once

#include "device_common.h"

namespace mit2hip {

// Channels per tap of the k=5 WaveNet conv (the model's hidden width).
constexpr int kConvC = 512;


enum AMode : int {
  A_PLAIN = 0,   // A[m][k] = A[m*lda + k]
  A_CONCAT = 1,  // k <  K1: A[m*lda + k];  k >= K1: A2[m*lda2 + k - K1]
  A_CONV5 = 2,   // k = tap*kConvC + c: A[(b*T + reflect(t + tap - 2))*lda + c], m = b*T + t
  A_CONV3Z = 3,  // k = tap*kConvC + c: A[(b*T + t + tap - 1)*lda + c], zero outside [0, T):
                 // A holds M + 1 rows and row M is all zero (the padding taps read it)
  A_CONVP = 4,   // any zero-padded conv, k = tap*conv_c + c (conv_c a multiple of 8, K padded
                 // to the stage width): A[(b*T + t + tap*conv_d - conv_pad)*lda + c], zero
                 // (read from A_zero) outside [0, T) and for tap >= conv_k
  A_CONVW = 5,   // internal: an A_CONVP product of one sequence (M = T) whose row block's
                 // input window sits in LDS (see conv_window_halves); launch_gemm picks it
                 // for A_CONVP when the window fits and conv_window is set
};

// A_CONVW: LDS halves of a BM-row block's input window.  The window holds
// rows m0 - conv_pad .. m0 + BM - 1 + (conv_k - 1) conv_d - conv_pad of the
// operand, each padded to conv_window_chunks(conv_c) 16-byte chunks (the
// extra ones zero: the padded K positions read them), for each half of a
// split pair.  Sized for BM + 50 rows of BN + 8 halves (the vocoder's convs
// have conv_c <= N and (conv_k - 1) conv_d <= 50), rounded to whole 512-lane
// fill rounds.
constexpr int conv_window_halves(int bm, int bn, int copies) {
  return (copies * (bm + 50) * (bn + 8) + 4095) / 4096 * 4096;
}
// 16-byte chunks per window row: conv_c / 8 data chunks and at least one zero
// chunk, an odd count (a row stride of an odd number of 16-byte chunks puts
// the 16 rows a fragment read spans in distinct LDS banks).
constexpr int conv_window_chunks(int conv_c) { return conv_c / 8 + 1 + ((conv_c / 8) & 1); }

enum EpiMode : int {
  EPI_F32 = 0,        // C32 = acc + bias + res (bias/res optional; C32 may be null when
                      // another output is set); optional f16 copy C16, optional
                      // normalised-operand outputs (C16s, ssq_out; see below)
  EPI_F16 = 1,        // C16 = acc + bias
  EPI_SWIGLU = 2,     // W rows interleaved [w1 x16 | w3 x16]: C16[m][c] = silu(h1) * h3
  EPI_GATE = 3,       // W rows interleaved [a x16 | b x16]: C16 = tanh(a+ca) * sigmoid(b+cb)
  EPI_QKV = 4,        // W rows paired for RoPE: write Q (rotated, x log2(e)/8), K (rotated), V^T
  EPI_RESSKIP = 5,    // WaveNet res/skip update (N = 2*512)
  EPI_FINALSKIP = 6,  // last WaveNet layer (N = 512), plus the res_projection add
  EPI_DUAL = 7,       // cols < N/2 -> C32 (+ f16 copy C16); cols >= N/2 -> C32b
  EPI_RESAVG = 8,     // v = acc + bias + res; C32 = v (optional); g = (flag ? C32b : 0) + v / 3
                      // -> C32b, and its f16 copy -> C16 (optional)
};

struct GemmArgs {
  int M = 0, N = 0, K = 0;
  // A operand
  const half_t* A = nullptr;
  int lda = 0;
  const half_t* A2 = nullptr;
  int lda2 = 0;
  int K1 = 0;
  int T = 0;        // tokens per branch (A_CONV5, EPI_QKV)
  int conv_c = 0;   // input channels per tap (A_CONV5, A_CONV3Z, A_CONVP)
  int conv_k = 0;   // A_CONVP: taps, dilation, left zero padding, 1 / conv_c
  int conv_d = 1;
  int conv_pad = 0;
  float conv_inv_c = 0.f;
  int n_store = 0;  // if nonzero: only columns < n_store are stored (weights zero-padded to N)
  const half_t* A_zero = nullptr;  // A_CONVP: >= conv_c zero halves, read by the padding taps
  int conv_window = 1;             // A_CONVP with M = T: 0 streams every tap's rows (no A_CONVW)
  uint32_t conv_magic = 0;         // A_CONVW, set by launch_gemm: ceil(2^32 / conv_c), so that
                                   // k / conv_c = umulhi(k, conv_magic) for k conv_c < 2^32
  // weights
  const half_t* W = nullptr;
  int ldw = 0;
  // epilogue
  const float* bias = nullptr;
  const float* res = nullptr;
  int ldres = 0;
  float* C32 = nullptr;
  int ldc32 = 0;
  half_t* C16 = nullptr;
  int ldc16 = 0;
  float* C32b = nullptr;
  int ldc32b = 0;
  const float* cond = nullptr;       // EPI_GATE: [a(512) | b(512)] global conditioning
  const uint32_t* mask = nullptr;    // per-row 0/1 (WaveNet epilogues)
  const float* rp = nullptr;         // EPI_FINALSKIP: res_projection [M][512]
  const float2* rope = nullptr;      // EPI_QKV: [T][32] (cos, sin)
  half_t* q = nullptr;               // EPI_QKV: [B][H][Tpad][64]
  half_t* k = nullptr;               // EPI_QKV: [B][H][Tpad][64]
  half_t* vt = nullptr;              // EPI_QKV: [B][H][64][Tpad]
  int Tpad = 0;
  int flag = 0;                      // EPI_RESSKIP: 0 -> skip accumulator starts at zero

  // AdaRMSNorm folded into a producer / consumer GEMM pair.  For the norm
  // y = aw*(x*rs*gamma) + ab, rs = 1/sqrt(mean(x^2) + 1e-5) of each row, the
  // consumer's product with W is rs * ((x*aw*gamma) . W^T) + ab . W^T, so:
  //  * the producer (EPI_F32, N = 512) also writes C16s = f16(v * sc_a * sc_g)
  //    (sc_a = aw, sc_g = gamma, per column) and, into ssq_out[m][N/32], the
  //    row's sum of squares over each 32-column block of v;
  //  * the consumer (EPI_SWIGLU, EPI_QKV) reads those partials (ssq_in, 16
  //    per row, K = 512), scales its accumulator by rs and adds bias, which
  //    holds ab . W^T for that step.
  half_t* C16s = nullptr;
  int ldc16s = 0;
  const float* sc_a = nullptr;
  const float* sc_g = nullptr;
  float* ssq_out = nullptr;
  const float* ssq_in = nullptr;
  // EPI_F32: per-row sums of each 32-column block of the output (layout of
  // ssq_out), for a norm whose statistics span whole rows or the whole tensor.
  float* sum_out = nullptr;

  // Split operands: fp32 arithmetic from f16 matrix cores.  A value v is
  // held as the pair hi = f16(v), lo = f16((v - hi) * kSplitScale), which
  // represents v to about 2^-22 relative.  split = 1: A is a pair (its lo
  // half at A + a_lo, A2 + a_lo; A_CONV3Z's zero row too), W is exact in
  // f16; split = 2: W is a pair as well (lo at W + w_lo).  The product is
  // hi.hi + (hi_A.lo_W + lo_A.hi_W) / kSplitScale in fp32 (the lo.lo term,
  // ~2^-22 relative, is dropped).  An f16 output (EPI_F16, EPI_RESAVG's C16)
  // also writes its lo half at C16 + c16_lo when c16_lo is nonzero.
  int split = 0;
  size_t a_lo = 0;
  size_t w_lo = 0;
  size_t c16_lo = 0;

  // EPI_F32: the weight rows are stored in column-pair order.  Within each
  // 32 output columns, row 16 h + 4 g + r (h < 2, g < 4, r < 4) holds column
  // 8 g + 4 h + r, so a lane's two 16-column MFMA blocks cover 8 consecutive
  // columns and its f16 outputs (C16, C16s) are 16-byte stores.  Every
  // result is the same as with unpermuted rows.  N must be a multiple of 32.
  int colperm = 0;

  // EPI_F32 / EPI_F16 / EPI_RESAVG: when set, the product of column n is
  // multiplied by colscale[n] (N floats) before the bias is added -- a
  // weight-normed conv stored as its direction v (exact in f16) with the
  // per-output-channel g / ||v|| applied here.
  const float* colscale = nullptr;

  // Row-tile skipping (the padded multi-request decode).  When row_nb > 0
  // the M rows are row_nb sequences of row_T rows, and only the first
  // row_need[b] rows of sequence b are needed (1 <= row_need[b] <= row_T).
  // A row tile that holds none of them is not computed: its outputs keep
  // whatever they held.  Rows of a computed tile are computed as without
  // skipping, so a needed row's result does not change.
  int row_T = 0;
  int row_nb = 0;
  int row_need[kMaxRowSeq] = {};
};

// Names a padded batch's needed-row prefixes (RowSkip) in a product over
// its rows; a product over other rows is left as it is (host side).
inline void apply_rows(const RowSkip& rows, GemmArgs& g) {
  if (rows.nb <= 0 || g.M != rows.nb * rows.T) return;
  g.row_T = rows.T;
  g.row_nb = rows.nb;
  for (int b = 0; b < rows.nb; ++b) g.row_need[b] = rows.need[b];
}

// Scale of the lo half of a split operand (2^11: lo then has the magnitude
// of hi, so it stays a normal f16 wherever hi does).
constexpr float kSplitScale = 2048.0f;
constexpr float kSplitInv = 1.0f / 2048.0f;

// hi / lo halves of a split operand (host side: weight uploads).
inline void split_f16_host(float v, half_t& hi, half_t& lo) {
  hi = (half_t)v;
  lo = (half_t)((v - (float)hi) * kSplitScale);
}

// hi / lo halves of a split operand in a kernel.  v first passes through an
// empty asm statement, so both halves derive from the one rounded fp32
// value: otherwise FP contraction may rewrite the conversion feeding lo as
// a fused mixed-precision FMA from v's unrounded producer (v_fma_mix) while
// hi is converted from the rounded v, and the pair then misses v by one f16
// ulp whenever the two roundings disagree.  (Not volatile, so the statement
// does not also fix the position of the loads around it.)
__device__ inline void split_f16(float v, half_t& hi, half_t& lo) {
  __asm__("" : "+v"(v));
  hi = (half_t)v;
  lo = (half_t)((v - (float)hi) * kSplitScale);
}

// Number of per-row partial sums of squares a 512-wide producer writes.
constexpr int kSsqParts = 16;

// Picks a tile shape for (M, N) and launches; returns hipSuccess or the
// launch error.  Host-side checks reject shapes the kernels do not cover.
hipError_t launch_gemm(const GemmArgs& a, AMode amode, EpiMode epi, hipStream_t stream);

}  // namespace mit2hip
