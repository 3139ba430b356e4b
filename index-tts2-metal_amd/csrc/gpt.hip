// gpt.hip -- GPT mel-code decoder on gfx950 (see gpt.h).
//
// Replaces run_gpt_kv_greedy_metal and its prefill / cached-attention passes
// (runtime/impl/gpt.cpp:1914-2240, the "ICB greedy decode") and the Metal
// kernels they record (fused f16-weight GEMV, LayerNorm, gelu, cached
// attention, argmax).
//
// One decode step (one token) is:
//   embed      x = mel_embedding[token] + mel_pos_embedding[position]
//              (or a prefix row, while the prefix is prefilled)
//   per layer  c_attn   qkv = W_attn LN1(x) + b; q -> q buffer, k and v -> the
//                       caches at row kv (no copy: the cache IS the output;
//                       head-major [head][row][64], so a head's keys are
//                       contiguous)
//              attention  softmax(q K^T / 8) V over the kv + 1 cached rows,
//                       per head, split over chunks of GPT_ATTN_KEYS (256) keys
//              c_proj   x += W_proj att + b
//              c_fc     f = gelu_new(W_fc LN2(x) + b)
//              c_proj   x += W_mp f + b          (the last layer advances kv)
//   head       logits = W_head LN_fn(LN_f(x)) + b, argmax, token bookkeeping
//
// Every matrix-vector product is HBM-bound: each weight is read once per
// step (f16, 0.98 GB for 24 layers) and used for one multiply-add.  The GEMV
// kernel loads the input vector, then streams whole rows into registers
// (16-byte loads, a group of 32 or 64 lanes per row), computes the LayerNorm
// of the input while the rows are in flight (each lane group holds the whole
// vector and computes the statistics by itself, so no barrier or LDS is
// needed), then reduces the row dot products across the lane group.  Everything the step needs (cache length, step, token,
// stop flag) lives in a device state block, so a whole step is one replayed
// HIP graph; the host only checks the stop flag every few steps.
#include "gpt.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "device_common.h"
#include "engine.h"
#include "image_io.h"

namespace mit2hip {

#define GPT_OK(expr)                                                                      \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess)                                                                 \
      throw HipError(std::string(#expr) + " failed: " + hipGetErrorString(e_) + " (" +   \
                     __FILE__ + ":" + std::to_string(__LINE__) + ")");                    \
  } while (0)

namespace {

constexpr int kW = 1280, kQKV = 3840, kMLP = 5120, kHeads = 20, kHD = 64;
constexpr int kVocab = GptDecoder::kVocab, kPos = GptDecoder::kPositions;
constexpr int kStart = (int)GptDecoder::kStartToken, kStop = (int)GptDecoder::kStopToken;
#ifndef GPT_ATTN_KEYS
#define GPT_ATTN_KEYS 256
#endif
constexpr int kChunk = GPT_ATTN_KEYS;  // keys per attention split
static_assert(kChunk % 64 == 0 && kChunk <= 512, "a split is whole passes of 64 keys, one score per thread");
constexpr int kStepsPerCheck = 8;  // decode steps replayed between stop-flag reads
constexpr int kPrefillRows = 8;    // prefix rows per prefill chunk

// Device-side decode state.
struct GptState {
  int32_t kv;         // rows in the key/value caches
  int32_t step;       // decode steps taken
  int32_t n_pred;     // predicted tokens written
  int32_t n_in;       // input tokens written (the start token included)
  int32_t stopped;    // 1 once the stop token was predicted
  int32_t stop_step;  // step of the first stop token, else -1
  int32_t cur_token;  // the last input token
  int32_t hf;         // position rule: step s > 0 uses position s + 1
  int32_t argmax;     // argmax of the last head launch
  int32_t max_pred;   // capacity of the predicted array (inputs: + 1)
  int32_t cap;        // rows of each key/value cache
  int32_t rows;       // rows of the prefix buffer
  int32_t pend;       // prefix rows the prefill chunks cover (rows 0..pend-1)
  int32_t top_k;      // sampling (sample_kernel): top-k (0: off)
  float temperature;  //   temperature, top-p, repetition penalty
  float top_p;
  float penalty;
  int32_t n_hist;     //   repetition-history prefix tokens
  uint64_t rng;       //   splitmix64 state, advanced once per sampled step
  int32_t hist_given; //   1: the history starts with the caller's prefix (even an
                      //   empty one), 0: with the start token
  int32_t pad[11];
};
static_assert(sizeof(GptState) == 128, "GptState layout");

enum { PRO_PLAIN = 0, PRO_LN = 1, PRO_LN2 = 2 };
enum { EPI_GELU = 0, EPI_RES = 1, EPI_QKV = 2, EPI_LOGITS = 3 };

struct GemvArgs {
  const half_t* w = nullptr;  // [N][K] f16
  const float* bias = nullptr;
  int N = 0;
  const float* x = nullptr;   // input vector [K]
  const float* g1 = nullptr;  // LayerNorm of PRO_LN, the first of PRO_LN2
  const float* b1 = nullptr;
  const float* g2 = nullptr;  // the second LayerNorm of PRO_LN2
  const float* b2 = nullptr;
  float* y = nullptr;         // GELU: out; RES: residual stream (in place); LOGITS: logits
  GptState* st = nullptr;
  float* q = nullptr;         // QKV: query, key cache, value cache
  float* kc = nullptr;
  float* vc = nullptr;
  int advance = 0;            // RES: block 0 advances st->kv
  int check_stop = 1;         // skip the launch once the stop token was predicted
  float* blk_val = nullptr;   // LOGITS: per-block maxima and their rows
  int* blk_idx = nullptr;
  float* lnf_out = nullptr;   // LOGITS: block 0 writes the two LayerNorm outputs
  float* fn_out = nullptr;
};

__device__ __forceinline__ float gelu_new(float v) {
  // cpu_gelu_new (tokenizer_tests.cpp:3931-3945)
  if (v > 10.0f) return v;
  if (v < -10.0f) return 0.0f;
  return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}

// Sum over the LPR lanes of a lane group (every lane gets the sum).
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// The 8-float chunks of a 1280-vector (or any vector a lane group spans) at
// lane j's positions 8 (j + c LPR) .. +7.
template <int LPR, int CH>
__device__ __forceinline__ void load_chunks(float (&v)[CH][8], const float* src, int j) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const float4* p = reinterpret_cast<const float4*>(src + 8 * (j + c * LPR));
    const float4 lo = p[0], hi = p[1];
    v[c][0] = lo.x; v[c][1] = lo.y; v[c][2] = lo.z; v[c][3] = lo.w;
    v[c][4] = hi.x; v[c][5] = hi.y; v[c][6] = hi.z; v[c][7] = hi.w;
  }
}

// LayerNorm, in place, of the vector a lane group holds in the chunk layout,
// as cpu_layernorm (tokenizer_tests.cpp:2992-3010): two passes, eps 1e-5;
// g and b are the weight and bias at the same positions.
template <int LPR, int CH>
__device__ __forceinline__ void group_layernorm(float (&xv)[CH][8], const float (&g)[CH][8],
                                                const float (&b)[CH][8]) {
  constexpr float kInvN = 1.0f / (8 * LPR * CH);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += xv[c][e];
  const float mean = group_sum<LPR>(s) * kInvN;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = xv[c][e] - mean;
      q += d * d;
    }
  const float inv = 1.0f / sqrtf(group_sum<LPR>(q) * kInvN + 1e-5f);
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[c][e] = (xv[c][e] - mean) * inv * g[c][e] + b[c][e];
}

template <int LPR, int CH>
__device__ __forceinline__ void store_chunks(const float (&xv)[CH][8], float* out, int j) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float4* o = reinterpret_cast<float4*>(out + 8 * (j + c * LPR));
    o[0] = make_float4(xv[c][0], xv[c][1], xv[c][2], xv[c][3]);
    o[1] = make_float4(xv[c][4], xv[c][5], xv[c][6], xv[c][7]);
  }
}

// y[r] = W[r] . pro(x) + b[r], then the epilogue.  A group of LPR lanes owns a
// row; lane j of the group handles the 8-half chunks j, j + LPR, ... of it.
// Each wave works on UR * 64 / LPR rows; a block has WAVES waves.  A
// LayerNorm prologue normalises the input in registers (its length is the
// lane group's span, 8 LPR CH).
template <int K, int LPR, int WAVES, int UR, int PRO, int EPI>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvArgs a) {
  constexpr int RPW = 64 / LPR;
  constexpr int CH = K / (8 * LPR);
  constexpr int ROWS = WAVES * RPW * UR;
  static_assert(K % (8 * LPR) == 0, "K must be a multiple of 8 * LPR");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, j = lane % LPR;
  // After a stop, the rest of a replayed group of steps stores nothing (the
  // cache length stops advancing too).  The flag is requested here, beside
  // the input vector, and tested only where the results are stored, so the
  // weight rows are requested without waiting for it (the row reductions
  // between are cross-lane operations, which keep those loads above the test).
  const bool stopped = a.check_stop && a.st->stopped;
  const int rbase = blockIdx.x * ROWS + wave * RPW * UR;

  // 1. the input vector at this lane's positions 8 (j + c LPR) + e (a lane
  //    group covers the whole vector once) and the first LayerNorm's
  //    weight and bias there.  Loaded first: loads complete in order, so the
  //    LayerNorm below can then run while the weight rows are in flight.
  float xv[CH][8];
  load_chunks<LPR, CH>(xv, a.x, j);
  float gv[PRO == PRO_PLAIN ? 1 : CH][8], bv[PRO == PRO_PLAIN ? 1 : CH][8];
  if constexpr (PRO != PRO_PLAIN) {
    load_chunks<LPR, CH>(gv, a.g1, j);
    load_chunks<LPR, CH>(bv, a.b1, j);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. the weight rows (rows past N re-read row N - 1; their results are dropped)
  half8 w[UR][CH];
#pragma unroll
  for (int u = 0; u < UR; ++u) {
    const int r = min(rbase + u * RPW + sub, a.N - 1);
    const half8* src = reinterpret_cast<const half8*>(a.w + (size_t)r * K) + j;
#pragma unroll
    for (int c = 0; c < CH; ++c) w[u][c] = src[c * LPR];
  }
  __builtin_amdgcn_sched_barrier(0);

  // LayerNorm prologues (ln_1 / ln_2; ln_f then final_norm for the head).
  if constexpr (PRO != PRO_PLAIN) {
    group_layernorm<LPR, CH>(xv, gv, bv);
    if constexpr (PRO == PRO_LN2) {
      const bool out = blockIdx.x == 0 && wave == 0 && sub == 0 && a.lnf_out && !stopped;
      if (out) store_chunks<LPR, CH>(xv, a.lnf_out, j);
      load_chunks<LPR, CH>(gv, a.g2, j);
      load_chunks<LPR, CH>(bv, a.b2, j);
      group_layernorm<LPR, CH>(xv, gv, bv);
      if (out) store_chunks<LPR, CH>(xv, a.fn_out, j);
    }
  }

  // 3. dot products, reduced over the lane group
  float acc[UR];
#pragma unroll
  for (int u = 0; u < UR; ++u) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        s0 += (float)w[u][c][e] * xv[c][e];
        s1 += (float)w[u][c][e + 1] * xv[c][e + 1];
      }
    }
    acc[u] = group_sum<LPR>(s0 + s1);
  }

  // 4. epilogue (lane 0 of each group)
  float rv[UR];
#pragma unroll
  for (int u = 0; u < UR; ++u) {
    const int r = rbase + u * RPW + sub;
    rv[u] = -INFINITY;
    if (j != 0 || r >= a.N || stopped) continue;
    const float v = acc[u] + a.bias[r];
    if constexpr (EPI == EPI_GELU) {
      a.y[r] = gelu_new(v);
    } else if constexpr (EPI == EPI_RES) {
      a.y[r] = a.y[r] + v;
    } else if constexpr (EPI == EPI_QKV) {
      if (r < kW) {
        a.q[r] = v;
      } else {
        const int kv = a.st->kv;
        if (kv < a.st->cap) {
          const int c = r - (r < 2 * kW ? kW : 2 * kW);  // head c / 64, dim c % 64
          float* cache = r < 2 * kW ? a.kc : a.vc;
          cache[((size_t)(c >> 6) * a.st->cap + kv) * kHD + (c & 63)] = v;
        }
      }
    } else {
      a.y[r] = v;
      rv[u] = v;
    }
  }
  if constexpr (EPI == EPI_RES) {
    if (a.advance && blockIdx.x == 0 && threadIdx.x == 0 && !stopped) a.st->kv += 1;
  }
  if constexpr (EPI == EPI_LOGITS) {
    // argmax_row (gpt.cpp:1297-1308), first stage: each block's first
    // maximum (argmax_kernel reduces the blocks).
    __shared__ float sv[ROWS];
    __shared__ int si[ROWS];
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      if (j == 0) {
        const int lr = wave * RPW * UR + u * RPW + sub;
        sv[lr] = rv[u];
        si[lr] = rbase + u * RPW + sub;
      }
    }
    __syncthreads();
    if (threadIdx.x == 0 && !stopped) {
      float bv = sv[0];
      int bi = si[0];
      for (int i = 1; i < ROWS; ++i)
        if (sv[i] > bv) { bv = sv[i]; bi = si[i]; }
      a.blk_val[blockIdx.x] = bv;
      a.blk_idx[blockIdx.x] = bi;
    }
  }
}

// The prefill's multi-row form of gemv_kernel: y[m] = W pro(x[m]) + b for the
// rows m < mrows = min(kPrefillRows, pend - kv) of a prefix chunk (rows kv..),
// so each weight row is read once per chunk instead of once per prefix row.
// The chunk's inputs (normalised first, for the LayerNorm prologue) are
// staged in LDS; every sum runs in gemv_kernel's order (the same lane
// layout, the same two partial sums, the same group reduction and the same
// LayerNorm statistics), so a prefix row gets the same values either way.
template <int K, int LPR, int WAVES, int PRO, int EPI>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_kernel(GemvArgs a) {
  constexpr int MR = kPrefillRows;
  constexpr int RPW = 64 / LPR;
  constexpr int CH = K / (8 * LPR);
  constexpr int ROWS = WAVES * RPW;
  static_assert(K % (8 * LPR) == 0, "K must be a multiple of 8 * LPR");
  static_assert(PRO != PRO_LN2 && EPI != EPI_LOGITS, "the prefill has no head");
  static_assert(PRO == PRO_PLAIN || K == kW, "LayerNorm prologues take the 1280-wide stream");
  __shared__ float4 xs[MR][K / 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, j = lane % LPR;
  const int kv = a.st->kv;
  const int mrows = min(MR, a.st->pend - kv);
  const int r = blockIdx.x * ROWS + wave * RPW + sub;

  half8 w[CH];
  {
    const half8* src = reinterpret_cast<const half8*>(a.w + (size_t)min(r, a.N - 1) * K) + j;
#pragma unroll
    for (int c = 0; c < CH; ++c) w[c] = src[c * LPR];
  }
  __builtin_amdgcn_sched_barrier(0);

  // stage the chunk's inputs (rows past mrows are zeros)
  if constexpr (PRO == PRO_PLAIN) {
    for (int i = threadIdx.x; i < MR * (K / 4); i += WAVES * 64) {
      const int mm = i / (K / 4), k4 = i % (K / 4);
      xs[mm][k4] = mm < mrows ? reinterpret_cast<const float4*>(a.x + (size_t)mm * K)[k4]
                              : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  } else {
    // one wave per row, lanes laid out as a 32-lane group (both halves
    // compute the same values; the first half stores them)
    constexpr int CH32 = K / (8 * 32);
    const int jj = lane & 31;
    for (int mm = wave; mm < MR; mm += WAVES) {
      float v[CH32][8];
      if (mm < mrows) {
        float g[CH32][8], b[CH32][8];
        load_chunks<32, CH32>(v, a.x + (size_t)mm * K, jj);
        load_chunks<32, CH32>(g, a.g1, jj);
        load_chunks<32, CH32>(b, a.b1, jj);
        group_layernorm<32, CH32>(v, g, b);
      } else {
#pragma unroll
        for (int c = 0; c < CH32; ++c)
#pragma unroll
          for (int e = 0; e < 8; ++e) v[c][e] = 0.f;
      }
      if (lane < 32) {
#pragma unroll
        for (int c = 0; c < CH32; ++c) {
          xs[mm][2 * (jj + 32 * c)] = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
          xs[mm][2 * (jj + 32 * c) + 1] = make_float4(v[c][4], v[c][5], v[c][6], v[c][7]);
        }
      }
    }
  }
  __syncthreads();

  float wf[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) wf[c][e] = (float)w[c][e];
  // one chunk row at a time (hoisting every row's LDS reads costs registers)
#pragma unroll
  for (int mm = 0; mm < MR; ++mm) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int q4 = 2 * (j + c * LPR);
      const float4 lo = xs[mm][q4], hi = xs[mm][q4 + 1];
      s0 += wf[c][0] * lo.x; s1 += wf[c][1] * lo.y;
      s0 += wf[c][2] * lo.z; s1 += wf[c][3] * lo.w;
      s0 += wf[c][4] * hi.x; s1 += wf[c][5] * hi.y;
      s0 += wf[c][6] * hi.z; s1 += wf[c][7] * hi.w;
    }
    const float acc = group_sum<LPR>(s0 + s1);
    if (j == 0 && r < a.N && mm < mrows) {
      const float v = acc + a.bias[r];
      if constexpr (EPI == EPI_GELU) {
        a.y[(size_t)mm * a.N + r] = gelu_new(v);
      } else if constexpr (EPI == EPI_RES) {
        a.y[(size_t)mm * a.N + r] += v;
      } else {
        if (r < kW) {
          a.q[(size_t)mm * kW + r] = v;
        } else if (kv + mm < a.st->cap) {
          const int c = r - (r < 2 * kW ? kW : 2 * kW);  // head c / 64, dim c % 64
          float* cache = r < 2 * kW ? a.kc : a.vc;
          cache[((size_t)(c >> 6) * a.st->cap + kv + mm) * kHD + (c & 63)] = v;
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The do_sample path of the decode loop (run_gpt_kv_greedy_metal with
// sampling, gpt.cpp:2221-2240): apply_gpt_sampling_processors (:1618-1718) to
// the step's logits over the history (the caller's repetition_history_prefix,
// else the start token; then the predictions so far) --
// repetition penalty once per distinct token, temperature, top-k (keep the
// scores >= the k-th largest), top-p (in ascending (score, index) order drop
// the tokens whose cumulative probability stays <= 1 - top_p; the largest
// always stays) -- then sample_gpt_token_from_logits (:1720-1750): one
// splitmix64 draw u, target u * sum exp(s - max), walked in index order.
// Every float and double operation is the reference's, in its order; the
// sequential sums run in one thread.  One block.  With top-k <= 1024 the
// k-th largest score comes from a radix select and only the survivors are
// sorted; otherwise every (score, index) pair is sorted in LDS (bitonic,
// 16384 slots) -- the slow path, for settings without top-k.  The processed
// logits go to `proc`.
constexpr int kSortN = 16384;
constexpr int kSampleThreads = 1024;
constexpr int kSmallList = 1024;  // survivors listed in index order when this few

__device__ __forceinline__ bool pair_less(float av, uint32_t ai, float bv, uint32_t bi) {
  return av < bv || (av == bv && ai < bi);
}

__device__ __forceinline__ double sm64_unit(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ULL);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  z = z ^ (z >> 31);
  return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(const float* logits, GptState* st,
                                                                uint32_t* predicted, uint32_t* inputs,
                                                                float* proc, const uint32_t* hist_prefix) {
  if (st->stopped) return;
  __shared__ float sv[kSortN];
  __shared__ uint32_t si[kSortN];
  __shared__ uint32_t seen[(kVocab + 31) / 32];
  __shared__ uint32_t lidx[kSmallList];  // survivors by index (small case)
  __shared__ int s_p0;
  const int tid = threadIdx.x;
  const int N = kVocab;
  const float penalty = st->penalty, temperature = st->temperature, top_p = st->top_p;
  const int top_k = st->top_k;
  for (int i = tid; i < kSortN; i += kSampleThreads) {
    sv[i] = i < N ? logits[i] : -INFINITY;
    si[i] = (uint32_t)i;
  }
  for (int i = tid; i < (N + 31) / 32; i += kSampleThreads) seen[i] = 0u;
  __syncthreads();
  if (penalty != 1.0f) {  // each distinct history token once (the order does not matter)
    // history = hist_prefix[0..n_hist) ++ predictions (inputs[1..n_in)) when a prefix
    // is given (even an empty one), else inputs[0..n_in) (the start token, then
    // the predictions)
    const int nh = st->n_hist;
    const int h0 = st->hist_given ? 1 : 0;
    const int total = nh + st->n_in - h0;
    for (int h = tid; h < total; h += kSampleThreads) {
      const uint32_t t = h < nh ? hist_prefix[h] : inputs[h - nh + h0];
      if (t >= (uint32_t)N) continue;
      const uint32_t bit = 1u << (t & 31);
      if (atomicOr(&seen[t >> 5], bit) & bit) continue;
      sv[t] = sv[t] < 0.0f ? sv[t] * penalty : sv[t] / penalty;
    }
    __syncthreads();
  }
  if (temperature != 1.0f) {
    for (int i = tid; i < N; i += kSampleThreads) sv[i] /= temperature;
    __syncthreads();
  }
  for (int i = tid; i < N; i += kSampleThreads) proc[i] = sv[i];  // index order, filtered below
  const bool use_k = top_k > 0 && top_k < N, use_p = top_p < 1.0f;
  int p0 = kSortN - N;  // first survivor in sorted order (the pads sort first)
  bool listed_by_index = false;
  if (use_k && top_k <= kSmallList) {
    // Top-k without sorting every score: the k-th largest by a 4 x 8-bit radix
    // select on order-preserving keys, the survivors (scores >= it) listed in
    // index order by a block prefix sum, and only they sorted by (score,
    // index), into the last slots of sv / si (pad slots: kSortN - 1024 > N).
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_prefix, s_kleft, s_wsum[kSampleThreads / 64], s_m;
    auto key_of = [](float f) {
      const uint32_t u = __float_as_uint(f);
      return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    };
    if (tid == 0) { s_prefix = 0u; s_kleft = (uint32_t)top_k; }
    uint32_t mask = 0u;
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) hist[tid] = 0u;
      __syncthreads();
      const uint32_t prefix = s_prefix;
      for (int i = tid; i < N; i += kSampleThreads) {
        const uint32_t key = key_of(sv[i]);
        if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid < 64) {
        // The highest bin b whose count, with every count above it, reaches
        // kleft.  Lane l holds bins 255 - 4 l .. 252 - 4 l; an exclusive scan
        // over the lanes gives each lane the count above its bins, and the
        // first lane (from the top) that reaches kleft names b -- the bin a
        // walk from 255 down would stop at, in a few wave steps instead of up
        // to 256 dependent steps on one thread.
        const uint32_t kleft = s_kleft;
        uint32_t h4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h4[j] = hist[255 - 4 * tid - j];
        const uint32_t t4 = (h4[0] + h4[1]) + (h4[2] + h4[3]);
        uint32_t incl = t4;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const uint32_t v = __shfl_up(incl, off, kWave);
          if (tid >= off) incl += v;
        }
        uint32_t cum = incl - t4;
        int fj = -1;
        uint32_t fcum = 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (fj < 0) {
            if (cum + h4[j] >= kleft) {
              fj = j;
              fcum = cum;
            } else {
              cum += h4[j];
            }
          }
        }
        const uint64_t hit = __ballot(fj >= 0);
        if (hit != 0ull && tid == __ffsll((unsigned long long)hit) - 1) {
          s_prefix = prefix | ((uint32_t)(255 - 4 * tid - fj) << shift);
          s_kleft = kleft - fcum;
        }
      }
      mask |= 255u << shift;
      __syncthreads();
    }
    const uint32_t pk = s_prefix;
    const float pivot = __uint_as_float((pk & 0x80000000u) ? (pk & 0x7fffffffu) : ~pk);
    // survivors in index order: thread t owns indices 9 t .. 9 t + 8
    constexpr int kPer = (kVocab + kSampleThreads - 1) / kSampleThreads;
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int i = tid * kPer + e;
      cnt += (i < N && sv[i] >= pivot) ? 1 : 0;
    }
    int incl = cnt;  // inclusive scan within the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off, kWave);
      if ((tid & 63) >= off) incl += v;
    }
    if ((tid & 63) == 63) s_wsum[tid >> 6] = (uint32_t)incl;
    __syncthreads();
    int base = incl - cnt;
    for (int w2 = 0; w2 < (tid >> 6); ++w2) base += (int)s_wsum[w2];
    if (tid == kSampleThreads - 1) s_m = (uint32_t)(base + cnt);
    __syncthreads();
    const int mm = (int)s_m;
    if (mm <= kSmallList) {
      const int slot0 = kSortN - mm;
      int q = base;
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const int i = tid * kPer + e;
        if (i < N && sv[i] >= pivot) {
          lidx[q] = (uint32_t)i;
          ++q;
        }
      }
      __syncthreads();  // every sv[i] < kSortN - 1024 read before the tail is rewritten
      int S = 2;
      while (S < mm) S <<= 1;
      const int seg = kSortN - S;
      for (int t = tid; t < S; t += kSampleThreads) {
        const int j = t - (S - mm);
        if (j >= 0) { sv[seg + t] = proc[lidx[j]]; si[seg + t] = lidx[j]; }
        else { sv[seg + t] = -INFINITY; si[seg + t] = 0xffffffffu; }
      }
      __syncthreads();
      if (S <= 64) {
        // The same bitonic network in one wavefront's registers: lane i holds
        // element i; of each compared pair (i, i ^ j) the lower lane keeps the
        // smaller (ascending block) or the larger, the upper lane the other.
        if (tid < 64) {
          float v = tid < S ? sv[seg + tid] : -INFINITY;
          uint32_t id = tid < S ? si[seg + tid] : 0xffffffffu;
          for (int k = 2; k <= S; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
              const float pv = __shfl_xor(v, j, kWave);
              const uint32_t pid = (uint32_t)__shfl_xor((int)id, j, kWave);
              const bool keep_min = (tid < (tid ^ j)) == ((tid & k) == 0);
              const bool take = keep_min ? pair_less(pv, pid, v, id) : pair_less(v, id, pv, pid);
              if (take) {
                v = pv;
                id = pid;
              }
            }
          }
          if (tid < S) {
            sv[seg + tid] = v;
            si[seg + tid] = id;
          }
        }
        __syncthreads();
      } else {
        for (int k = 2; k <= S; k <<= 1) {
          for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < S; i += kSampleThreads) {
              const int ixj = i ^ j;
              if (ixj <= i) continue;
              const bool up = (i & k) == 0;
              const float a = sv[seg + i], b = sv[seg + ixj];
              const uint32_t ai = si[seg + i], bi = si[seg + ixj];
              if (pair_less(b, bi, a, ai) == up) {
                sv[seg + i] = b; sv[seg + ixj] = a;
                si[seg + i] = bi; si[seg + ixj] = ai;
              }
            }
            __syncthreads();
          }
        }
      }
      for (int i = tid; i < N; i += kSampleThreads)
        if (proc[i] < pivot) proc[i] = -INFINITY;
      p0 = slot0;
      listed_by_index = true;
      __syncthreads();
    }
  }
  if ((use_k || use_p) && !listed_by_index) {
    // ascending by (score, index)
    for (int k = 2; k <= kSortN; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < kSortN; i += kSampleThreads) {
          const int ixj = i ^ j;
          if (ixj <= i) continue;
          const bool up = (i & k) == 0;
          const float a = sv[i], b = sv[ixj];
          const uint32_t ai = si[i], bi = si[ixj];
          if (pair_less(b, bi, a, ai) == up) {
            sv[i] = b; sv[ixj] = a;
            si[i] = bi; si[ixj] = ai;
          }
        }
        __syncthreads();
      }
    }
    if (use_k) {  // keep the scores >= the k-th largest
      const float pivot = sv[kSortN - top_k];
      for (int p = tid; p < kSortN; p += kSampleThreads)
        if (sv[p] >= pivot && (p == 0 || sv[p - 1] < pivot)) s_p0 = p;
      __syncthreads();
      p0 = s_p0;
      for (int i = tid; i < N; i += kSampleThreads)
        if (proc[i] < pivot) proc[i] = -INFINITY;
      __syncthreads();
    }
  }
  const int m = kSortN - p0;  // survivors (finite), sorted positions p0 .. kSortN-1
  const bool small = m <= kSmallList;
  if (small && (use_k || use_p) && !listed_by_index) {  // the survivors' indices in index order (bitonic, m <= 1024)
    if (tid < kSmallList) lidx[tid] = tid < m ? si[p0 + tid] : 0xffffffffu;
    __syncthreads();
    for (int k = 2; k <= kSmallList; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        const int i = tid;
        const int ixj = i ^ j;
        if (i < kSmallList && ixj > i) {
          const bool up = (i & k) == 0;
          const uint32_t a = lidx[i], b = lidx[ixj];
          if ((b < a) == up) { lidx[i] = b; lidx[ixj] = a; }
        }
        __syncthreads();
      }
    }
  }
  // the largest score (sorted: the last slot; else a block-wide max)
  __shared__ float s_wmax[kSampleThreads / 64];
  float mx;
  if (use_k || use_p) {
    mx = sv[kSortN - 1];
  } else {
    float v = -INFINITY;
    for (int i = tid; i < N; i += kSampleThreads) v = fmaxf(v, proc[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    if ((tid & 63) == 0) s_wmax[tid >> 6] = v;
    __syncthreads();
    mx = s_wmax[0];
    for (int w2 = 1; w2 < kSampleThreads / 64; ++w2) mx = fmaxf(mx, s_wmax[w2]);
  }
  // small case: every survivor's exp(score - max) in parallel, by index order
  // (pl) and by sorted order (ps); the sums stay sequential (thread 0)
  __shared__ double pl[kSmallList], ps[kSmallList];
  const bool listed = small && (use_k || use_p);
  if (listed && tid < m) {
    pl[tid] = exp((double)(proc[lidx[tid]] - mx));
    ps[tid] = exp((double)(sv[p0 + tid] - mx));
  }
  __syncthreads();
  if (tid != 0) return;
  // survivors in index order: (index, its exp) -- removed ones are skipped
  auto index_walk = [&](auto&& f) {
    if (listed) {
      for (int q = 0; q < m; ++q) {
        const uint32_t i = lidx[q];
        if (proc[i] != -INFINITY) f(i, pl[q]);
      }
    } else {
      for (int i = 0; i < N; ++i) {
        const float v = proc[i];
        if (v != -INFINITY) f((uint32_t)i, exp((double)(v - mx)));
      }
    }
  };
  if (use_p) {
    double total = 0.0;
    index_walk([&](uint32_t, double pr) { total += pr; });
    const double low_tail = 1.0 - (double)top_p;
    double cumulative = 0.0;
    for (int p = p0; p < kSortN; ++p) {
      cumulative += (listed ? ps[p - p0] : exp((double)(sv[p] - mx))) / total;
      if (cumulative <= low_tail && p != kSortN - 1) proc[si[p]] = -INFINITY;
    }
  }
  double total = 0.0;
  index_walk([&](uint32_t, double pr) { total += pr; });
  uint64_t rng = st->rng;
  const double target = sm64_unit(rng) * total;
  st->rng = rng;
  double cumulative = 0.0;
  uint32_t last = 0, pick = 0xffffffffu;
  index_walk([&](uint32_t i, double pr) {
    if (pick != 0xffffffffu || pr <= 0.0) return;
    last = i;
    cumulative += pr;
    if (target < cumulative) pick = i;
  });
  const int next = (int)(pick == 0xffffffffu ? last : pick);
  st->argmax = next;
  if (st->n_pred < st->max_pred) predicted[st->n_pred] = (uint32_t)next;
  st->n_pred += 1;
  if (next == kStop) {
    st->stopped = 1;
    st->stop_step = st->step;
  } else {
    if (st->n_in < st->max_pred + 1) inputs[st->n_in] = (uint32_t)next;
    st->n_in += 1;
    st->cur_token = next;
  }
  st->step += 1;
}

// Rows kv .. kv + mrows - 1 of the prefix into the chunk buffer.
__global__ __launch_bounds__(256) void embed_rows_kernel(const GptState* st, const float* rows, float* x) {
  const int mrows = min(kPrefillRows, st->pend - st->kv);
  const float4* src = reinterpret_cast<const float4*>(rows + (size_t)st->kv * kW);
  for (int i = threadIdx.x; i < mrows * (kW / 4); i += 256) reinterpret_cast<float4*>(x)[i] = src[i];
}

// The chunk is done: its rows join the caches.
__global__ void advance_rows_kernel(GptState* st) {
  st->kv += max(0, min(kPrefillRows, st->pend - st->kv));
}

// argmax_row (gpt.cpp:1297-1308), second stage: the first maximum over the
// head blocks' maxima (ties go to the lower row), then the bookkeeping of the
// loop of run_gpt_kv_greedy_cpu (gpt.cpp:1890-1909): record the prediction,
// stop at the stop token, else append it to the inputs.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* blk_val, const int* blk_idx, int nb,
                                                      GptState* st, uint32_t* predicted, uint32_t* inputs,
                                                      int check_stop) {
  if (check_stop && st->stopped) return;
  __shared__ float wv[16];
  __shared__ int wi[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  constexpr int kPer = 4;  // up to 4096 blocks in one round trip
  float vals[kPer];
  int idxs[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int b = min(tid + 1024 * u, nb - 1);
    vals[u] = blk_val[b];
    idxs[u] = blk_idx[b];
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u)
    if (tid + 1024 * u < nb && (vals[u] > bv || (vals[u] == bv && idxs[u] < bi))) { bv = vals[u]; bi = idxs[u]; }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  if (lane == 0) { wv[wave] = bv; wi[wave] = bi; }
  __syncthreads();
  if (tid != 0) return;
  for (int w2 = 1; w2 < 16; ++w2)
    if (wv[w2] > bv || (wv[w2] == bv && wi[w2] < bi)) { bv = wv[w2]; bi = wi[w2]; }
  st->argmax = bi;
  if (st->stopped) return;
  if (st->n_pred < st->max_pred) predicted[st->n_pred] = (uint32_t)bi;
  st->n_pred += 1;
  if (bi == kStop) {
    st->stopped = 1;
    st->stop_step = st->step;
  } else {
    if (st->n_in < st->max_pred + 1) inputs[st->n_in] = (uint32_t)bi;
    st->n_in += 1;
    st->cur_token = bi;
  }
  st->step += 1;
}

// x = prefix row st->kv (mode 0), or mel_embedding[token] +
// mel_pos_embedding[position] (mode 1, build_gpt_greedy_current_cpu,
// gpt.cpp:1545-1554, with gpt_cached_generate_position, :1873-1875).
__global__ __launch_bounds__(320) void embed_kernel(const GptState* st, const float* mel_emb,
                                                     const float* pos_emb, const float* rows, int mode,
                                                     float* x) {
  const int i = threadIdx.x;  // float4 index, 320 x 4 = 1280
  if (mode == 1 && st->stopped) return;
  float4 v;
  if (mode == 0) {
    const int r = min(st->kv, st->rows - 1);
    v = reinterpret_cast<const float4*>(rows + (size_t)r * kW)[i];
  } else {
    const int tok = min(max(st->cur_token, 0), kVocab - 1);
    int pos = (st->hf && st->step > 0) ? st->step + 1 : st->step;
    pos = min(pos, kPos - 1);
    const float4 e = reinterpret_cast<const float4*>(mel_emb + (size_t)tok * kW)[i];
    const float4 p = reinterpret_cast<const float4*>(pos_emb + (size_t)pos * kW)[i];
    v = make_float4(e.x + p.x, e.y + p.y, e.z + p.z, e.w + p.w);
  }
  reinterpret_cast<float4*>(x)[i] = v;
}

// Cached attention of the current query (run_gpt_cached_attention_current_cpu,
// gpt.cpp:1147-1170, with cpu_attention_single_query, tokenizer_tests.cpp:
// 4034-4060) over the st->kv + 1 cache rows (the current row included: the
// c_attn kernel already wrote it), in two launches with no waiting between
// blocks.  attn_split_kernel: block (head h, split s, query row z) takes keys
// 256 s .. 256 s + 255 -- all of its key and value loads issued together
// (the kernel is latency-bound) -- and writes the split's max m_s, sum
// l_s = sum exp(score - m_s) and unnormalised output sum exp(score - m_s) v;
// a head with a single split writes its output directly.  attn_combine_kernel
// merges the splits: out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s with
// M = max m_s (eight splits per round trip, rescaled when M grows).  Scores: 8 lanes per key, 8 dims each; the output: 16 lanes
// per key, 4 dims each.  z is the query row of a prefill chunk (row z sees
// the keys up to its own position kv + z); a decode step has one query.
constexpr int kAttnThreads = 512;
constexpr int kPartF = 2 + kHD;  // per split: max, sum, unnormalised output

// What an attention block needs from the state: whether it has nothing to do
// (the decode stopped, row z is past the prefill chunk, or the caches have
// no rows) and row z's key count.  The four fields are read before anything
// is decided, and all of them decide, so the loads are issued together and
// their latencies overlap; tested one after another (as short-circuit tests
// with the key count read after them), each load waited for the one before.
struct AttnRow {
  bool idle;
  int keys;
};
__device__ __forceinline__ AttnRow attn_row(const GptState* st, int z, int check_stop) {
  const int kv = st->kv, stopped = st->stopped, cap = st->cap, pend = st->pend;
  const bool live = gridDim.z == 1 || z < min((int)gridDim.z, pend - kv);
  return {(check_stop && stopped) || !live || cap <= 0, min(kv + z + 1, cap)};
}

__global__ __launch_bounds__(kAttnThreads) void attn_split_kernel(const float* q, const float* kc, const float* vc,
                                                                  const GptState* st, float* part, float* out,
                                                                  int nsplit_max, int check_stop) {
  constexpr int kWaves = kAttnThreads / 64;
  constexpr int kKeysPerPass = kAttnThreads / 8, kPass = kChunk / kKeysPerPass;
  constexpr int kVKeysPerPass = kAttnThreads / 16, kVPass = kChunk / kVKeysPerPass;
  constexpr int kGroups = kAttnThreads / 16;  // output key groups
  const int h = blockIdx.x, sp = blockIdx.y, z = blockIdx.z, tid = threadIdx.x;
  const AttnRow row = attn_row(st, z, check_stop);
  if (row.idle) return;
  const int kvn = row.keys;
  const int nsplit = (kvn + kChunk - 1) / kChunk;
  if (sp >= nsplit) return;
  q += (size_t)z * kW;
  const int t0 = sp * kChunk, n = min(kChunk, kvn - t0), last = kvn - 1;
  __shared__ float sc[kChunk];
  __shared__ float4 red[kGroups][kHD / 4];
  __shared__ float wm[kWaves], wl[kWaves];
  // head-major caches: head h's rows are contiguous, [cap][64]
  const float* kh = kc + (size_t)h * st->cap * kHD;
  const float* vh = vc + (size_t)h * st->cap * kHD;
  const int g = tid >> 3, e = tid & 7;       // scores: key group, dims 8 e ..
  const int d4 = tid & 15, g16 = tid >> 4;   // output: dims 4 d4 .., key group
  const int lane = tid & 63, wave = tid >> 6;
  const float4* q4 = reinterpret_cast<const float4*>(q + h * kHD) + 2 * e;
  const float4 qa = q4[0], qb = q4[1];
  float4 ka[kPass], kb[kPass], vv[kVPass];  // past the end: re-read the last key (dropped)
#pragma unroll
  for (int it = 0; it < kPass; ++it) {
    const float4* k4 =
        reinterpret_cast<const float4*>(kh + (size_t)min(t0 + g + kKeysPerPass * it, last) * kHD) + 2 * e;
    ka[it] = k4[0];
    kb[it] = k4[1];
  }
#pragma unroll
  for (int it = 0; it < kVPass; ++it)
    vv[it] = reinterpret_cast<const float4*>(vh + (size_t)min(t0 + g16 + kVKeysPerPass * it, last) * kHD)[d4];
#pragma unroll
  for (int it = 0; it < kPass; ++it) {
    float d = ((qa.x * ka[it].x + qa.y * ka[it].y) + (qa.z * ka[it].z + qa.w * ka[it].w)) +
              ((qb.x * kb[it].x + qb.y * kb[it].y) + (qb.z * kb[it].z + qb.w * kb[it].w));
    d += __shfl_xor(d, 4, kWave);
    d += __shfl_xor(d, 2, kWave);
    d += __shfl_xor(d, 1, kWave);
    const int i = g + kKeysPerPass * it;
    if (e == 0 && i < n) sc[i] = d * 0.125f;  // 1 / sqrt(64)
  }
  __syncthreads();
  float v = tid < n ? sc[tid] : -INFINITY;  // kChunk <= kAttnThreads: one score per thread
  float m = v;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  if (lane == 0) wm[wave] = m;
  __syncthreads();
  m = wm[0];
#pragma unroll
  for (int w2 = 1; w2 < kWaves; ++w2) m = fmaxf(m, wm[w2]);
  const float p = tid < n ? expf(v - m) : 0.f;
  if (tid < kChunk) sc[tid] = p;
  const float lw = warp_sum(p);
  if (lane == 0) wl[wave] = lw;
  __syncthreads();
  float l = 0.f;
#pragma unroll
  for (int w2 = 0; w2 < kWaves; ++w2) l += wl[w2];
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int it = 0; it < kVPass; ++it) {
    const int i = g16 + kVKeysPerPass * it;
    const float pi = i < n ? sc[i] : 0.f;
    o.x += pi * vv[it].x; o.y += pi * vv[it].y; o.z += pi * vv[it].z; o.w += pi * vv[it].w;
  }
  red[g16][d4] = o;
  __syncthreads();
  if (tid < kHD) {
    float od = 0.f;
#pragma unroll
    for (int gg = 0; gg < kGroups; ++gg) od += reinterpret_cast<const float*>(&red[gg][0])[tid];
    if (nsplit == 1) {
      out[(size_t)z * kW + h * kHD + tid] = od / l;
    } else {
      float* pp = part + (((size_t)z * kHeads + h) * nsplit_max + sp) * kPartF;
      pp[2 + tid] = od;
      if (tid == 0) { pp[0] = m; pp[1] = l; }
    }
  }
}

__global__ __launch_bounds__(64) void attn_combine_kernel(const GptState* st, const float* part, float* out,
                                                          int nsplit_max, int check_stop) {
  const int h = blockIdx.x, z = blockIdx.z, d = threadIdx.x;
  const AttnRow row = attn_row(st, z, check_stop);
  if (row.idle) return;
  const int nsplit = (row.keys + kChunk - 1) / kChunk;
  if (nsplit == 1) return;  // written by the split kernel
  const float* ph = part + ((size_t)z * kHeads + h) * nsplit_max * kPartF;
  // eight splits per round trip (the loads are issued before they are used)
  float M = -INFINITY, L = 0.f, O = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += 8) {
    float mm[8], ll[8], oo[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sx = min(s0 + u, nsplit - 1);
      mm[u] = ph[(size_t)sx * kPartF];
      ll[u] = ph[(size_t)sx * kPartF + 1];
      oo[u] = ph[(size_t)sx * kPartF + 2 + d];
    }
    float Mn = M;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < nsplit) Mn = fmaxf(Mn, mm[u]);
    const float r = expf(M - Mn);  // rescale what is summed so far (0 at the start)
    L *= r;
    O *= r;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (s0 + u < nsplit) {
        const float f = expf(mm[u] - Mn);
        L += f * ll[u];
        O += f * oo[u];
      }
    }
    M = Mn;
  }
  out[(size_t)z * kW + h * kHD + d] = O / L;
}

// Launch shapes: rows per block = WAVES * (64 / LPR) * UR.
template <int K, int LPR, int WAVES, int UR, int PRO, int EPI>
void launch_gemv(const GemvArgs& a, hipStream_t s) {
  constexpr int rows = WAVES * (64 / LPR) * UR;
  const int blocks = (a.N + rows - 1) / rows;
  hipLaunchKernelGGL((gemv_kernel<K, LPR, WAVES, UR, PRO, EPI>), dim3(blocks), dim3(WAVES * 64), 0, s, a);
}
// Launch shapes (lanes per row, waves per block, rows per lane group), chosen
// by timing graph-replayed loops of each product over 24 layers' weights.
// The lanes per row fix every sum's order, so the other two change no bit.
// Two rows per lane group halve the input-vector loads per row (with the
// LayerNorm prologue the input, its weight and its bias are 30 of a lane's
// 35 loads): c_attn 5.1 -> 4.6 us, c_fc 6.9 -> 5.9 us; mlp c_proj gains from
// two-wave blocks (5.8 -> 5.1 us).
#ifndef GPT_QKV_SHAPE
#define GPT_QKV_SHAPE 32, 4, 2
#endif
#ifndef GPT_PROJ_SHAPE
#define GPT_PROJ_SHAPE 32, 2, 1
#endif
#ifndef GPT_FC_SHAPE
#define GPT_FC_SHAPE 32, 2, 2
#endif
#ifndef GPT_MP_SHAPE
#define GPT_MP_SHAPE 64, 2, 1
#endif
#ifndef GPT_HEAD_SHAPE
#define GPT_HEAD_SHAPE 32, 4, 1
#endif
template <int LPR, int WAVES, int UR>
constexpr int rows_of() { return WAVES * (64 / LPR) * UR; }
constexpr int head_blocks() { return (kVocab + rows_of<GPT_HEAD_SHAPE>() - 1) / rows_of<GPT_HEAD_SHAPE>(); }
static_assert(head_blocks() <= 4096, "argmax_kernel reduces at most 4096 block maxima");

void launch_qkv(const GemvArgs& a, hipStream_t s) { launch_gemv<kW, GPT_QKV_SHAPE, PRO_LN, EPI_QKV>(a, s); }
void launch_attn_proj(const GemvArgs& a, hipStream_t s) { launch_gemv<kW, GPT_PROJ_SHAPE, PRO_PLAIN, EPI_RES>(a, s); }
void launch_fc(const GemvArgs& a, hipStream_t s) { launch_gemv<kW, GPT_FC_SHAPE, PRO_LN, EPI_GELU>(a, s); }
void launch_mlp_proj(const GemvArgs& a, hipStream_t s) { launch_gemv<kMLP, GPT_MP_SHAPE, PRO_PLAIN, EPI_RES>(a, s); }
void launch_head(const GemvArgs& a, hipStream_t s) { launch_gemv<kW, GPT_HEAD_SHAPE, PRO_LN2, EPI_LOGITS>(a, s); }

// The prefill chunk's GEMVs (lanes per row, waves per block).
template <int K, int LPR, int WAVES, int PRO, int EPI>
void launch_rows(const GemvArgs& a, hipStream_t s) {
  constexpr int rows = WAVES * (64 / LPR);
  hipLaunchKernelGGL((gemv_rows_kernel<K, LPR, WAVES, PRO, EPI>), dim3((a.N + rows - 1) / rows), dim3(WAVES * 64), 0,
                     s, a);
}

inline size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

}  // namespace

// ---------------------------------------------------------------- weights
struct GptLayerDev {
  float *ln1_w, *ln1_b, *attn_b, *proj_b, *ln2_w, *ln2_b, *fc_b, *mp_b;
  half_t *attn_w, *proj_w, *fc_w, *mp_w;  // [out][in]
};

struct GptDecoder::Impl {
  hipStream_t s = nullptr;
  int L = 0;
  Arena wa;  // weights
  std::vector<GptLayerDev> layer;
  float *lnf_w, *lnf_b, *fn_w, *fn_b, *head_b, *mel_emb, *pos_emb;
  half_t* head_w;

  // workspace (grows)
  Arena ws;
  int cap = 0;       // key/value cache rows
  int rows_cap = 0;  // prefix rows
  int pred_cap = 0;  // predicted tokens
  GptState* st = nullptr;
  uint32_t *predicted = nullptr, *inputs = nullptr;
  float *x, *q, *att, *fc, *logits, *lnf, *fn, *blk_val, *kc, *vc, *rows;
  float *xr, *qr, *attr, *fcr;  // a prefill chunk's rows: [8][1280] x3, [8][5120]
  float* proc = nullptr;        // the sampler's processed logits [8194]
  uint32_t* hist = nullptr;     // the repetition-history prefix [kMaxHistory]
  float* part = nullptr;        // attention splits: [8 query rows][20 heads][nsplit_max][66]
  int nsplit_max = 0;

  // check_stop: the launch does nothing once the stop token was predicted
  // (decode steps; the timing hook passes 0).
  void launch_attention(const float* qv, const float* K, const float* V, float* out, int rows_z,
                        int check_stop = 1) {
    hipLaunchKernelGGL(attn_split_kernel, dim3(kHeads, nsplit_max, rows_z), dim3(kAttnThreads), 0, s, qv, K, V, st,
                       part, out, nsplit_max, check_stop);
    hipLaunchKernelGGL(attn_combine_kernel, dim3(kHeads, 1, rows_z), dim3(kHD), 0, s, st, part, out, nsplit_max,
                       check_stop);
  }
  int* blk_idx;
  GptState* host_state = nullptr;  // pinned
  // row, row + head, token + head, prefill chunk, kStepsPerCheck token steps,
  // then the sampled forms of the last two token graphs
  hipGraphExec_t graph[7] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  bool use_graph = true;  // env MIT2CFM_GRAPH=0: launch every kernel directly (for profilers)
  // The measurement hook's launch loop, captured once per (kernel, count)
  // and replayed, so that back-to-back launches are timed without the host's
  // launch rate between them.
  hipGraphExec_t prof_graph = nullptr;
  int prof_kernel = -1, prof_launches = -1;

  ~Impl() {
    drop_graphs();
    for (auto& e : ev)
      if (e) (void)hipEventDestroy(e);
    if (host_state) (void)hipHostFree(host_state);
  }
  void drop_graphs() {
    for (auto& g : graph) {
      if (g) (void)hipGraphExecDestroy(g);
      g = nullptr;
    }
    if (prof_graph) (void)hipGraphExecDestroy(prof_graph);
    prof_graph = nullptr;
    prof_kernel = prof_launches = -1;
  }

  // Every weight array with its element count, in a fixed order (the device
  // image's layout).
  template <typename F>
  void visit_weights(F&& f) {
    for (auto& w : layer) {
      f(w.ln1_w, kW); f(w.ln1_b, kW); f(w.attn_w, (size_t)kQKV * kW); f(w.attn_b, kQKV);
      f(w.proj_w, (size_t)kW * kW); f(w.proj_b, kW); f(w.ln2_w, kW); f(w.ln2_b, kW);
      f(w.fc_w, (size_t)kMLP * kW); f(w.fc_b, kMLP); f(w.mp_w, (size_t)kW * kMLP); f(w.mp_b, kW);
    }
    f(lnf_w, kW); f(lnf_b, kW); f(fn_w, kW); f(fn_b, kW);
    f(head_w, (size_t)kVocab * kW); f(head_b, kVocab);
    f(mel_emb, (size_t)kVocab * kW); f(pos_emb, (size_t)kPos * kW);
  }

  void init_host_side() {
    if (const char* g = std::getenv("MIT2CFM_GRAPH")) use_graph = std::atoi(g) != 0;
    GPT_OK(hipHostMalloc(reinterpret_cast<void**>(&host_state), sizeof(GptState), hipHostMallocDefault));
    for (auto& e : ev) GPT_OK(hipEventCreate(&e));
  }

  half_t* up_f16(const std::vector<float>& v) {
    std::vector<_Float16> h(v.size());
    for (size_t i = 0; i < v.size(); ++i) h[i] = (_Float16)v[i];
    half_t* d = static_cast<half_t*>(wa.take(h.size() * 2));
    GPT_OK(hipMemcpy(d, h.data(), h.size() * 2, hipMemcpyHostToDevice));
    return d;
  }
  // Conv1D [in][out] -> f16 [out][in] (transpose_gpt_conv1d_weight, gpt.cpp:208-216)
  half_t* up_conv1d(const std::vector<float>& v, int in, int out) {
    std::vector<_Float16> h((size_t)in * out);
    for (int i = 0; i < in; ++i) {
      const float* src = v.data() + (size_t)i * out;
      for (int o = 0; o < out; ++o) h[(size_t)o * in + i] = (_Float16)src[o];
    }
    half_t* d = static_cast<half_t*>(wa.take(h.size() * 2));
    GPT_OK(hipMemcpy(d, h.data(), h.size() * 2, hipMemcpyHostToDevice));
    return d;
  }
  float* up_f32(const std::vector<float>& v) {
    float* d = static_cast<float*>(wa.take(v.size() * 4));
    GPT_OK(hipMemcpy(d, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    return d;
  }

  // Workspace for `kv_rows` cache rows, `prefix_rows` prefix rows and
  // `steps` predicted tokens; regrows (and drops the graphs) when needed.
  void ensure(int kv_rows, int prefix_rows, int steps) {
    if (kv_rows <= cap && prefix_rows <= rows_cap && steps <= pred_cap && st) return;
    drop_graphs();
    cap = std::max(std::max(kv_rows, cap), 256);
    cap = (cap + kChunk - 1) / kChunk * kChunk;
    rows_cap = std::max(std::max(prefix_rows, rows_cap), 16);
    pred_cap = std::max(std::max(steps, pred_cap), 64);
    const size_t f = sizeof(float);
    size_t bytes = align256(sizeof(GptState)) + align256((size_t)pred_cap * 4) +
                   align256(((size_t)pred_cap + 1) * 4) + 3 * align256(kW * f) + align256(kMLP * f) +
                   align256(kVocab * f) + 2 * align256(kW * f) + align256((size_t)head_blocks() * f) +
                   align256((size_t)head_blocks() * 4) +
                   3 * align256((size_t)kPrefillRows * kW * f) + align256((size_t)kPrefillRows * kMLP * f) +
                   align256((size_t)kPrefillRows * kHeads * (cap / kChunk) * kPartF * f) + align256(kVocab * f) +
                   2 * align256((size_t)L * cap * kW * f) + align256((size_t)rows_cap * kW * f) +
                   align256((size_t)GptDecoder::kMaxHistory * 4);
    ws.reserve(bytes);
    st = static_cast<GptState*>(ws.take(sizeof(GptState)));
    predicted = static_cast<uint32_t*>(ws.take((size_t)pred_cap * 4));
    inputs = static_cast<uint32_t*>(ws.take(((size_t)pred_cap + 1) * 4));
    x = static_cast<float*>(ws.take(kW * f));
    q = static_cast<float*>(ws.take(kW * f));
    att = static_cast<float*>(ws.take(kW * f));
    fc = static_cast<float*>(ws.take(kMLP * f));
    logits = static_cast<float*>(ws.take(kVocab * f));
    lnf = static_cast<float*>(ws.take(kW * f));
    fn = static_cast<float*>(ws.take(kW * f));
    blk_val = static_cast<float*>(ws.take((size_t)head_blocks() * f));
    blk_idx = static_cast<int*>(ws.take((size_t)head_blocks() * 4));
    xr = static_cast<float*>(ws.take((size_t)kPrefillRows * kW * f));
    qr = static_cast<float*>(ws.take((size_t)kPrefillRows * kW * f));
    attr = static_cast<float*>(ws.take((size_t)kPrefillRows * kW * f));
    fcr = static_cast<float*>(ws.take((size_t)kPrefillRows * kMLP * f));
    proc = static_cast<float*>(ws.take(kVocab * f));
    hist = static_cast<uint32_t*>(ws.take((size_t)GptDecoder::kMaxHistory * 4));
    nsplit_max = cap / kChunk;
    part = static_cast<float*>(ws.take((size_t)kPrefillRows * kHeads * nsplit_max * kPartF * f));
    kc = static_cast<float*>(ws.take((size_t)L * cap * kW * f));
    vc = static_cast<float*>(ws.take((size_t)L * cap * kW * f));
    rows = static_cast<float*>(ws.take((size_t)rows_cap * kW * f));
    GPT_OK(hipStreamSynchronize(s));
  }

  GemvArgs base_args() const {
    GemvArgs a;
    a.st = st;
    return a;
  }

  // One token step: embed (mode 0: prefix row, 1: token), the layers, and the
  // head when `head` is set.
  void enqueue_step(int mode, bool head, bool sample = false) {
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(320), 0, s, st, mel_emb, pos_emb, rows, mode, x);
    for (int l = 0; l < L; ++l) {
      const GptLayerDev& w = layer[l];
      float* K = kc + (size_t)l * cap * kW;
      float* V = vc + (size_t)l * cap * kW;
      GemvArgs a = base_args();
      a.w = w.attn_w; a.bias = w.attn_b; a.N = kQKV; a.x = x; a.g1 = w.ln1_w; a.b1 = w.ln1_b;
      a.q = q; a.kc = K; a.vc = V;
      launch_qkv(a, s);
      launch_attention(q, K, V, att, 1);
      a = base_args();
      a.w = w.proj_w; a.bias = w.proj_b; a.N = kW; a.x = att; a.y = x;
      launch_attn_proj(a, s);
      a = base_args();
      a.w = w.fc_w; a.bias = w.fc_b; a.N = kMLP; a.x = x; a.g1 = w.ln2_w; a.b1 = w.ln2_b; a.y = fc;
      launch_fc(a, s);
      a = base_args();
      a.w = w.mp_w; a.bias = w.mp_b; a.N = kW; a.x = fc; a.y = x; a.advance = l == L - 1;
      launch_mlp_proj(a, s);
    }
    if (head) {
      GemvArgs a = base_args();
      a.w = head_w; a.bias = head_b; a.N = kVocab; a.x = x; a.g1 = lnf_w; a.b1 = lnf_b; a.g2 = fn_w;
      a.b2 = fn_b; a.y = logits; a.blk_val = blk_val; a.blk_idx = blk_idx; a.lnf_out = lnf; a.fn_out = fn;
      launch_head(a, s);
      if (sample)
        hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kSampleThreads), 0, s, logits, st, predicted, inputs, proc,
                           hist);
      else
        hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, blk_val, blk_idx, head_blocks(), st, predicted,
                           inputs, 1);
    }
    GPT_OK(hipGetLastError());
  }

  // One prefill chunk: up to kPrefillRows prefix rows through every layer.
  void enqueue_chunk() {
    hipLaunchKernelGGL(embed_rows_kernel, dim3(1), dim3(256), 0, s, st, rows, xr);
    for (int l = 0; l < L; ++l) {
      const GptLayerDev& w = layer[l];
      float* K = kc + (size_t)l * cap * kW;
      float* V = vc + (size_t)l * cap * kW;
      GemvArgs a = base_args();
      a.w = w.attn_w; a.bias = w.attn_b; a.N = kQKV; a.x = xr; a.g1 = w.ln1_w; a.b1 = w.ln1_b;
      a.q = qr; a.kc = K; a.vc = V;
      launch_rows<kW, 32, 4, PRO_LN, EPI_QKV>(a, s);
      launch_attention(qr, K, V, attr, kPrefillRows);
      a = base_args();
      a.w = w.proj_w; a.bias = w.proj_b; a.N = kW; a.x = attr; a.y = xr;
      launch_rows<kW, 32, 4, PRO_PLAIN, EPI_RES>(a, s);
      a = base_args();
      a.w = w.fc_w; a.bias = w.fc_b; a.N = kMLP; a.x = xr; a.g1 = w.ln2_w; a.b1 = w.ln2_b; a.y = fcr;
      launch_rows<kW, 32, 4, PRO_LN, EPI_GELU>(a, s);
      a = base_args();
      a.w = w.mp_w; a.bias = w.mp_b; a.N = kW; a.x = fcr; a.y = xr;
      launch_rows<kMLP, 64, 8, PRO_PLAIN, EPI_RES>(a, s);
    }
    hipLaunchKernelGGL(advance_rows_kernel, dim3(1), dim3(1), 0, s, st);
    GPT_OK(hipGetLastError());
  }

  // 0 row, 1 row + head, 2 token + head, 3 prefill chunk, 4 = 2 x kStepsPerCheck,
  // 5 token + head + sampler, 6 = 5 x kStepsPerCheck
  void run_step(int which) {
    auto enqueue = [&] {
      if (which == 3) {
        enqueue_chunk();
      } else if (which == 4 || which == 6) {
        for (int i = 0; i < kStepsPerCheck; ++i) enqueue_step(1, true, which == 6);
      } else if (which == 5) {
        enqueue_step(1, true, true);
      } else {
        enqueue_step(which == 2 ? 1 : 0, which != 0);
      }
    };
    if (!use_graph) {
      enqueue();
      return;
    }
    if (!graph[which]) {
      hipGraph_t g = nullptr;
      GPT_OK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
      try {
        enqueue();
      } catch (...) {
        (void)hipStreamEndCapture(s, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      GPT_OK(hipStreamEndCapture(s, &g));
      hipGraphExec_t e = nullptr;
      const hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      GPT_OK(err);
      graph[which] = e;
    }
    GPT_OK(hipGraphLaunch(graph[which], s));
  }

  // Prefix rows into the caches: chunks of kPrefillRows rows (env
  // MIT2CFM_GPT_ROW_PREFILL=1: one row at a time, through the decode
  // step's kernels -- the same values, for checking).
  void prefill(int n) {
    const char* e = std::getenv("MIT2CFM_GPT_ROW_PREFILL");
    if (e && std::atoi(e) != 0) {
      for (int i = 0; i < n; ++i) run_step(0);
    } else {
      for (int i = 0; i < n; i += kPrefillRows) run_step(3);
    }
  }

  void reset_state(int prefix_rows, int pend, bool hf, int steps, const GptDecoder::Sampling* smp = nullptr) {
    GptState h{};
    h.temperature = 1.0f;
    h.top_p = 1.0f;
    h.penalty = 1.0f;
    if (smp) {
      h.top_k = (int32_t)smp->top_k;
      h.temperature = smp->temperature;
      h.top_p = smp->top_p;
      h.penalty = smp->repetition_penalty;
      h.rng = smp->seed;
      h.n_hist = (int32_t)smp->n_history;
      h.hist_given = smp->history != nullptr ? 1 : 0;
    }
    h.kv = 0;
    h.step = 0;
    h.n_pred = 0;
    h.n_in = 1;
    h.stopped = 0;
    h.stop_step = -1;
    h.cur_token = kStart;
    h.hf = hf ? 1 : 0;
    h.argmax = -1;
    h.max_pred = pred_cap;
    h.cap = cap;
    h.rows = std::max(prefix_rows, 1);
    h.pend = pend;
    (void)steps;
    *host_state = h;
    const uint32_t start = (uint32_t)kStart;
    GPT_OK(hipMemcpyAsync(st, host_state, sizeof(GptState), hipMemcpyHostToDevice, s));
    GPT_OK(hipMemcpyAsync(inputs, &start, 4, hipMemcpyHostToDevice, s));
    if (smp && smp->n_history)
      GPT_OK(hipMemcpyAsync(hist, smp->history, (size_t)smp->n_history * 4, hipMemcpyHostToDevice, s));
    GPT_OK(hipStreamSynchronize(s));  // host_state, `start` and the history are reused below
  }
};

bool GptDecoder::present(const std::unordered_map<std::string, std::vector<float>>& t) {
  for (const auto& kv : t)
    if (kv.first.compare(0, 10, "gpt.gpt.h.") == 0) return true;
  return false;
}

GptDecoder::GptDecoder(const std::unordered_map<std::string, std::vector<float>>& t, hipStream_t stream)
    : d_(new Impl) {
  Impl& d = *d_;
  d.s = stream;
  try {
    auto get = [&](const std::string& name, size_t elems) -> const std::vector<float>& {
      auto it = t.find(name);
      if (it == t.end()) throw std::invalid_argument("missing tensor: " + name);
      if (it->second.size() != elems)
        throw std::invalid_argument("tensor " + name + " has " + std::to_string(it->second.size()) +
                                    " elements, expected " + std::to_string(elems));
      return it->second;
    };
    int L = 0;
    while (t.count("gpt.gpt.h." + std::to_string(L) + ".ln_1.weight")) ++L;
    if (L == 0) throw std::invalid_argument("GPT decoder: no layer tensors (gpt.gpt.h.0.*)");
    for (const auto& kv : t) {
      int l = -1;
      if (std::sscanf(kv.first.c_str(), "gpt.gpt.h.%d.", &l) == 1 && (l < 0 || l >= L))
        throw std::invalid_argument("GPT decoder: layer tensors must be numbered 0..L-1 (" + kv.first + ")");
    }
    d.L = L;
    const size_t per_layer = 2 * ((size_t)kQKV * kW + (size_t)kW * kW + 2 * (size_t)kMLP * kW) +
                             4 * (6 * (size_t)kW + kQKV + kMLP) + 12 * 256;
    d.wa.reserve((size_t)L * per_layer + 2 * (size_t)kVocab * kW + 4 * (size_t)(kVocab + kPos) * kW +
                 4 * ((size_t)kVocab + 4 * kW) + 16 * 256);
    d.layer.resize(L);
    for (int l = 0; l < L; ++l) {
      const std::string p = "gpt.gpt.h." + std::to_string(l) + ".";
      GptLayerDev& w = d.layer[l];
      w.ln1_w = d.up_f32(get(p + "ln_1.weight", kW));
      w.ln1_b = d.up_f32(get(p + "ln_1.bias", kW));
      w.attn_w = d.up_conv1d(get(p + "attn.c_attn.weight", (size_t)kW * kQKV), kW, kQKV);
      w.attn_b = d.up_f32(get(p + "attn.c_attn.bias", kQKV));
      w.proj_w = d.up_conv1d(get(p + "attn.c_proj.weight", (size_t)kW * kW), kW, kW);
      w.proj_b = d.up_f32(get(p + "attn.c_proj.bias", kW));
      w.ln2_w = d.up_f32(get(p + "ln_2.weight", kW));
      w.ln2_b = d.up_f32(get(p + "ln_2.bias", kW));
      w.fc_w = d.up_conv1d(get(p + "mlp.c_fc.weight", (size_t)kW * kMLP), kW, kMLP);
      w.fc_b = d.up_f32(get(p + "mlp.c_fc.bias", kMLP));
      w.mp_w = d.up_conv1d(get(p + "mlp.c_proj.weight", (size_t)kMLP * kW), kMLP, kW);
      w.mp_b = d.up_f32(get(p + "mlp.c_proj.bias", kW));
    }
    d.lnf_w = d.up_f32(get("gpt.gpt.ln_f.weight", kW));
    d.lnf_b = d.up_f32(get("gpt.gpt.ln_f.bias", kW));
    d.fn_w = d.up_f32(get("gpt.final_norm.weight", kW));
    d.fn_b = d.up_f32(get("gpt.final_norm.bias", kW));
    d.head_w = d.up_f16(get("gpt.mel_head.weight", (size_t)kVocab * kW));
    d.head_b = d.up_f32(get("gpt.mel_head.bias", kVocab));
    d.mel_emb = d.up_f32(get("gpt.mel_embedding.weight", (size_t)kVocab * kW));
    d.pos_emb = d.up_f32(get("gpt.mel_pos_embedding.emb.weight", (size_t)kPos * kW));
    d.init_host_side();
  } catch (...) {
    delete d_;
    throw;
  }
}

// Image section: u64 arena bytes, i32 layers, u64 offset per weight array
// (Impl::visit_weights order), then the arena bytes.
void GptDecoder::append_image(std::vector<uint8_t>& out) const {
  Impl& d = *d_;
  ImageWriter w{out};
  const char* base = d.wa.base();
  const size_t used = d.wa.used();
  w.put<uint64_t>(used);
  w.put<int32_t>(d.L);
  d.visit_weights([&](auto* p, size_t) { w.put<uint64_t>(arena_offset(p, base)); });
  std::vector<uint8_t> host(used);
  GPT_OK(hipMemcpy(host.data(), base, used, hipMemcpyDeviceToHost));
  w.bytes(host.data(), used);
}

GptDecoder::GptDecoder(const uint8_t* image, size_t bytes, hipStream_t stream) : d_(new Impl) {
  Impl& d = *d_;
  d.s = stream;
  try {
    ImageReader r{image, bytes};
    const uint64_t used = r.get<uint64_t>();
    const int32_t L = r.get<int32_t>();
    if (used == 0 || used > (uint64_t(64) << 30) || L < 1 || L > 64)
      throw std::runtime_error("device image: bad GPT section header");
    d.L = L;
    d.layer.resize(L);
    d.wa.reserve(used);
    d.wa.set_used(used);
    char* base = d.wa.base();
    d.visit_weights([&](auto*& p, size_t n) {
      using T = std::remove_pointer_t<std::remove_reference_t<decltype(p)>>;
      p = arena_span<T>(r.get<uint64_t>(), n, base, used);
    });
    GPT_OK(hipMemcpy(base, r.bytes(used), used, hipMemcpyHostToDevice));
    if (r.at != bytes) throw std::runtime_error("device image: trailing bytes in the GPT section");
    d.init_host_side();
  } catch (...) {
    delete d_;
    throw;
  }
}

GptDecoder::~GptDecoder() { delete d_; }

size_t GptDecoder::weight_bytes() const { return d_->wa.used(); }
int GptDecoder::layers() const { return d_->L; }

void GptDecoder::kv_greedy(const float* prefix, int prefix_tokens, int steps, bool hf, Greedy& out) {
  generate(prefix, prefix_tokens, steps, hf, nullptr, out);
}

void GptDecoder::kv_sample(const float* prefix, int prefix_tokens, int steps, bool hf, const Sampling& sampling,
                           Greedy& out) {
  // apply_gpt_sampling_processors' checks (gpt.cpp:1624-1662)
  if (!(sampling.temperature > 0.0f)) throw std::invalid_argument("gpt: sampling temperature must be positive");
  if (!(sampling.repetition_penalty > 0.0f)) throw std::invalid_argument("gpt: repetition penalty must be positive");
  if (!(sampling.top_p > 0.0f && sampling.top_p <= 1.0f)) throw std::invalid_argument("gpt: top_p must be in (0, 1]");
  if (sampling.n_history > kMaxHistory)
    throw std::invalid_argument("gpt: the repetition history prefix holds more than " + std::to_string(kMaxHistory) +
                                " tokens");
  if (sampling.n_history && !sampling.history)
    throw std::invalid_argument("gpt: history prefix must not be NULL when its count is nonzero");
  generate(prefix, prefix_tokens, steps, hf, &sampling, out);
}

void GptDecoder::generate(const float* prefix, int prefix_tokens, int steps, bool hf, const Sampling* sampling,
                          Greedy& out) {
  Impl& d = *d_;
  if (prefix_tokens < 0 || steps < 0) throw std::invalid_argument("gpt: prefix_tokens and steps must be >= 0");
  if (prefix_tokens > 0 && !prefix) throw std::invalid_argument("gpt: prefix must not be NULL");
  if (steps > 0) {
    const int last = (hf && steps - 1 > 0) ? steps : steps - 1;  // position of the last step
    if (last >= kPos)
      throw std::invalid_argument("gpt: " + std::to_string(steps) + " steps pass the " +
                                  std::to_string(kPos) + "-row mel position table");
  }
  d.ensure(prefix_tokens + steps + 1, prefix_tokens + 1, steps);
  d.reset_state(prefix_tokens, prefix_tokens, hf, steps, sampling);
  if (prefix_tokens > 0)
    GPT_OK(hipMemcpyAsync(d.rows, prefix, (size_t)prefix_tokens * kW * sizeof(float), hipMemcpyHostToDevice, d.s));
  GPT_OK(hipEventRecord(d.ev[0], d.s));
  d.prefill(prefix_tokens);
  GPT_OK(hipEventRecord(d.ev[1], d.s));
  int done = 0;
  while (done < steps) {
    const int n = std::min(kStepsPerCheck, steps - done);
    if (n == kStepsPerCheck) {
      d.run_step(sampling ? 6 : 4);  // one graph of kStepsPerCheck steps
    } else {
      for (int i = 0; i < n; ++i) d.run_step(sampling ? 5 : 2);
    }
    done += n;
    GPT_OK(hipMemcpyAsync(d.host_state, d.st, sizeof(GptState), hipMemcpyDeviceToHost, d.s));
    GPT_OK(hipStreamSynchronize(d.s));
    if (d.host_state->stopped) break;
  }
  GPT_OK(hipEventRecord(d.ev[2], d.s));
  GPT_OK(hipMemcpyAsync(d.host_state, d.st, sizeof(GptState), hipMemcpyDeviceToHost, d.s));
  GPT_OK(hipStreamSynchronize(d.s));
  const GptState h = *d.host_state;
  out.first_stop_step = h.stop_step;
  out.predicted.assign((size_t)h.n_pred, 0);
  out.input_tokens.assign((size_t)h.n_in, 0);
  out.last_logits.assign(steps > 0 ? kVocab : 0, 0.f);
  if (h.n_pred) GPT_OK(hipMemcpy(out.predicted.data(), d.predicted, (size_t)h.n_pred * 4, hipMemcpyDeviceToHost));
  GPT_OK(hipMemcpy(out.input_tokens.data(), d.inputs, (size_t)h.n_in * 4, hipMemcpyDeviceToHost));
  if (steps > 0) GPT_OK(hipMemcpy(out.last_logits.data(), d.logits, kVocab * sizeof(float), hipMemcpyDeviceToHost));
  out.last_processed_logits.assign(steps > 0 ? kVocab : 0, 0.f);
  if (steps > 0)
    GPT_OK(hipMemcpy(out.last_processed_logits.data(), sampling ? d.proc : d.logits, kVocab * sizeof(float),
                     hipMemcpyDeviceToHost));
  float ms = 0.f;
  GPT_OK(hipEventElapsedTime(&ms, d.ev[0], d.ev[1]));
  out.prefill_ms = ms;
  GPT_OK(hipEventElapsedTime(&ms, d.ev[1], d.ev[2]));
  out.decode_ms = ms;
}

uint32_t GptDecoder::cached_decode(const float* rows, int prefix_tokens, float* ln_f, float* final_norm,
                                   float* logits) {
  Impl& d = *d_;
  if (prefix_tokens < 0) throw std::invalid_argument("gpt: prefix_tokens must be >= 0");
  if (!rows) throw std::invalid_argument("gpt: rows must not be NULL");
  d.ensure(prefix_tokens + 1, prefix_tokens + 1, 1);
  d.reset_state(prefix_tokens + 1, prefix_tokens, false, 1);
  GPT_OK(hipMemcpyAsync(d.rows, rows, ((size_t)prefix_tokens + 1) * kW * sizeof(float), hipMemcpyHostToDevice, d.s));
  d.prefill(prefix_tokens);
  d.run_step(1);
  GPT_OK(hipMemcpyAsync(d.host_state, d.st, sizeof(GptState), hipMemcpyDeviceToHost, d.s));
  GPT_OK(hipStreamSynchronize(d.s));
  if (ln_f) GPT_OK(hipMemcpy(ln_f, d.lnf, kW * sizeof(float), hipMemcpyDeviceToHost));
  if (final_norm) GPT_OK(hipMemcpy(final_norm, d.fn, kW * sizeof(float), hipMemcpyDeviceToHost));
  if (logits) GPT_OK(hipMemcpy(logits, d.logits, kVocab * sizeof(float), hipMemcpyDeviceToHost));
  return (uint32_t)d.host_state->argmax;
}

const char* GptDecoder::profile_launch(int kernel, int launches, double* bytes) {
  Impl& d = *d_;
  static const char* names[6] = {"gemv c_attn 3840x1280 (LN prologue, K/V to cache)",
                                 "gemv attn c_proj 1280x1280 (+residual)",
                                 "gemv c_fc 5120x1280 (LN prologue, gelu_new)",
                                 "gemv mlp c_proj 1280x5120 (+residual)",
                                 "gemv mel_head 8194x1280 (two LNs) + argmax",
                                 "cached attention, 1024 keys x 20 heads"};
  if (kernel < 0 || kernel > 5) throw std::invalid_argument("gpt profile: kernel must be 0..5");
  constexpr int kKeys = 1024;
  d.ensure(kKeys + 1, 1, 1);
  if (launches == 0) {
    const double f16 = 2.0, f32 = 4.0;
    const double b[6] = {
        kQKV * (double)kW * f16 + (kW * 3.0 + kQKV) * f32 + kQKV * f32,
        kW * (double)kW * f16 + (kW * 3.0) * f32,
        kMLP * (double)kW * f16 + (kW * 3.0 + kMLP) * f32 + kMLP * f32,
        kW * (double)kMLP * f16 + (kMLP + kW * 3.0) * f32,
        kVocab * (double)kW * f16 + (kW * 5.0 + kVocab) * f32 + kVocab * f32,
        2.0 * kKeys * kW * f32 + 2.0 * kW * f32};
    if (bytes) *bytes = b[kernel];
    return names[kernel];
  }
  // A state with kKeys - 1 cached rows; the caches hold whatever they hold
  // (timing only).
  d.reset_state(1, 0, false, 1);
  d.host_state->kv = kKeys - 1;
  GPT_OK(hipMemcpyAsync(d.st, d.host_state, sizeof(GptState), hipMemcpyHostToDevice, d.s));
  GPT_OK(hipMemsetAsync(d.x, 0, kW * sizeof(float), d.s));
  GPT_OK(hipMemsetAsync(d.fc, 0, kMLP * sizeof(float), d.s));
  GPT_OK(hipMemsetAsync(d.att, 0, kW * sizeof(float), d.s));
  const bool graphed = d.use_graph && launches > 0;
  if (graphed && d.prof_graph && d.prof_kernel == kernel && d.prof_launches == launches) {
    GPT_OK(hipGraphLaunch(d.prof_graph, d.s));
    if (bytes) *bytes = 0;
    return names[kernel];
  }
  if (graphed) {
    if (d.prof_graph) {
      GPT_OK(hipStreamSynchronize(d.s));  // the previous loop may still be replaying
      (void)hipGraphExecDestroy(d.prof_graph);
      d.prof_graph = nullptr;
    }
    GPT_OK(hipStreamBeginCapture(d.s, hipStreamCaptureModeThreadLocal));
  }
  for (int i = 0; i < launches; ++i) {
    // cycle through the layers so that, as in a decode step, the weights are
    // not already in the caches
    const GptLayerDev& w = d.layer[i % d.L];
    GemvArgs a = d.base_args();
    a.check_stop = 0;  // time the kernels whatever the last decode left in the state
    switch (kernel) {
      case 0:
        a.w = w.attn_w; a.bias = w.attn_b; a.N = kQKV; a.x = d.x; a.g1 = w.ln1_w; a.b1 = w.ln1_b;
        a.q = d.q; a.kc = d.kc; a.vc = d.vc;
        launch_qkv(a, d.s);
        break;
      case 1:
        a.w = w.proj_w; a.bias = w.proj_b; a.N = kW; a.x = d.att; a.y = d.lnf;
        launch_attn_proj(a, d.s);
        break;
      case 2:
        a.w = w.fc_w; a.bias = w.fc_b; a.N = kMLP; a.x = d.x; a.g1 = w.ln2_w; a.b1 = w.ln2_b; a.y = d.fc;
        launch_fc(a, d.s);
        break;
      case 3:
        a.w = w.mp_w; a.bias = w.mp_b; a.N = kW; a.x = d.fc; a.y = d.lnf;
        launch_mlp_proj(a, d.s);
        break;
      case 4:
        a.w = d.head_w; a.bias = d.head_b; a.N = kVocab; a.x = d.x; a.g1 = d.lnf_w; a.b1 = d.lnf_b;
        a.g2 = d.fn_w; a.b2 = d.fn_b; a.y = d.logits; a.blk_val = d.blk_val; a.blk_idx = d.blk_idx;
        a.check_stop = 0;
        launch_head(a, d.s);
        hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, d.s, d.blk_val, d.blk_idx, head_blocks(), d.st,
                           d.predicted, d.inputs, 0);
        break;
      default:
        d.launch_attention(d.q, d.kc + (size_t)(i % d.L) * d.cap * kW, d.vc + (size_t)(i % d.L) * d.cap * kW,
                           d.att, 1, 0);
        break;
    }
  }
  if (graphed) {
    hipGraph_t g = nullptr;
    const hipError_t ce = hipStreamEndCapture(d.s, &g);
    if (ce != hipSuccess) {
      if (g) (void)hipGraphDestroy(g);
      GPT_OK(ce);
    }
    const hipError_t ie = hipGraphInstantiate(&d.prof_graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    GPT_OK(ie);
    d.prof_kernel = kernel;
    d.prof_launches = launches;
    GPT_OK(hipGraphLaunch(d.prof_graph, d.s));
  }
  GPT_OK(hipGetLastError());
  if (bytes) *bytes = 0;
  return names[kernel];
}

}  // namespace mit2hip
