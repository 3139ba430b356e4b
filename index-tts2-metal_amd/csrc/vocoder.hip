// vocoder.hip -- BigVGAN vocoder on gfx950 (see vocoder.h).
//
// Replaces run_bigvgan_vocoder_metal / _single_pass
// (runtime/impl/dit_cfm_bigvgan.cpp:4102-4223) and its kernels
// (kernels.metal:1607-1749: conv1d, transposed conv, anti-aliased activation,
// add, avg3, clamp).
//
// Differences in HOW, not WHAT:
//  * convs are implicit GEMMs on the matrix cores with fp32 accumulation;
//    weights are laid out tap-major [out][tap * in + ic].  The reference runs
//    the vocoder in fp32, so by default every activation operand is a split
//    f16 pair (hi, lo: GemmArgs::split), which gives fp32-level products.  A
//    conv whose weight norm is per output channel keeps its direction v
//    (exact in f16) and applies g / ||v|| to its outputs (GemmArgs::colscale);
//    the transposed convs, normed per input channel, keep the weight-normed
//    weight as a split pair.  An f16 mode uses the hi halves alone;
//  * a transposed conv with stride s, kernel 2s and padding s/2 is a k = 3
//    conv over the input (taps q-1, q, q+1) whose s * out output columns are
//    the s phases of the upsampled signal: output row q, column r * out + oc
//    is sample s q + r, so the GEMM writes the token-major upsampled tensor;
//  * the residual add of each AMP pair and the /3 average of the three
//    resblocks are fused into the second conv's epilogue (EPI_RESAVG), which
//    also writes the f16 operand of the next upsampler;
//  * the activation keeps the two-times-upsampled, snake'd signal of a run of
//    tokens in registers, so each upsampled value is computed once.
#include "vocoder.h"

#include <array>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

#include "engine.h"
#include "gemm.h"
#include "image_io.h"

namespace mit2hip {

#define VOC_OK(expr)                                                                      \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess)                                                                 \
      throw HipError(std::string(#expr) + " failed: " + hipGetErrorString(e_) + " (" +   \
                     __FILE__ + ":" + std::to_string(__LINE__) + ")");                    \
  } while (0)

namespace {

// kBigVGANUpsamplers (dit_cfm_bigvgan.cpp:3681-3688) and kBigVGANResblocks
// (:3960-3979).
struct UpsSpec {
  const char* prefix;
  int cin, cout, kernel, stride, padding;
};
constexpr UpsSpec kUps[6] = {{"bigvgan.ups.0.0", 1536, 768, 8, 4, 2}, {"bigvgan.ups.1.0", 768, 384, 8, 4, 2},
                             {"bigvgan.ups.2.0", 384, 192, 4, 2, 1},  {"bigvgan.ups.3.0", 192, 96, 4, 2, 1},
                             {"bigvgan.ups.4.0", 96, 48, 4, 2, 1},    {"bigvgan.ups.5.0", 48, 24, 4, 2, 1}};
constexpr int kRbKernel[3] = {3, 7, 11};
constexpr int kDil[3] = {1, 3, 5};
inline int rb_channels(int j) { return 768 >> (j / 3); }
inline int round_up(int v, int m) { return (v + m - 1) / m * m; }

// ---------------------------------------------------------------- kernels
// The two 12-tap filters of one anti-aliased activation, passed by value so
// every tap is a scalar operand.
struct ActFilters {
  float up[12];
  float down[12];
};

// Anti-aliased SnakeBeta (cpu_bigvgan_activation, tokenizer_tests.cpp:3811):
//   U(u) = 2 sum_{k: (u+15-k) even} x[clamp((u+15-k)/2 - 5)] up[k]
//   Z(u) = U + sin(alpha U)^2 / (beta + 1e-9)
//   out[t] = sum_k Z(clamp(2t + k - 5, 0, 2T-1)) down[k]
// By parity, U(2v) = 2 sum_j x[v+2-j] up[2j+1] and U(2v+1) = 2 sum_j x[v+3-j]
// up[2j] (j = 0..5).  A lane owns one channel and R consecutive tokens; its
// x window (tokens t0-6 .. t0+R+5, clamped) and the 2R+10 Z values its
// outputs need stay in registers, so each Z is computed once and nothing
// goes through LDS.  Lanes are (run, channel) pairs in channel-fastest
// order, so a wave reads whole row segments and no lane idles when C is not
// a multiple of 64 (the 24- and 48-channel stages).
constexpr int kActR = 16;

template <bool OUT16>
__global__ __launch_bounds__(256) void snake_aa_kernel(const float* __restrict__ x, ActFilters f,
                                                       const float* __restrict__ alpha,
                                                       const float* __restrict__ inv_beta, int T,
                                                       int C, void* __restrict__ out, size_t out_lo) {
  constexpr int R = kActR;
  constexpr int XW = R + 12;      // x window
  constexpr int ZW = 2 * R + 10;  // Z window: u = 2 t0 - 5 + i
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  const int run = (int)(g / C);
  const int c = (int)(g - (long)run * C);
  const int t0 = run * R;
  if (t0 >= T) return;
  // The activation is read and written through buffer resources: one 32-bit
  // byte offset per access (T x C < 2^29, checked on the host), and the
  // hardware drops the stores of rows past T.
  const buffer_rsrc_t rX = make_buffer_rsrc(x, T * C * 4);
  // Rows t0 - 6 + i, clamped to [0, T): consecutive rows are C values
  // apart, so the offsets advance by additions and the clamp applies to them.
  const int e_first = c, e_last = (T - 1) * C + c;
  float xw[XW];
  int e = (t0 - 6) * C + c;
#pragma unroll
  for (int i = 0; i < XW; ++i, e += C) xw[i] = buffer_load_f32(rX, min(max(e, e_first), e_last) * 4);
  const float a = alpha[c], ib = inv_beta[c];
  float z[ZW];
#pragma unroll
  for (int i = 0; i < ZW; ++i) {
    float acc = 0.0f;
    if (i & 1) {  // u even: x window index (i-5)/2 + 8 - j, taps up[2j+1]
#pragma unroll
      for (int j = 0; j < 6; ++j) acc += xw[(i - 5) / 2 + 8 - j] * f.up[2 * j + 1];
    } else {      // u odd: x window index (i-6)/2 + 9 - j, taps up[2j]
#pragma unroll
      for (int j = 0; j < 6; ++j) acc += xw[(i - 6) / 2 + 9 - j] * f.up[2 * j];
    }
    const float y = 2.0f * acc;
    const float sn = __sinf(y * a);
    z[i] = y + (sn * sn) * ib;
  }
  // Upsampled positions outside [0, 2T) take the value at the nearest end.
  if (t0 == 0) {
#pragma unroll
    for (int i = 0; i < 5; ++i) z[i] = z[5];
  }
  const int i_end = 2 * (T - t0) + 4;  // slot of u = 2T - 1
  if (i_end < ZW - 1) {
    float ze = z[0];
#pragma unroll
    for (int i = 0; i < ZW; ++i) ze = i == i_end ? z[i] : ze;
#pragma unroll
    for (int i = 0; i < ZW; ++i) z[i] = i > i_end ? ze : z[i];
  }
  const buffer_rsrc_t rO = make_buffer_rsrc(out, T * C * (OUT16 ? 2 : 4));
  const buffer_rsrc_t rL = make_buffer_rsrc(static_cast<half_t*>(out) + out_lo, T * C * 2);
  e = t0 * C + c;
#pragma unroll
  for (int r = 0; r < R; ++r, e += C) {
    // rows t0 + r >= T fall past the resources' ranges: their stores are dropped
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 12; ++k) acc += z[2 * r + k] * f.down[k];
    if constexpr (OUT16) {
      if (out_lo) {
        half_t h, l;
        split_f16(acc, h, l);
        buffer_store_f16(rO, e * 2, h);
        buffer_store_f16(rL, e * 2, l);
      } else {
        buffer_store_f16(rO, e * 2, (half_t)acc);
      }
    } else {
      buffer_store_f32(rO, e * 4, acc);
    }
  }
}

// conv_post (k = 7, 24 -> 1, zero bias) and the final clamp
// (run_bigvgan_post_cpu, dit_cfm_bigvgan.cpp:4030-4039).  A workgroup stages
// its 256 + 6 input rows (one contiguous block) in LDS, row stride 25 so the
// lanes' reads fall in distinct banks.
__global__ __launch_bounds__(256) void conv_post_clamp_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ w, int T,
                                                              float* __restrict__ wav) {
  constexpr int RS = 25;
  __shared__ float ws[24 * 7];
  __shared__ float as[262 * RS];
  const int t0 = blockIdx.x * 256;
  if (threadIdx.x < 24 * 7) ws[threadIdx.x] = w[threadIdx.x];
  // The block's rows through a buffer resource, every load issued before the
  // first LDS store: rows outside [0, T) fall outside its range (a negative
  // offset too, read as unsigned) and load zero, so no branch surrounds a
  // load (one per element made each wait for the one before).  The host
  // keeps T x 24 x 4 bytes below 2^31.
  const buffer_rsrc_t rA = make_buffer_rsrc(a, T * 24 * 4);
  constexpr int kN = (262 * 24 + 255) / 256;
  float v[kN];
#pragma unroll
  for (int u = 0; u < kN; ++u) {
    const int idx = threadIdx.x + u * 256;
    v[u] = buffer_load_f32(rA, ((t0 - 3) * 24 + idx) * 4);  // row t0 - 3 + idx / 24, channel idx % 24
  }
#pragma unroll
  for (int u = 0; u < kN; ++u) {
    const int idx = threadIdx.x + u * 256;
    if (idx < 262 * 24) as[(idx / 24) * RS + idx % 24] = v[u];
  }
  __syncthreads();
  const int t = t0 + threadIdx.x;
  if (t >= T) return;
  float acc = 0.0f;
  for (int ic = 0; ic < 24; ++ic) {
#pragma unroll
    for (int k = 0; k < 7; ++k) acc += as[(threadIdx.x + k) * RS + ic] * ws[ic * 7 + k];
  }
  wav[t] = fminf(1.0f, fmaxf(-1.0f, acc));
}

__global__ void voc_f32_to_f16_kernel(const float* __restrict__ in, half_t* __restrict__ out,
                                      size_t n, size_t lo_off) {
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

const std::vector<float>& get(const std::unordered_map<std::string, std::vector<float>>& t,
                              const std::string& name, size_t elems) {
  auto it = t.find(name);
  if (it == t.end()) throw std::invalid_argument("missing tensor: " + name);
  if (it->second.size() != elems)
    throw std::invalid_argument("tensor " + name + " has " + std::to_string(it->second.size()) +
                                " elements, expected " + std::to_string(elems));
  return it->second;
}

// weight_norm_rowmajor (gpt.cpp:5109): w = g * v / ||v|| per row.
std::vector<float> wnorm(const std::vector<float>& g, const std::vector<float>& v, size_t rows,
                         size_t cols) {
  std::vector<float> w(rows * cols);
  for (size_t r = 0; r < rows; ++r) {
    float n = 0.f;
    for (size_t c = 0; c < cols; ++c) n += v[r * cols + c] * v[r * cols + c];
    n = std::sqrt(n);
    const float s = g[r] / n;
    for (size_t c = 0; c < cols; ++c) w[r * cols + c] = v[r * cols + c] * s;
  }
  return w;
}

}  // namespace

// ---------------------------------------------------------------- weights
struct Vocoder::Conv {
  // [N][K] f16, tap-major, zero-padded.  Without `scale`: the weight-normed
  // weight as split pairs (hi halves, then the lo halves, [N][K] each).  With
  // `scale`: the direction v itself, exact in f16, one copy, and the product
  // of output channel n is multiplied by scale[n] = g / ||v|| in the GEMM
  // epilogue.
  half_t* w = nullptr;
  float* b = nullptr;      // [N]
  float* scale = nullptr;  // [N] or null
  int N = 0, n_out = 0, K = 0, cin = 0, k = 0;
};

struct Vocoder::Act {
  ActFilters filt;
  float* alpha = nullptr;     // exp(alpha_log) [C]
  float* inv_beta = nullptr;  // 1 / (exp(beta_log) + 1e-9) [C]
  int C = 0;
};

struct Vocoder::Impl {
  hipStream_t s;
  Arena wa;
  Conv pre, ups[6], rb[18][3][2];
  Act act[18][6], act_post;
  float* post_w = nullptr;   // [24 * 7]
  half_t* zero = nullptr;    // 2048 zero halves: the padding taps of every conv
  size_t bytes = 0;
  // workspace, sized for cap mel tokens
  Arena ws;
  int cap = 0;
  // f16 operand buffers, each a split pair: hi values, then lo values at
  // + the *_lo element offset.
  half_t *mel16, *pre16, *a16, *g16;
  size_t mel16_lo = 0, pre16_lo = 0, a16_lo = 0, g16_lo = 0;
  float *x32, *h32, *t32, *g32, *act32;
  bool f32 = true;  // split operands (fp32-level products); false: f16 operands
  // Narrow convs with their input window resident in LDS (the same bits as
  // streaming every tap's rows; MIT2CFM_CONV_WINDOW=0 at construction turns
  // it off, for comparison).
  int conv_window = 1;

  // Weights as split pairs: [n] hi halves, then [n] lo halves.
  void upload_f16(half_t*& d, const std::vector<float>& v) {
    const size_t n = v.size();
    std::vector<_Float16> h(2 * n);
    for (size_t i = 0; i < n; ++i) split_f16_host(v[i], h[i], h[n + i]);
    d = static_cast<half_t*>(wa.take(h.size() * 2));
    VOC_OK(hipMemcpy(d, h.data(), h.size() * 2, hipMemcpyHostToDevice));
  }
  void upload_f32(float*& d, const std::vector<float>& v) {
    d = static_cast<float*>(wa.take(v.size() * 4));
    VOC_OK(hipMemcpy(d, v.data(), v.size() * 4, hipMemcpyHostToDevice));
  }

  // One f16 copy of values that are exact in f16.
  void upload_exact(half_t*& d, const std::vector<float>& v) {
    std::vector<_Float16> h(v.size());
    for (size_t i = 0; i < v.size(); ++i) h[i] = (_Float16)v[i];
    d = static_cast<half_t*>(wa.take(h.size() * 2));
    VOC_OK(hipMemcpy(d, h.data(), h.size() * 2, hipMemcpyHostToDevice));
  }

  // Zero-padded conv (weight_v [out][in][k], weight_g [out]).  Weight norm is
  // per output channel, w = (g / ||v||) v, so when v is exact in f16 (the
  // checkpoint's values are) the conv keeps v and applies g / ||v|| to its
  // outputs: fp32-level products need A split only (two matrix-core
  // products per term instead of three) and the weight bytes halve.
  void make_conv(Conv& c, const std::unordered_map<std::string, std::vector<float>>& t,
                 const std::string& prefix, int cout, int cin, int k, bool bias) {
    const auto& g = get(t, prefix + ".weight_g", cout);
    const auto& v = get(t, prefix + ".weight_v", (size_t)cout * cin * k);
    bool exact = true;
    for (float x : v)
      if ((float)(_Float16)x != x) {
        exact = false;
        break;
      }
    c.n_out = cout;
    c.N = round_up(cout, 32);
    c.K = round_up(k * cin, 64);
    c.cin = cin;
    c.k = k;
    std::vector<float> wt((size_t)c.N * c.K, 0.f), bt(c.N, 0.f), st(c.N, 0.f);
    if (exact) {
      // ||v|| of each output row in the order wnorm sums it.
      for (int oc = 0; oc < cout; ++oc) {
        float n = 0.f;
        const float* vr = v.data() + (size_t)oc * cin * k;
        for (size_t i = 0; i < (size_t)cin * k; ++i) n += vr[i] * vr[i];
        st[oc] = g[oc] / std::sqrt(n);
      }
    }
    const std::vector<float> w = exact ? v : wnorm(g, v, cout, (size_t)cin * k);
    for (int oc = 0; oc < cout; ++oc)
      for (int ic = 0; ic < cin; ++ic)
        for (int tap = 0; tap < k; ++tap)
          wt[(size_t)oc * c.K + tap * cin + ic] = w[((size_t)oc * cin + ic) * k + tap];
    if (bias) {
      const auto& b = get(t, prefix + ".bias", cout);
      for (int oc = 0; oc < cout; ++oc) bt[oc] = b[oc];
    }
    if (exact) {
      upload_exact(c.w, wt);
      upload_f32(c.scale, st);
    } else {
      upload_f16(c.w, wt);
    }
    upload_f32(c.b, bt);
  }

  // Transposed conv (weight_v [in][out][kernel], weight_g [in]) as a k = 3
  // conv: output column r * cout + oc of row q is sample s q + r; input tap
  // i = q - 1 + tap contributes w[ic][oc][kk] with kk = s (1 - tap) + r + p.
  void make_ups(Conv& c, const std::unordered_map<std::string, std::vector<float>>& t, const UpsSpec& u) {
    const int s = u.stride;
    if (u.kernel != 2 * s || 2 * u.padding != s)
      throw std::invalid_argument(std::string(u.prefix) + ": upsampler must have kernel 2s and padding s/2");
    const auto w = wnorm(get(t, std::string(u.prefix) + ".weight_g", u.cin),
                         get(t, std::string(u.prefix) + ".weight_v", (size_t)u.cin * u.cout * u.kernel), u.cin,
                         (size_t)u.cout * u.kernel);
    const auto& b = get(t, std::string(u.prefix) + ".bias", u.cout);
    c.n_out = s * u.cout;
    c.N = round_up(c.n_out, 32);
    c.K = round_up(3 * u.cin, 64);
    c.cin = u.cin;
    c.k = 3;
    std::vector<float> wt((size_t)c.N * c.K, 0.f), bt(c.N, 0.f);
    for (int r = 0; r < s; ++r)
      for (int oc = 0; oc < u.cout; ++oc) {
        const int n = r * u.cout + oc;
        bt[n] = b[oc];
        for (int tap = 0; tap < 3; ++tap) {
          const int kk = s * (1 - tap) + r + u.padding;
          if (kk < 0 || kk >= u.kernel) continue;
          for (int ic = 0; ic < u.cin; ++ic)
            wt[(size_t)n * c.K + tap * u.cin + ic] = w[((size_t)ic * u.cout + oc) * u.kernel + kk];
        }
      }
    upload_f16(c.w, wt);
    upload_f32(c.b, bt);
  }

  void make_act(Act& a, const std::unordered_map<std::string, std::vector<float>>& t, const std::string& prefix,
                int C) {
    a.C = C;
    const auto& fu = get(t, prefix + ".upsample.filter", 12);
    const auto& fd = get(t, prefix + ".downsample.lowpass.filter", 12);
    for (int k = 0; k < 12; ++k) {
      a.filt.up[k] = fu[k];
      a.filt.down[k] = fd[k];
    }
    const auto& al = get(t, prefix + ".act.alpha", C);
    const auto& bl = get(t, prefix + ".act.beta", C);
    std::vector<float> alpha(C), ib(C);
    for (int c = 0; c < C; ++c) {
      alpha[c] = std::exp(al[c]);
      ib[c] = 1.0f / (std::exp(bl[c]) + 1e-9f);
    }
    upload_f32(a.alpha, alpha);
    upload_f32(a.inv_beta, ib);
  }

  void ensure(int T) {
    if (T <= cap) return;
    const size_t big = (size_t)T * 6144;  // C * T_s of every stage from the second on
    const size_t need = 2 * ((size_t)T * 80 * 2 + (size_t)T * 1536 * 2 + 2 * big * 2) + 5 * big * 4 + 9 * 256;
    VOC_OK(hipStreamSynchronize(s));
    ws.reserve(need + 4096);
    mel16_lo = (size_t)T * 80;
    pre16_lo = (size_t)T * 1536;
    a16_lo = g16_lo = big;
    mel16 = static_cast<half_t*>(ws.take(mel16_lo * 2 * 2));
    pre16 = static_cast<half_t*>(ws.take(pre16_lo * 2 * 2));
    a16 = static_cast<half_t*>(ws.take(big * 2 * 2));
    g16 = static_cast<half_t*>(ws.take(big * 2 * 2));
    x32 = static_cast<float*>(ws.take(big * 4));
    h32 = static_cast<float*>(ws.take(big * 4));
    t32 = static_cast<float*>(ws.take(big * 4));
    g32 = static_cast<float*>(ws.take(big * 4));
    act32 = static_cast<float*>(ws.take(big * 4));
    cap = T;
  }

  // ---------------------------------------------------------- launches
  // Conv of the f16 operand A (a split pair with lo at + a_lo); C16 (when
  // given) is a split pair buffer with lo at + c16_lo.
  void conv(const Conv& c, const half_t* A, size_t a_lo, int T, int d, int pad, int epi, float* C32,
            const float* res, float* C32b, half_t* C16, size_t c16_lo, int flag) {
    GemmArgs g;
    if (f32) {
      g.split = c.scale ? 1 : 2;  // A split; W split too unless it holds v exactly
      g.a_lo = a_lo;
      g.w_lo = c.scale ? 0 : (size_t)c.N * c.K;
      g.c16_lo = C16 ? c16_lo : 0;
    }
    g.colscale = c.scale;
    g.M = T;
    g.N = c.N;
    g.K = c.K;
    g.A = A;
    g.lda = c.cin;
    g.T = T;
    g.conv_c = c.cin;
    g.conv_k = c.k;
    g.conv_d = d;
    g.conv_pad = pad;
    g.conv_inv_c = 1.0f / (float)c.cin;
    g.A_zero = zero;
    g.conv_window = conv_window;
    g.W = c.w;
    g.ldw = c.K;
    g.bias = c.b;
    g.n_store = c.N == c.n_out ? 0 : c.n_out;
    g.C32 = C32;
    g.ldc32 = c.n_out;
    g.res = res;
    g.ldres = c.n_out;
    g.C32b = C32b;
    g.ldc32b = c.n_out;
    g.C16 = C16;
    g.ldc16 = c.n_out;
    g.flag = flag;
    VOC_OK(launch_gemm(g, A_CONVP, (EpiMode)epi, s));
  }

  // out16: out is a split pair buffer (lo at + out_lo, written in f32 mode).
  void activation(const Act& a, const float* in, int T, void* out, bool out16, size_t out_lo = 0) {
    // the kernel addresses the T x C activation with 32-bit byte offsets
    if ((size_t)T * (size_t)a.C >= (size_t(1) << 29)) VOC_OK(hipErrorInvalidValue);
    const size_t lanes = (size_t)((T + kActR - 1) / kActR) * a.C;
    const dim3 grid((unsigned)((lanes + 255) / 256));
    if (out16)
      hipLaunchKernelGGL(snake_aa_kernel<true>, grid, dim3(256), 0, s, in, a.filt, a.alpha, a.inv_beta,
                         T, a.C, out, f32 ? out_lo : 0);
    else
      hipLaunchKernelGGL(snake_aa_kernel<false>, grid, dim3(256), 0, s, in, a.filt, a.alpha, a.inv_beta,
                         T, a.C, out, (size_t)0);
    VOC_OK(hipGetLastError());
  }

  // One resblock j over x [T][C]: three (act, dilated conv, act, conv, + res)
  // pairs.  The last pair folds into the group mean g (flag: add to g rather
  // than start it) and, when given, writes the block output to out32 and the
  // updated mean's f16 copy to g16o.
  void resblock(int j, const float* x, int T, float* out32, float* g, int flag, half_t* g16o) {
    const int k = kRbKernel[j % 3];
    const float* h = x;
    for (int pr = 0; pr < 3; ++pr) {
      activation(act[j][2 * pr], h, T, a16, true, a16_lo);
      const int d = kDil[pr];
      conv(rb[j][pr][0], a16, a16_lo, T, d, (k - 1) * d / 2, EPI_F32, t32, nullptr, nullptr, nullptr, 0, 0);
      activation(act[j][2 * pr + 1], t32, T, a16, true, a16_lo);
      if (pr < 2) {
        conv(rb[j][pr][1], a16, a16_lo, T, 1, (k - 1) / 2, EPI_F32, h32, h, nullptr, nullptr, 0, 0);
        h = h32;
      } else {
        conv(rb[j][pr][1], a16, a16_lo, T, 1, (k - 1) / 2, EPI_RESAVG, out32, h, g, g16o, g16_lo, flag);
      }
    }
  }

  // Resblock group i over the upsampled x [T][C]: g = mean of the three
  // resblocks; g16o receives its f16 copy (the next upsampler's operand).
  void group(int i, const float* x, int T, float* g, half_t* g16o) {
    for (int r = 0; r < 3; ++r) resblock(3 * i + r, x, T, nullptr, g, r > 0, r == 2 ? g16o : nullptr);
  }

  void to_f16(const float* in, half_t* out, size_t n, size_t lo_off) {
    hipLaunchKernelGGL(voc_f32_to_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, out, n,
                       f32 ? lo_off : 0);
    VOC_OK(hipGetLastError());
  }

  void post(const float* x, int T, float* wav) {
    activation(act_post, x, T, act32, false);
    hipLaunchKernelGGL(conv_post_clamp_kernel, dim3((T + 255) / 256), dim3(256), 0, s, act32, post_w, T, wav);
    VOC_OK(hipGetLastError());
  }

  // mel [T][80] (device) -> g32 [256 T][24] (the body's output).
  void body(const float* mel, int T) {
    to_f16(mel, mel16, (size_t)T * 80, mel16_lo);
    conv(pre, mel16, mel16_lo, T, 1, 3, EPI_F16, nullptr, nullptr, nullptr, pre16, pre16_lo, 0);
    const half_t* cur = pre16;
    size_t cur_lo = pre16_lo;
    int Ts = T;
    for (int i = 0; i < 6; ++i) {
      conv(ups[i], cur, cur_lo, Ts, 1, 1, EPI_F32, x32, nullptr, nullptr, nullptr, 0, 0);
      Ts *= kUps[i].stride;
      group(i, x32, Ts, g32, g16);
      cur = g16;
      cur_lo = g16_lo;
    }
  }
};

bool Vocoder::present(const std::unordered_map<std::string, std::vector<float>>& t) {
  for (const auto& kv : t)
    if (kv.first.compare(0, 8, "bigvgan.") == 0) return true;
  return false;
}

Vocoder::Vocoder(const std::unordered_map<std::string, std::vector<float>>& t, hipStream_t stream)
    : d_(new Impl) {
  Impl& d = *d_;
  d.s = stream;
  if (const char* e = std::getenv("MIT2CFM_CONV_WINDOW")) d.conv_window = std::atoi(e) != 0;
  d.wa.reserve(size_t(600) << 20);  // ~236 MB of f16 weights, twice (split pairs)
  try {
    d.make_conv(d.pre, t, "bigvgan.conv_pre", 1536, 80, 7, true);
    for (int i = 0; i < 6; ++i) d.make_ups(d.ups[i], t, kUps[i]);
    for (int j = 0; j < 18; ++j) {
      const int C = rb_channels(j), k = kRbKernel[j % 3];
      const std::string p = "bigvgan.resblocks." + std::to_string(j);
      for (int pr = 0; pr < 3; ++pr) {
        d.make_conv(d.rb[j][pr][0], t, p + ".convs1." + std::to_string(pr), C, C, k, true);
        d.make_conv(d.rb[j][pr][1], t, p + ".convs2." + std::to_string(pr), C, C, k, true);
      }
      for (int a = 0; a < 6; ++a) d.make_act(d.act[j][a], t, p + ".activations." + std::to_string(a), C);
    }
    d.make_act(d.act_post, t, "bigvgan.activation_post", 24);
    d.upload_f32(d.post_w, wnorm(get(t, "bigvgan.conv_post.weight_g", 1),
                                 get(t, "bigvgan.conv_post.weight_v", 24 * 7), 1, 24 * 7));
    d.zero = static_cast<half_t*>(d.wa.take(2048 * 2));
    VOC_OK(hipMemset(d.zero, 0, 2048 * 2));
    d.bytes = d.wa.used();
  } catch (...) {
    delete d_;
    throw;
  }
}

// Image section: arena bytes used, then every conv (weight, bias and output
// scale offsets -- ~0 when the weight is a split pair --, N, stored columns,
// K, input channels, taps) and activation (filters,
// alpha and 1/beta offsets, channels) in construction order, conv_post and
// the zero buffer's offsets, then the arena bytes.
namespace {
template <typename F>
void visit_convs(Vocoder::Conv& pre, Vocoder::Conv (&ups)[6], Vocoder::Conv (&rb)[18][3][2], F&& f) {
  f(pre);
  for (auto& c : ups) f(c);
  for (auto& j : rb)
    for (auto& pr : j)
      for (auto& c : pr) f(c);
}
}  // namespace

void Vocoder::append_image(std::vector<uint8_t>& out) const {
  Impl& d = *d_;
  ImageWriter w{out};
  const char* base = d.wa.base();
  const size_t used = d.wa.used();
  w.put<uint64_t>(used);
  visit_convs(d.pre, d.ups, d.rb, [&](Conv& c) {
    w.put<uint64_t>(arena_offset(c.w, base));
    w.put<uint64_t>(arena_offset(c.b, base));
    w.put<uint64_t>(c.scale ? arena_offset(c.scale, base) : ~uint64_t(0));  // ~0: no scale (split weight)
    w.put<int32_t>(c.N);
    w.put<int32_t>(c.n_out);
    w.put<int32_t>(c.K);
    w.put<int32_t>(c.cin);
    w.put<int32_t>(c.k);
  });
  auto put_act = [&](const Act& a) {
    w.put(a.filt);
    w.put<uint64_t>(arena_offset(a.alpha, base));
    w.put<uint64_t>(arena_offset(a.inv_beta, base));
    w.put<int32_t>(a.C);
  };
  for (auto& j : d.act)
    for (auto& a : j) put_act(a);
  put_act(d.act_post);
  w.put<uint64_t>(arena_offset(d.post_w, base));
  w.put<uint64_t>(arena_offset(d.zero, base));
  std::vector<uint8_t> host(used);
  VOC_OK(hipMemcpy(host.data(), base, used, hipMemcpyDeviceToHost));
  w.bytes(host.data(), used);
}

Vocoder::Vocoder(const uint8_t* image, size_t bytes, hipStream_t stream) : d_(new Impl) {
  Impl& d = *d_;
  d.s = stream;
  if (const char* e = std::getenv("MIT2CFM_CONV_WINDOW")) d.conv_window = std::atoi(e) != 0;
  try {
    ImageReader r{image, bytes};
    const uint64_t used = r.get<uint64_t>();
    if (used == 0 || used > (uint64_t(8) << 30)) throw std::runtime_error("device image: bad vocoder arena size");
    d.wa.reserve(used);
    d.wa.set_used(used);
    char* base = d.wa.base();
    // The architecture fixes every conv's shape: (stored outputs, inputs, taps)
    // in visit order; the image must agree before any kernel trusts it.
    std::vector<std::array<int, 3>> shapes;
    shapes.push_back({1536, 80, 7});
    for (const UpsSpec& u : kUps) shapes.push_back({u.stride * u.cout, u.cin, 3});
    for (int j = 0; j < 18; ++j)
      for (int n = 0; n < 6; ++n) shapes.push_back({rb_channels(j), rb_channels(j), kRbKernel[j % 3]});
    size_t ci = 0;
    visit_convs(d.pre, d.ups, d.rb, [&](Conv& c) {
      const uint64_t wo = r.get<uint64_t>(), bo = r.get<uint64_t>(), so = r.get<uint64_t>();
      c.N = r.get<int32_t>();
      c.n_out = r.get<int32_t>();
      c.K = r.get<int32_t>();
      c.cin = r.get<int32_t>();
      c.k = r.get<int32_t>();
      const auto& e = shapes[ci++];
      if (c.n_out != e[0] || c.cin != e[1] || c.k != e[2] || c.N != round_up(e[0], 32) ||
          c.K != round_up(e[2] * e[1], 64))
        throw std::runtime_error("device image: vocoder conv shape differs from the model");
      // split pairs, or v alone with its output scale
      c.w = arena_span<half_t>(wo, (size_t)(so == ~uint64_t(0) ? 2 : 1) * c.N * c.K, base, used);
      c.b = arena_span<float>(bo, (size_t)c.N, base, used);
      c.scale = so == ~uint64_t(0) ? nullptr : arena_span<float>(so, (size_t)c.N, base, used);
    });
    auto get_act = [&](Act& a, int C) {
      a.filt = r.get<ActFilters>();
      const uint64_t ao = r.get<uint64_t>(), bo = r.get<uint64_t>();
      a.C = r.get<int32_t>();
      if (a.C != C) throw std::runtime_error("device image: vocoder activation width differs from the model");
      a.alpha = arena_span<float>(ao, (size_t)C, base, used);
      a.inv_beta = arena_span<float>(bo, (size_t)C, base, used);
    };
    for (int j = 0; j < 18; ++j)
      for (auto& a : d.act[j]) get_act(a, rb_channels(j));
    get_act(d.act_post, 24);
    d.post_w = arena_span<float>(r.get<uint64_t>(), 24 * 7, base, used);
    d.zero = arena_span<half_t>(r.get<uint64_t>(), 2048, base, used);
    VOC_OK(hipMemcpy(base, r.bytes(used), used, hipMemcpyHostToDevice));
    if (r.at != bytes) throw std::runtime_error("device image: trailing bytes in the vocoder section");
    d.bytes = used;
  } catch (...) {
    delete d_;
    throw;
  }
}

Vocoder::~Vocoder() { delete d_; }

void Vocoder::set_f32(bool on) { d_->f32 = on; }
bool Vocoder::f32() const { return d_->f32; }

size_t Vocoder::weight_bytes() const { return d_->bytes; }

void Vocoder::vocode_device(const float* mel, int tokens, float* wav) {
  if (tokens <= 0) throw std::invalid_argument("vocoder: tokens must be positive");
  d_->ensure(tokens);
  d_->body(mel, tokens);
  d_->post(d_->g32, tokens * 256, wav);
}

size_t Vocoder::stage_in_floats(int stage, int index, int tokens) {
  switch (stage) {
    case 0: return (size_t)tokens * 80;
    case 1: return index >= 0 && index < 6 ? (size_t)tokens * kUps[index].cin : 0;
    case 2: return index >= 0 && index < 108 ? (size_t)tokens * rb_channels(index / 6)
                                             : index == 108 ? (size_t)tokens * 24 : 0;
    case 3: return index >= 0 && index < 18 ? (size_t)tokens * rb_channels(index) : 0;
    case 4: return index >= 0 && index < 6 ? (size_t)tokens * kUps[index].cout : 0;
    case 5: return (size_t)tokens * 24;
    case 6: return (size_t)tokens * 80;
    default: return 0;
  }
}

size_t Vocoder::stage_out_floats(int stage, int index, int tokens) {
  switch (stage) {
    case 0: return (size_t)tokens * 1536;
    case 1: return index >= 0 && index < 6 ? (size_t)tokens * kUps[index].stride * kUps[index].cout : 0;
    case 2: case 3: case 4: return stage_in_floats(stage, index, tokens);
    case 5: return (size_t)tokens;
    case 6: return (size_t)tokens * 256 * 24;
    default: return 0;
  }
}

size_t Vocoder::stage_host(int stage, int index, const float* in, int tokens, float* out) {
  const size_t nin = stage_in_floats(stage, index, tokens), nout = stage_out_floats(stage, index, tokens);
  if (tokens <= 0 || nin == 0 || nout == 0) throw std::invalid_argument("vocoder stage: bad stage/index/tokens");
  Impl& d = *d_;
  // The stage buffers hold 6144 floats per mel token of capacity: size them
  // so this stage's input and output fit (conv_pre and the body take mel
  // tokens, whose own buffers are per token).
  const int cap_tokens = (int)((std::max(nin, nout) + 6143) / 6144) + 1;
  d.ensure(stage == 0 || stage == 6 ? std::max(tokens, cap_tokens) : cap_tokens);
  float* din = nullptr;
  float* dout = nullptr;
  VOC_OK(hipMalloc(&din, nin * 4));
  VOC_OK(hipMalloc(&dout, nout * 4));
  try {
    VOC_OK(hipMemcpyAsync(din, in, nin * 4, hipMemcpyHostToDevice, d.s));
    switch (stage) {
      case 0:
        d.to_f16(din, d.mel16, nin, d.mel16_lo);
        d.conv(d.pre, d.mel16, d.mel16_lo, tokens, 1, 3, EPI_F32, dout, nullptr, nullptr, nullptr, 0, 0);
        break;
      case 1:
        d.to_f16(din, d.a16, nin, d.a16_lo);
        d.conv(d.ups[index], d.a16, d.a16_lo, tokens, 1, 1, EPI_F32, dout, nullptr, nullptr, nullptr, 0, 0);
        break;
      case 2:
        d.activation(index == 108 ? d.act_post : d.act[index / 6][index % 6], din, tokens, dout, false);
        break;
      case 3:
        d.resblock(index, din, tokens, dout, d.g32, 0, nullptr);
        break;
      case 4:
        d.group(index, din, tokens, dout, nullptr);
        break;
      case 5:
        d.post(din, tokens, dout);
        break;
      case 6:
        d.body(din, tokens);
        VOC_OK(hipMemcpyAsync(dout, d.g32, nout * 4, hipMemcpyDeviceToDevice, d.s));
        break;
    }
    VOC_OK(hipMemcpyAsync(out, dout, nout * 4, hipMemcpyDeviceToHost, d.s));
    VOC_OK(hipStreamSynchronize(d.s));
  } catch (...) {
    (void)hipStreamSynchronize(d.s);
    (void)hipFree(din);
    (void)hipFree(dout);
    throw;
  }
  VOC_OK(hipFree(din));
  VOC_OK(hipFree(dout));
  return nout;
}

}  // namespace mit2hip
