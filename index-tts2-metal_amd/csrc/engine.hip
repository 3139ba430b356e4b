// engine.hip -- host engine of the HIP DiT-CFM decoder.
//
// Replaces the reference's Metal pass runtime for this path
// (runtime/metal_context.mm: resident weights :677-694, pass workspace
// :448-461, :4560-4661) and the single-pass decode recorder
// (runtime/impl/dit_cfm_bigvgan.cpp:2367-2713, t-tables :2946-3023).
//
// Differences in HOW, not WHAT:
//  * weights are prepared once at create: weight norm folded, f16, rows
//    permuted for the fused epilogues (RoPE pairs, SwiGLU halves, WaveNet
//    gate halves), the k=5 conv laid out tap-major for an implicit GEMM;
//  * step-invariant work is hoisted out of the Euler loop: the content
//    projection and the prompt/content/style part of the input-merge GEMM
//    are computed once per decode; only the 80 mel columns are re-multiplied
//    per step (the sum is re-associated, not changed);
//  * the whole decode (tables, set-up, S steps) is captured once per shape
//    into a hipGraph and replayed on one stream.
#include "engine.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <thread>
#include <type_traits>
#include <unordered_map>

#include "condition.h"
#include "gemm.h"
#include "gpt.h"
#include "image_io.h"
#include "rowops.h"
#include "vocoder.h"

namespace mit2hip {

#define HIP_OK(expr)                                                                      \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess)                                                                 \
      throw HipError(std::string(#expr) + " failed: " + hipGetErrorString(e_) + " (" +   \
                     __FILE__ + ":" + std::to_string(__LINE__) + ")");                    \
  } while (0)

static const char* kPfx = "s2mel.net.cfm.estimator.";
constexpr int kTcondPerStep = 36864;  // [13 attn | 13 ffn | final norm] x 1024, final ss 1024, wn cond 8192
constexpr int kFinalSsOff = 27 * 1024;
constexpr int kWnCondOff = 28 * 1024;
// Row pitch of Workspace::hg16: f16(h) (512) | SwiGLU output (1536).
constexpr int kHgLd = 2048;

// ------------------------------------------------------------------ no-alloc scratch
// Scratch of the allocation-free condition producer
// (Engine::condition_device_noalloc): the length regulator's buffers for up
// to kNoAllocMaxCodes codes, as LrView lays them out, in one static device
// array.  Each GPU the library runs on holds its own copy until the process
// ends; every context on that GPU shares it.
namespace {
constexpr int kNoAllocMaxFrames = (int)((float)Engine::kNoAllocMaxCodes * 1.72f);  // generated_frames
constexpr size_t al256(size_t b) { return (b + 255) / 256 * 256; }
constexpr size_t kScrS16 = 0;
constexpr size_t kScrP16 = kScrS16 + al256((size_t)Engine::kNoAllocMaxCodes * 1024 * 2 * 2);
constexpr size_t kScrX16 = kScrP16 + al256((size_t)Engine::kNoAllocMaxCodes * 512 * 2 * 2);
constexpr size_t kScrY32 = kScrX16 + al256((size_t)(kNoAllocMaxFrames + 1) * 512 * 2 * 2);
constexpr size_t kScrSum = kScrY32 + al256((size_t)kNoAllocMaxFrames * 512 * 4);
constexpr size_t kScrSsq = kScrSum + al256((size_t)kNoAllocMaxFrames * 16 * 4);
constexpr size_t kScratchBytes = kScrSsq + al256((size_t)kNoAllocMaxFrames * 16 * 4);  // 13.7 MB
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
// Device address of `scratch` per GPU (hipGetSymbolAddress with that GPU
// current); the array's name is only a host-side stand-in.
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};
// Orders the calls that use a GPU's scratch: each call's stream waits for the
// event the previous call recorded after its last kernel, then records it
// again after its own, so calls from contexts on different streams run one
// after another instead of overlapping.  Held under g_scratch_call_mu while
// a call is enqueued, so two host threads cannot interleave their wait and
// record.
hipEvent_t g_scratch_ev[kMaxScratchDevices] = {};
std::mutex g_scratch_call_mu;

// Resolves this GPU's scratch address (and creates its ordering event) once;
// the caller has made `device` current.  Called when a context is created.
void resolve_scratch(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return;  // the no-alloc call then reports it
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    throw HipError(std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
  hipEvent_t ev = nullptr;
  const hipError_t ee = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (ee != hipSuccess) throw HipError(std::string("hipEventCreate failed: ") + hipGetErrorString(ee));
  g_scratch_ev[device] = ev;
  g_scratch_ptr[device] = p;
}

char* scratch_ptr(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return static_cast<char*>(g_scratch_ptr[device]);
}
}  // namespace

// ------------------------------------------------------------------ arena
Arena::~Arena() {
  if (base_) (void)hipFree(base_);
}

void Arena::reserve(size_t bytes) {
  if (base_) {
    HIP_OK(hipFree(base_));
    base_ = nullptr;
  }
  cap_ = bytes;
  used_ = 0;
  if (bytes) HIP_OK(hipMalloc(reinterpret_cast<void**>(&base_), bytes));
}

void* Arena::take(size_t bytes) {
  const size_t off = (used_ + 255) & ~size_t(255);
  if (off + bytes > cap_) throw HipError("device arena exhausted");
  used_ = off + bytes;
  return base_ + off;
}

// ------------------------------------------------------------------ weights
struct Weights {
  Arena arena;
  // timestep-conditioning (fp32)
  float* te_freqs[2];
  float* te_w0[2];
  float* te_b0[2];
  float* te_w2[2];
  float* te_b2[2];
  float* proj_w;  // [27*1024][512]
  float* proj_b;
  float* ada_w;   // [1024][512]
  float* ada_b;
  float* wnc_w;   // [8192][512] weight-normed
  float* wnc_b;
  float* gamma[27];
  // GEMM weights (f16)
  half_t* cp_w;  float* cp_b;
  half_t* mx_w;                // [512][kMelPad]
  half_t* mc_w;  float* mc_b;  // [512][kMcWidth]
  half_t* qkv_w[13];
  half_t* wo_w[13];
  half_t* w13_w[13];
  half_t* w2_w[13];
  half_t* si_w[13]; float* si_b[13];
  // Blocks 7..12: skip_in_l([out_{l-1} | skip]) with out_{l-1} = h + w2 . g
  // (block l-1's FFN output, read by nothing else) as one map over
  // [f16(h) | g | skip]: [Wsi_x | Wsi_x . W2_{l-1} | Wsi_skip], [512][2560].
  half_t* fold_w[13];
  half_t* sl_w;  float* sl_b;  // [512][512 + kMelPad]
  // conv1|res_projection . skip_linear as one map (nothing else reads the
  // skip_linear output): [1024][512 + kMelPad] and [1024].
  half_t* post_w; float* post_b;
  half_t* in_w[8]; float* in_b[8];  // [1024][2560]
  half_t* rs_w[8]; float* rs_b[8];
  half_t* fin_w; float* fin_b;
  half_t* c2_w;  float* c2_b;   // [80][512]
  // conv2 . final_layer.linear as one map (both are linear and nothing reads
  // the 512-wide final-layer output in between): [80][512] and [80].
  half_t* c2f_w; float* c2f_b;
  // Length regulator (condition producer), present when the bundle has it:
  // content_in_proj [512][1024]; conv k=3 taps tap-major [512][3 * 512];
  // GroupNorm affine [512]; the k=1 output conv [512][512].  Its GEMM
  // weights are split pairs (hi, then lo at + the hi element count, see
  // GemmArgs::split); lr_wsplit is 2 when some lo half is nonzero (weights
  // not exact in f16), else 1.
  bool has_lr = false;
  int lr_wsplit = 1;
  half_t* lr_proj_w; float* lr_proj_b;
  half_t* lr_conv_w[4]; float* lr_conv_b[4];
  float* lr_gn_w[4]; float* lr_gn_b[4];
  half_t* lr_out_w; float* lr_out_b;
};

namespace {

// Every device array of Weights with its element count, in a fixed order
// (the device image stores their arena offsets in this order).  Arrays a
// model lacks (the length regulator's, the skip-in of layers 0..6) are null.
template <typename F>
void visit_weights(Weights& W, F&& f) {
  for (int i = 0; i < 2; ++i) {
    f(W.te_freqs[i], 128);
    f(W.te_w0[i], 512 * 256);
    f(W.te_b0[i], 512);
    f(W.te_w2[i], 512 * 512);
    f(W.te_b2[i], 512);
  }
  f(W.proj_w, (size_t)27 * 1024 * 512);
  f(W.proj_b, 27 * 1024);
  f(W.ada_w, 1024 * 512);
  f(W.ada_b, 1024);
  f(W.wnc_w, (size_t)8192 * 512);
  f(W.wnc_b, 8192);
  for (auto& g : W.gamma) f(g, 512);
  f(W.cp_w, 512 * 512);
  f(W.cp_b, 512);
  f(W.mx_w, 512 * kMelPad);
  f(W.mc_w, 512 * kMcWidth);
  f(W.mc_b, 512);
  for (int l = 0; l < 13; ++l) {
    f(W.qkv_w[l], 1536 * 512);
    f(W.wo_w[l], 512 * 512);
    f(W.w13_w[l], 3072 * 512);
    f(W.w2_w[l], 512 * 1536);
    f(W.si_w[l], 512 * 1024);
    f(W.si_b[l], 512);
    f(W.fold_w[l], 512 * 2560);
  }
  f(W.sl_w, 512 * (512 + kMelPad));
  f(W.sl_b, 512);
  f(W.post_w, 1024 * (512 + kMelPad));
  f(W.post_b, 1024);
  for (int l = 0; l < 8; ++l) {
    f(W.in_w[l], 1024 * 2560);
    f(W.in_b[l], 1024);
    f(W.rs_w[l], (l < 7 ? 1024 : 512) * 512);
    f(W.rs_b[l], l < 7 ? 1024 : 512);
  }
  f(W.fin_w, 512 * 512);
  f(W.fin_b, 512);
  f(W.c2_w, 80 * 512);
  f(W.c2_b, 80);
  f(W.c2f_w, 80 * 512);
  f(W.c2f_b, 80);
  f(W.lr_proj_w, 2 * 512 * 1024);  // split pairs: hi then lo
  f(W.lr_proj_b, 512);
  for (int b = 0; b < 4; ++b) {
    f(W.lr_conv_w[b], 2 * 512 * 1536);
    f(W.lr_conv_b[b], 512);
    f(W.lr_gn_w[b], 512);
    f(W.lr_gn_b[b], 512);
  }
  f(W.lr_out_w, 2 * 512 * 512);
  f(W.lr_out_b, 512);
}

// Device image layout: "MIT2HIPI", u32 version, u32 section flags (1 vocoder,
// 2 GPT decoder), u64 payload bytes, u64 payload checksum, then the payload:
// the decoder section (u64 arena bytes, u8 length regulator: 0 absent, else
// its weight split mode 1 or 2, u64 offset per visit_weights array, the
// arena bytes), then each flagged section as u64 length + bytes
// (Vocoder::append_image, GptDecoder::append_image).
constexpr char kImageMagic[8] = {'M', 'I', 'T', '2', 'H', 'I', 'P', 'I'};
constexpr uint32_t kImageVersion = 6;
constexpr uint32_t kImageVocoder = 1, kImageGpt = 2;  // section flags

struct HostModel {
  std::unordered_map<std::string, std::vector<float>> t;
  bool has(const std::string& full) const { return t.count(full) != 0; }
  const std::vector<float>& get_full(const std::string& full, size_t elems) const {
    auto it = t.find(full);
    if (it == t.end()) throw std::invalid_argument("missing tensor: " + full);
    if (it->second.size() != elems)
      throw std::invalid_argument("tensor " + full + " has " + std::to_string(it->second.size()) +
                                  " elements, expected " + std::to_string(elems));
    return it->second;
  }
  const std::vector<float>& get(const std::string& tail, size_t elems) const {
    auto it = t.find(std::string(kPfx) + tail);
    if (it == t.end()) throw std::invalid_argument("missing tensor: " + std::string(kPfx) + tail);
    if (it->second.size() != elems)
      throw std::invalid_argument("tensor " + std::string(kPfx) + tail + " has " +
                                  std::to_string(it->second.size()) + " elements, expected " +
                                  std::to_string(elems));
    return it->second;
  }
};

float half_bits_to_float(uint16_t h) {
  _Float16 v;
  std::memcpy(&v, &h, 2);
  return (float)v;
}

// w = g * v / ||v|| per output row (gpt.cpp:5109 weight_norm_rowmajor).
std::vector<float> weight_norm(const std::vector<float>& g, const std::vector<float>& v, size_t rows,
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

class Uploader {
 public:
  explicit Uploader(Arena& a) : a_(a) {}
  float* f32(const std::vector<float>& v) {
    float* d = static_cast<float*>(a_.take(v.size() * sizeof(float)));
    HIP_OK(hipMemcpy(d, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
    return d;
  }
  half_t* f16(const std::vector<float>& v) {
    std::vector<_Float16> h(v.size());
    for (size_t i = 0; i < v.size(); ++i) h[i] = (_Float16)v[i];
    half_t* d = static_cast<half_t*>(a_.take(h.size() * sizeof(_Float16)));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(_Float16), hipMemcpyHostToDevice));
    return d;
  }
  // Split pair of v (hi, then lo at + v.size(), GemmArgs::split); *lo_used
  // is set when some lo half is nonzero.
  half_t* f16_pair(const std::vector<float>& v, bool* lo_used) {
    const size_t n = v.size();
    std::vector<_Float16> h(2 * n);
    for (size_t i = 0; i < n; ++i) {
      split_f16_host(v[i], h[i], h[n + i]);
      if ((float)h[n + i] != 0.0f) *lo_used = true;
    }
    half_t* d = static_cast<half_t*>(a_.take(h.size() * sizeof(_Float16)));
    HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(_Float16), hipMemcpyHostToDevice));
    return d;
  }

 private:
  Arena& a_;
};

// Row permutations used by the paired epilogues (32-row groups).
// RoPE pairs: GEMM row 32g + j holds original row 32g + 2j (j < 16) or 32g + 2(j-16) + 1.
int rope_pair_row(int c) {
  const int g = c >> 5, j = c & 31;
  return 32 * g + (j < 16 ? 2 * j : 2 * (j - 16) + 1);
}
// Halves interleave: GEMM row 32g + j holds first-half row 16g + j (j < 16) or
// second-half row half + 16g + (j - 16).
int halves_row(int c, int half) {
  const int g = c >> 5, j = c & 31;
  return j < 16 ? 16 * g + j : half + 16 * g + (j - 16);
}

std::vector<float> permute_rows(const std::vector<float>& w, int rows, int cols,
                                int (*map)(int, int), int arg) {
  std::vector<float> out((size_t)rows * cols);
  for (int c = 0; c < rows; ++c)
    std::memcpy(&out[(size_t)c * cols], &w[(size_t)map(c, arg) * cols], cols * sizeof(float));
  return out;
}

int rope_map(int c, int) { return rope_pair_row(c); }
int halves_map(int c, int half) { return halves_row(c, half); }
// Column pairs (GemmArgs::colperm): GEMM row 32q + 16h + 4g + r holds output
// column 32q + 8g + 4h + r, so a lane's two MFMA blocks write 8 consecutive
// columns.  Used for the weights of the GEMMs that produce a folded-norm
// operand (wo, w2, the folded w2|skip-in, skip-in, the per-step merge).
int colpair_map(int c, int) { return (c & ~31) | (((c >> 2) & 3) << 3) | (((c >> 4) & 1) << 2) | (c & 3); }

// Copies a column block [c0, c0+n) of src [rows][scols] into dst [rows][dcols] at column d0.
void copy_cols(const std::vector<float>& src, int rows, int scols, int c0, int n,
               std::vector<float>& dst, int dcols, int d0) {
  for (int r = 0; r < rows; ++r)
    std::memcpy(&dst[(size_t)r * dcols + d0], &src[(size_t)r * scols + c0], n * sizeof(float));
}

}  // namespace

// ------------------------------------------------------------------ workspace
struct Workspace {
  Arena arena;
  int capR = 0, capT = 0, capTpad = 0, capB = 0, capS = 0, capReq = 0;
  float* x_cur;
  half_t* xmel16;
  half_t* cond16;
  half_t* mc16;
  float* xin_const;
  float* xa;
  float* xb;
  half_t* skip16[6];
  half_t* x16;
  half_t* n16;
  half_t* q;
  half_t* k;
  half_t* vt;
  half_t* o16;
  // [R][kHgLd]: columns 0..511 f16(h) (the post-attention stream, written by
  // the wo GEMM of a block whose w2 is folded into the next skip-in),
  // columns 512..2047 the SwiGLU output g16 points at.
  half_t* hg16;
  half_t* g16;
  half_t* ls16;
  float* wn_x;
  half_t* wn_x16;
  float* rp;
  float* wn_out;
  half_t* gate16;
  float* fin;
  uint32_t* mask;
  float* kbias;  // [B][Tpad] attention key bias (0 valid, -inf masked/padding), then [B] key counts
  uint32_t* P;
  float2* rope;
  float* tvals;
  float* temb;
  float* th;
  float* t1;
  float* t2;
  float* tab;
  float* ssq;   // [R][kSsqParts] partial row sums of squares (folded AdaRMSNorm)
  float* nbq;   // [S][13][1536] folded attention-norm column bias (ab . Wqkv^T)
  float* nbw;   // [S][13][3072] folded ffn-norm column bias (ab . W13^T)
  // The workspace's own one-step tables (estimator forwards, stage entry points).
  TableBufs one() const { return TableBufs{tvals, temb, th, t1, t2, tab, nbq, nbw}; }
  // staging for host-pointer entry points
  float* in_x;
  float* in_prompt;
  float* in_cond;
  float* in_style;
  float* out_x;
  float* dphi;
  float* stage_a;
  float* stage_b;
  float* stage_c;
  int Tcur = 0;  // T the rope table currently holds
  // What ws.mask / ws.P hold for the decode path (every other writer of
  // ws.mask clears mask_host).
  std::vector<uint32_t> mask_host, P_host;
};

// ------------------------------------------------------------------ engine
Engine::Engine(const std::vector<HostTensor>& tensors, int device) : device_(device) {
  HIP_OK(hipSetDevice(device_));
  resolve_scratch(device_);
  HIP_OK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  if (const char* g = std::getenv("MIT2CFM_GRAPH")) use_graph_ = std::atoi(g) != 0;

  HostModel hm;
  for (const auto& ht : tensors) {
    std::vector<float> v(ht.elems);
    if (ht.dtype == 0) {
      std::memcpy(v.data(), ht.data, ht.elems * sizeof(float));
    } else if (ht.dtype == 1) {
      const uint16_t* h = static_cast<const uint16_t*>(ht.data);
      for (uint64_t i = 0; i < ht.elems; ++i) v[i] = half_bits_to_float(h[i]);
    } else {
      throw std::invalid_argument("tensor " + ht.name + ": dtype must be f32 or f16");
    }
    hm.t[ht.name] = std::move(v);
  }

  w_ = std::make_unique<Weights>();
  Weights& W = *w_;
  // Size: f16 GEMM weights ~150 MB + fp32 table weights ~80 MB; reserve with slack.
  W.arena.reserve(size_t(320) << 20);
  Uploader up(W.arena);

  const char* te[2] = {"t_embedder", "t_embedder2"};
  for (int i = 0; i < 2; ++i) {
    const std::string p = te[i];
    W.te_freqs[i] = up.f32(hm.get(p + ".freqs", 128));
    W.te_w0[i] = up.f32(hm.get(p + ".mlp.0.weight", 512 * 256));
    W.te_b0[i] = up.f32(hm.get(p + ".mlp.0.bias", 512));
    W.te_w2[i] = up.f32(hm.get(p + ".mlp.2.weight", 512 * 512));
    W.te_b2[i] = up.f32(hm.get(p + ".mlp.2.bias", 512));
  }
  {
    std::vector<float> pw((size_t)27 * 1024 * 512), pb((size_t)27 * 1024);
    for (int id = 0; id < 27; ++id) {
      std::string p = id < 13   ? "transformer.layers." + std::to_string(id) + ".attention_norm"
                      : id < 26 ? "transformer.layers." + std::to_string(id - 13) + ".ffn_norm"
                                : std::string("transformer.norm");
      const auto& w = hm.get(p + ".project_layer.weight", 1024 * 512);
      const auto& b = hm.get(p + ".project_layer.bias", 1024);
      std::memcpy(&pw[(size_t)id * 1024 * 512], w.data(), w.size() * sizeof(float));
      std::memcpy(&pb[(size_t)id * 1024], b.data(), b.size() * sizeof(float));
      W.gamma[id] = up.f32(hm.get(p + ".norm.weight", 512));
    }
    W.proj_w = up.f32(pw);
    W.proj_b = up.f32(pb);
  }
  W.ada_w = up.f32(hm.get("final_layer.adaLN_modulation.1.weight", 1024 * 512));
  W.ada_b = up.f32(hm.get("final_layer.adaLN_modulation.1.bias", 1024));
  {
    const std::string p = "wavenet.cond_layer.conv.conv";
    W.wnc_w = up.f32(weight_norm(hm.get(p + ".weight_g", 8192), hm.get(p + ".weight_v", 8192 * 512),
                                 8192, 512));
    W.wnc_b = up.f32(hm.get(p + ".bias", 8192));
  }

  W.cp_w = up.f16(hm.get("cond_projection.weight", 512 * 512));
  W.cp_b = up.f32(hm.get("cond_projection.bias", 512));
  {
    const auto& mw = hm.get("cond_x_merge_linear.weight", 512 * 864);
    std::vector<float> mx((size_t)512 * kMelPad, 0.f), mc((size_t)512 * kMcWidth, 0.f);
    copy_cols(mw, 512, 864, 0, 80, mx, kMelPad, 0);               // x
    copy_cols(mw, 512, 864, 80, 80, mc, kMcWidth, 0);             // prompt_x
    copy_cols(mw, 512, 864, 160, 512, mc, kMcWidth, kMcContent);  // content projection
    copy_cols(mw, 512, 864, 672, 192, mc, kMcWidth, kMcStyle);    // style
    W.mx_w = up.f16(permute_rows(mx, 512, kMelPad, colpair_map, 0));
    W.mc_w = up.f16(mc);
    W.mc_b = up.f32(hm.get("cond_x_merge_linear.bias", 512));
  }
  for (int l = 0; l < 13; ++l) {
    const std::string p = "transformer.layers." + std::to_string(l);
    W.qkv_w[l] = up.f16(permute_rows(hm.get(p + ".attention.wqkv.weight", 1536 * 512), 1536, 512,
                                     rope_map, 0));
    W.wo_w[l] = up.f16(permute_rows(hm.get(p + ".attention.wo.weight", 512 * 512), 512, 512, colpair_map, 0));
    {
      const auto& w1 = hm.get(p + ".feed_forward.w1.weight", 1536 * 512);
      const auto& w3 = hm.get(p + ".feed_forward.w3.weight", 1536 * 512);
      std::vector<float> w13((size_t)3072 * 512);
      std::memcpy(w13.data(), w1.data(), w1.size() * sizeof(float));
      std::memcpy(w13.data() + w1.size(), w3.data(), w3.size() * sizeof(float));
      W.w13_w[l] = up.f16(permute_rows(w13, 3072, 512, halves_map, 1536));
    }
    W.w2_w[l] = up.f16(permute_rows(hm.get(p + ".feed_forward.w2.weight", 512 * 1536), 512, 1536, colpair_map, 0));
    if (l > 6) {
      W.si_w[l] = up.f16(permute_rows(hm.get(p + ".skip_in_linear.weight", 512 * 1024), 512, 1024, colpair_map, 0));
      W.si_b[l] = up.f32(hm.get(p + ".skip_in_linear.bias", 512));
    } else {
      W.si_w[l] = nullptr;
      W.si_b[l] = nullptr;
    }
    W.fold_w[l] = nullptr;
  }
  {
    // Blocks 7..12: skip_in_l([h + W2 g | skip]) = Wsi_x h + (Wsi_x W2) g +
    // Wsi_skip skip + b (block l-1's w2 has no bias), Wsi_x W2 summed in
    // double from the fp32 weights and rounded once to f16.  One thread per
    // block (about 0.4 G multiply-adds each).
    std::vector<std::vector<float>> fw(13);
    std::vector<std::thread> th;
    for (int l = 7; l < 13; ++l) {
      const auto& si = hm.get(std::string("transformer.layers.") + std::to_string(l) +
                                  ".skip_in_linear.weight", 512 * 1024);
      const auto& w2 = hm.get(std::string("transformer.layers.") + std::to_string(l - 1) +
                                  ".feed_forward.w2.weight", 512 * 1536);
      fw[l].assign((size_t)512 * 2560, 0.f);
      th.emplace_back([&si, &w2, out = fw[l].data()] {
        std::vector<double> row(1536);
        for (int n = 0; n < 512; ++n) {
          std::fill(row.begin(), row.end(), 0.0);
          const float* sn = si.data() + (size_t)n * 1024;
          for (int j = 0; j < 512; ++j) {
            const double c = sn[j];
            const float* wj = w2.data() + (size_t)j * 1536;
            for (int k = 0; k < 1536; ++k) row[k] += c * wj[k];
          }
          float* on = out + (size_t)n * 2560;
          std::memcpy(on, sn, 512 * sizeof(float));
          for (int k = 0; k < 1536; ++k) on[512 + k] = (float)row[k];
          std::memcpy(on + 2048, sn + 512, 512 * sizeof(float));
        }
      });
    }
    for (auto& t : th) t.join();
    for (int l = 7; l < 13; ++l) W.fold_w[l] = up.f16(permute_rows(fw[l], 512, 2560, colpair_map, 0));
  }
  {
    const auto& sw = hm.get("skip_linear.weight", 512 * 592);
    std::vector<float> s((size_t)512 * (512 + kMelPad), 0.f);
    copy_cols(sw, 512, 592, 0, 592, s, 512 + kMelPad, 0);
    W.sl_w = up.f16(s);
    W.sl_b = up.f32(hm.get("skip_linear.bias", 512));
  }
  {
    const auto& c1 = hm.get("conv1.weight", 512 * 512);
    const auto& rpw = hm.get("res_projection.weight", 512 * 512);
    std::vector<float> w((size_t)1024 * 512), b(1024);
    std::memcpy(w.data(), c1.data(), c1.size() * sizeof(float));
    std::memcpy(w.data() + c1.size(), rpw.data(), rpw.size() * sizeof(float));
    const auto& c1b = hm.get("conv1.bias", 512);
    const auto& rpb = hm.get("res_projection.bias", 512);
    std::memcpy(b.data(), c1b.data(), 512 * sizeof(float));
    std::memcpy(b.data() + 512, rpb.data(), 512 * sizeof(float));
    // [c1; rp] (W_sl x + b_sl) + [b_c1; b_rp], summed in double from the fp32
    // weights, rounded once to f16.
    const auto& sw = hm.get("skip_linear.weight", 512 * 592);
    const auto& sb = hm.get("skip_linear.bias", 512);
    constexpr int kw = 512 + kMelPad;
    std::vector<float> pw((size_t)1024 * kw, 0.f), pb(1024);
    std::vector<double> row(592);
    for (int n = 0; n < 1024; ++n) {
      std::fill(row.begin(), row.end(), 0.0);
      double bsum = b[n];
      const float* wn = w.data() + (size_t)n * 512;
      for (int j = 0; j < 512; ++j) {
        const double c = wn[j];
        bsum += c * sb[j];
        const float* srow = sw.data() + (size_t)j * 592;
        for (int k = 0; k < 592; ++k) row[k] += c * srow[k];
      }
      pb[n] = (float)bsum;
      for (int k = 0; k < 592; ++k) pw[(size_t)n * kw + k] = (float)row[k];
    }
    W.post_w = up.f16(pw);
    W.post_b = up.f32(pb);
  }
  for (int l = 0; l < 8; ++l) {
    const std::string p = "wavenet.in_layers." + std::to_string(l) + ".conv.conv";
    // [1024][512*5] (index ic*5 + k) -> tap-major [1024][k*512 + ic], rows interleaved a|b.
    auto wn = weight_norm(hm.get(p + ".weight_g", 1024), hm.get(p + ".weight_v", 1024 * 512 * 5),
                          1024, 2560);
    std::vector<float> tm((size_t)1024 * 2560);
    for (int oc = 0; oc < 1024; ++oc)
      for (int ic = 0; ic < 512; ++ic)
        for (int k = 0; k < 5; ++k)
          tm[(size_t)oc * 2560 + k * 512 + ic] = wn[(size_t)oc * 2560 + ic * 5 + k];
    W.in_w[l] = up.f16(permute_rows(tm, 1024, 2560, halves_map, 512));
    const auto& b = hm.get(p + ".bias", 1024);
    std::vector<float> bp(1024);
    for (int c = 0; c < 1024; ++c) bp[c] = b[halves_row(c, 512)];
    W.in_b[l] = up.f32(bp);

    const int rc = l < 7 ? 1024 : 512;
    const std::string q = "wavenet.res_skip_layers." + std::to_string(l) + ".conv.conv";
    W.rs_w[l] = up.f16(weight_norm(hm.get(q + ".weight_g", rc), hm.get(q + ".weight_v", (size_t)rc * 512),
                                   rc, 512));
    W.rs_b[l] = up.f32(hm.get(q + ".bias", rc));
  }
  {
    // dphi = Wc2 (Wf y + bf) + bc2 = (Wc2 Wf) y + (Wc2 bf + bc2), summed in
    // double from the fp32 weights (weight norm applied), rounded once to f16.
    const std::vector<float> wf = weight_norm(hm.get("final_layer.linear.weight_g", 512),
                                              hm.get("final_layer.linear.weight_v", 512 * 512), 512, 512);
    const std::vector<float>& bf = hm.get("final_layer.linear.bias", 512);
    const std::vector<float>& wc = hm.get("conv2.weight", 80 * 512);
    const std::vector<float>& bc = hm.get("conv2.bias", 80);
    W.fin_w = up.f16(wf);
    W.fin_b = up.f32(bf);
    W.c2_w = up.f16(wc);
    W.c2_b = up.f32(bc);
    std::vector<double> acc((size_t)80 * 512, 0.0);
    std::vector<float> wcf((size_t)80 * 512), bcf(80);
    for (int n = 0; n < 80; ++n) {
      double bsum = bc[n];
      for (int j = 0; j < 512; ++j) {
        const double c = wc[(size_t)n * 512 + j];
        bsum += c * bf[j];
        const float* wrow = wf.data() + (size_t)j * 512;
        double* arow = acc.data() + (size_t)n * 512;
        for (int k = 0; k < 512; ++k) arow[k] += c * wrow[k];
      }
      bcf[n] = (float)bsum;
      for (int k = 0; k < 512; ++k) wcf[(size_t)n * 512 + k] = (float)acc[(size_t)n * 512 + k];
    }
    W.c2f_w = up.f16(wcf);
    W.c2f_b = up.f32(bcf);
  }

  // Length regulator (gpt.cpp:5271-5340): all of its tensors or none.
  {
    const std::string lp = "s2mel.net.length_regulator.";
    int present = 0;
    for (const auto& kv : hm.t) present += kv.first.compare(0, lp.size(), lp) == 0;
    if (present) {
      bool lo_used = false;
      W.lr_proj_w = up.f16_pair(hm.get_full(lp + "content_in_proj.weight", 512 * 1024), &lo_used);
      W.lr_proj_b = up.f32(hm.get_full(lp + "content_in_proj.bias", 512));
      const int conv_i[4] = {0, 3, 6, 9}, norm_i[4] = {1, 4, 7, 10};
      for (int b = 0; b < 4; ++b) {
        const std::string c = lp + "model." + std::to_string(conv_i[b]);
        const std::string n = lp + "model." + std::to_string(norm_i[b]);
        // PyTorch [oc][ic][k] -> tap-major [oc][k * 512 + ic]
        const auto& w = hm.get_full(c + ".weight", (size_t)512 * 512 * 3);
        std::vector<float> tw((size_t)512 * 1536);
        for (int oc = 0; oc < 512; ++oc)
          for (int ic = 0; ic < 512; ++ic)
            for (int k = 0; k < 3; ++k)
              tw[(size_t)oc * 1536 + k * 512 + ic] = w[((size_t)oc * 512 + ic) * 3 + k];
        W.lr_conv_w[b] = up.f16_pair(tw, &lo_used);
        W.lr_conv_b[b] = up.f32(hm.get_full(c + ".bias", 512));
        W.lr_gn_w[b] = up.f32(hm.get_full(n + ".weight", 512));
        W.lr_gn_b[b] = up.f32(hm.get_full(n + ".bias", 512));
      }
      W.lr_out_w = up.f16_pair(hm.get_full(lp + "model.12.weight", 512 * 512), &lo_used);
      W.lr_out_b = up.f32(hm.get_full(lp + "model.12.bias", 512));
      W.lr_wsplit = lo_used ? 2 : 1;
      if (present != 20)
        throw std::invalid_argument("length regulator: expected 20 tensors, found " +
                                    std::to_string(present));
      W.has_lr = true;
    }
  }

  if (Vocoder::present(hm.t)) voc_ = std::make_unique<Vocoder>(hm.t, stream_);
  if (GptDecoder::present(hm.t)) gpt_ = std::make_unique<GptDecoder>(hm.t, stream_);
  ws_ = std::make_unique<Workspace>();
}

void Engine::write_image(const std::string& path) const {
  HIP_OK(hipSetDevice(device_));
  HIP_OK(hipStreamSynchronize(stream_));
  std::vector<uint8_t> payload;
  ImageWriter w{payload};
  Weights& W = *w_;
  const char* base = W.arena.base();
  const size_t used = W.arena.used();
  w.put<uint64_t>(used);
  w.put<uint8_t>(W.has_lr ? (uint8_t)W.lr_wsplit : 0);
  visit_weights(W, [&](auto* p, size_t) { w.put<uint64_t>(arena_offset(p, base)); });
  std::vector<uint8_t> host(used);
  HIP_OK(hipMemcpy(host.data(), base, used, hipMemcpyDeviceToHost));
  w.bytes(host.data(), used);
  // optional sections, each preceded by its length
  auto section = [&](auto& part) {
    std::vector<uint8_t> sec;
    part->append_image(sec);
    w.put<uint64_t>(sec.size());
    w.bytes(sec.data(), sec.size());
  };
  if (voc_) section(voc_);
  if (gpt_) section(gpt_);
  std::vector<uint8_t> head;
  ImageWriter h{head};
  h.bytes(kImageMagic, 8);
  h.put<uint32_t>(kImageVersion);
  h.put<uint32_t>((voc_ ? kImageVocoder : 0u) | (gpt_ ? kImageGpt : 0u));
  h.put<uint64_t>(payload.size());
  h.put<uint64_t>(image_checksum(payload.data(), payload.size()));
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) throw std::invalid_argument("device image: cannot write " + path);
  f.write(reinterpret_cast<const char*>(head.data()), (std::streamsize)head.size());
  f.write(reinterpret_cast<const char*>(payload.data()), (std::streamsize)payload.size());
  if (!f) throw std::runtime_error("device image: write failed: " + path);
}

Engine::Engine(const std::string& image_path, int device) : device_(device) {
  std::ifstream f(image_path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("device image: cannot open " + image_path);
  const size_t total = (size_t)f.tellg();
  f.seekg(0);
  std::vector<uint8_t> file(total);
  if (!f.read(reinterpret_cast<char*>(file.data()), (std::streamsize)total))
    throw std::runtime_error("device image: cannot read " + image_path);
  ImageReader h{file.data(), file.size()};
  if (std::memcmp(h.bytes(8), kImageMagic, 8) != 0) throw std::runtime_error("device image: bad magic");
  if (h.get<uint32_t>() != kImageVersion) throw std::runtime_error("device image: unsupported version");
  const uint32_t sections = h.get<uint32_t>();
  if (sections & ~(kImageVocoder | kImageGpt)) throw std::runtime_error("device image: unknown sections");
  const uint64_t plen = h.get<uint64_t>();
  const uint64_t sum = h.get<uint64_t>();
  const uint8_t* payload = h.bytes(plen);
  if (h.at != file.size()) throw std::runtime_error("device image: trailing bytes");
  if (image_checksum(payload, plen) != sum) throw std::runtime_error("device image: checksum mismatch");

  HIP_OK(hipSetDevice(device_));
  resolve_scratch(device_);
  HIP_OK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  try {
    if (const char* g = std::getenv("MIT2CFM_GRAPH")) use_graph_ = std::atoi(g) != 0;
    ImageReader r{payload, plen};
    w_ = std::make_unique<Weights>();
    Weights& W = *w_;
    const uint64_t used = r.get<uint64_t>();
    if (used == 0 || used > (uint64_t(8) << 30)) throw std::runtime_error("device image: bad arena size");
    const uint8_t lr_mode = r.get<uint8_t>();
    if (lr_mode > 2) throw std::runtime_error("device image: bad length-regulator mode");
    W.has_lr = lr_mode != 0;
    W.lr_wsplit = lr_mode == 2 ? 2 : 1;
    W.arena.reserve(used);
    W.arena.set_used(used);
    char* base = W.arena.base();
    visit_weights(W, [&](auto*& p, size_t n) {
      using T = std::remove_pointer_t<std::remove_reference_t<decltype(p)>>;
      const uint64_t off = r.get<uint64_t>();
      p = off == UINT64_MAX ? nullptr : arena_span<T>(off, n, base, used);
    });
    // Arrays every decode reads must be present; the length regulator's all or none.
    bool ok = W.proj_w && W.wnc_w && W.cp_w && W.mc_w && W.sl_w && W.post_w && W.c2f_w;
    for (int l = 0; l < 13; ++l)
      ok = ok && W.qkv_w[l] && W.w13_w[l] && W.w2_w[l] && (l <= 6 || (W.si_w[l] && W.fold_w[l]));
    for (int l = 0; l < 8; ++l) ok = ok && W.in_w[l] && W.rs_w[l];
    ok = ok && (!W.has_lr || (W.lr_proj_w && W.lr_out_w && W.lr_conv_w[3] && W.lr_gn_b[3]));
    if (!ok) throw std::runtime_error("device image: missing decoder arrays");
    HIP_OK(hipMemcpy(base, r.bytes(used), used, hipMemcpyHostToDevice));
    if (sections & kImageVocoder) {
      const uint64_t n = r.get<uint64_t>();
      voc_ = std::make_unique<Vocoder>(r.bytes(n), n, stream_);
    }
    if (sections & kImageGpt) {
      const uint64_t n = r.get<uint64_t>();
      gpt_ = std::make_unique<GptDecoder>(r.bytes(n), n, stream_);
    }
    if (r.at != plen) throw std::runtime_error("device image: trailing bytes");
    ws_ = std::make_unique<Workspace>();
  } catch (...) {
    gpt_.reset();
    voc_.reset();
    w_.reset();
    (void)hipStreamDestroy(stream_);
    stream_ = nullptr;
    throw;
  }
}

Engine::~Engine() {
  clear_graphs();
  destroy_graphs(cond_graphs_);
  if (voc_io_) (void)hipFree(voc_io_);
  gpt_.reset();
  voc_.reset();
  ws_.reset();
  w_.reset();
  if (stream_) (void)hipStreamDestroy(stream_);
}

size_t Engine::weight_bytes() const {
  return w_->arena.used() + (voc_ ? voc_->weight_bytes() : 0) + (gpt_ ? gpt_->weight_bytes() : 0);
}

GptDecoder& Engine::gpt() {
  if (!gpt_) throw std::runtime_error("gpt: the context has no gpt.gpt.h.* tensors");
  HIP_OK(hipSetDevice(device_));
  return *gpt_;
}

template <typename Map>
void Engine::destroy_graphs(Map& graphs) {
  for (auto& kv : graphs) {
    if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
    if (kv.second.graph) (void)hipGraphDestroy(kv.second.graph);
  }
  graphs.clear();
}

void Engine::clear_graphs() { destroy_graphs(graphs_); }

template <typename Key, typename F>
void Engine::run_graph(std::map<Key, GraphEntry>& graphs, const Key& key, F&& enqueue) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIP_OK(hipStreamIsCapturing(stream_, &cs));
  if (!use_graph_ || cs != hipStreamCaptureStatusNone) {
    enqueue();
    return;
  }
  auto it = graphs.find(key);
  if (it == graphs.end()) {
    if (graphs.size() >= kMaxGraphs) {
      // Evict the least recently used graph.  Launches already enqueued on
      // the stream may still read its executable, so wait for them first
      // (a new shape pays a capture anyway).
      auto lru = graphs.begin();
      for (auto g = graphs.begin(); g != graphs.end(); ++g)
        if (g->second.last_use < lru->second.last_use) lru = g;
      HIP_OK(hipStreamSynchronize(stream_));
      (void)hipGraphExecDestroy(lru->second.exec);
      (void)hipGraphDestroy(lru->second.graph);
      graphs.erase(lru);
    }
    GraphEntry ge;
    HIP_OK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    try {
      enqueue();
    } catch (...) {
      hipGraph_t g = nullptr;
      (void)hipStreamEndCapture(stream_, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    HIP_OK(hipStreamEndCapture(stream_, &ge.graph));
    const hipError_t ie = hipGraphInstantiate(&ge.exec, ge.graph, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
      (void)hipGraphDestroy(ge.graph);
      throw HipError(std::string("hipGraphInstantiate failed: ") + hipGetErrorString(ie));
    }
    it = graphs.emplace(key, ge).first;
  }
  it->second.last_use = ++use_tick_;
  HIP_OK(hipGraphLaunch(it->second.exec, stream_));
}

void Engine::sync() { HIP_OK(hipStreamSynchronize(stream_)); }

void Engine::ensure_workspace(int B, int T, int S, int nreq) {
  Workspace& ws = *ws_;
  const int R = B * T;
  const int Tpad = (T + 63) / 64 * 64;
  if (R <= ws.capR && T <= ws.capT && Tpad <= ws.capTpad && B <= ws.capB && S <= ws.capS &&
      nreq <= ws.capReq) {
    return;
  }
  HIP_OK(hipStreamSynchronize(stream_));
  clear_graphs();
  const int cR = std::max(R, ws.capR), cT = std::max(T, ws.capT), cB = std::max(B, ws.capB);
  const int cTpad = std::max(Tpad, ws.capTpad), cS = std::max(S, ws.capS);
  const int cReq = std::max(nreq, ws.capReq);
  const int cRpad = cB * cTpad;  // rows of the head-major Q/K/V^T buffers
  const size_t r = (size_t)cR;
  size_t bytes = 0;
  auto f = [&](size_t n) { bytes += ((n * 4) + 255) / 256 * 256; };
  auto h = [&](size_t n) { bytes += ((n * 2) + 255) / 256 * 256; };
  f((size_t)cReq * cT * 80); h(r * kMelPad); h(r * 512); h(r * kMcWidth); f(r * 512); f(r * 512); f(r * 512);
  for (int i = 0; i < 6; ++i) h(r * 512);
  h(r * 512); h(r * 512);
  h((size_t)cRpad * 512); h((size_t)cRpad * 512); h((size_t)cRpad * 512);
  h(r * 512); h(r * kHgLd); h(r * 512);
  f(r * 512); h(r * 512); f(r * 512); f(r * 512); h(r * 512); f(r * 512);
  bytes += (r * 4 + 255) / 256 * 256 + ((size_t)cReq * 4 + 255) / 256 * 256;
  f((size_t)cRpad + cB);
  f((size_t)cT * 64);
  f(cS); f((size_t)cS * 256); f((size_t)cS * 512); f((size_t)cS * 512); f((size_t)cS * 512);
  f((size_t)cS * kTcondPerStep);
  f(r * kSsqParts); f((size_t)cS * 13 * 1536); f((size_t)cS * 13 * 3072);
  f(r * 80); f(r * 80); f(r * 512); f((size_t)cB * 192); f(r * 80); f(r * 80);
  f(r * 1024); f(r * 1024); f(r * 1024);
  bytes += 64 * 256;

  ws.arena.reserve(bytes);
  Arena& a = ws.arena;
  auto F = [&](size_t n) { return static_cast<float*>(a.take(n * 4)); };
  auto H = [&](size_t n) { return static_cast<half_t*>(a.take(n * 2)); };
  ws.x_cur = F((size_t)cReq * cT * 80);
  ws.xmel16 = H(r * kMelPad);
  ws.cond16 = H(r * 512);
  ws.mc16 = H(r * kMcWidth);
  ws.xin_const = F(r * 512);
  ws.xa = F(r * 512);
  ws.xb = F(r * 512);
  for (int i = 0; i < 6; ++i) ws.skip16[i] = H(r * 512);
  ws.x16 = H(r * 512);
  ws.n16 = H(r * 512);
  ws.q = H((size_t)cRpad * 512);
  ws.k = H((size_t)cRpad * 512);
  ws.vt = H((size_t)cRpad * 512);
  ws.o16 = H(r * 512);
  ws.hg16 = H(r * kHgLd);
  ws.g16 = ws.hg16 + 512;
  ws.ls16 = H(r * 512);
  ws.wn_x = F(r * 512);
  ws.wn_x16 = H(r * 512);
  ws.rp = F(r * 512);
  ws.wn_out = F(r * 512);
  ws.gate16 = H(r * 512);
  ws.fin = F(r * 512);
  ws.mask = static_cast<uint32_t*>(a.take(r * 4));
  ws.kbias = F((size_t)cRpad + cB);
  ws.P = static_cast<uint32_t*>(a.take((size_t)cReq * 4));
  ws.rope = reinterpret_cast<float2*>(F((size_t)cT * 64));
  ws.tvals = F(cS);
  ws.temb = F((size_t)cS * 256);
  ws.th = F((size_t)cS * 512);
  ws.t1 = F((size_t)cS * 512);
  ws.t2 = F((size_t)cS * 512);
  ws.tab = F((size_t)cS * kTcondPerStep);
  ws.ssq = F(r * kSsqParts);
  ws.nbq = F((size_t)cS * 13 * 1536);
  ws.nbw = F((size_t)cS * 13 * 3072);
  ws.in_x = F(r * 80);
  ws.in_prompt = F(r * 80);
  ws.in_cond = F(r * 512);
  ws.in_style = F((size_t)cB * 192);
  ws.out_x = F(r * 80);
  ws.dphi = F(r * 80);
  ws.stage_a = F(r * 1024);
  ws.stage_b = F(r * 1024);
  ws.stage_c = F(r * 1024);
  // Everything starts finite (the attention tiles read padding rows of K/V^T).
  HIP_OK(hipMemsetAsync(ws.x_cur, 0, a.used(), stream_));  // x_cur is the arena's first slice
  HIP_OK(hipStreamSynchronize(stream_));
  ws.capR = cR; ws.capT = cT; ws.capTpad = cTpad; ws.capB = cB; ws.capS = cS; ws.capReq = cReq;
  ws.Tcur = 0;
  ws.mask_host.clear();
  ws.P_host.clear();
}

// RoPE table [T][32] of (cos, sin), theta = t / 10000^(2i/64)
// (tokenizer_tests.cpp:4266-4281 apply_rope_inplace).
static std::vector<float> rope_table(int T) {
  std::vector<float> r((size_t)T * 64);
  for (int t = 0; t < T; ++t)
    for (int pair = 0; pair < 32; ++pair) {
      const float theta = (float)t / std::pow(10000.0f, (float)(pair * 2) / 64.0f);
      r[(size_t)t * 64 + pair * 2] = std::cos(theta);
      r[(size_t)t * 64 + pair * 2 + 1] = std::sin(theta);
    }
  return r;
}

void Engine::ensure_rope(int T) {
  Workspace& ws = *ws_;
  if (ws.Tcur == T) return;
  auto rt = rope_table(T);
  HIP_OK(hipMemcpyAsync(ws.rope, rt.data(), rt.size() * 4, hipMemcpyHostToDevice, stream_));
  HIP_OK(hipStreamSynchronize(stream_));
  ws.Tcur = T;
}

// ------------------------------------------------------------------ tables
static std::vector<float> euler_times(int steps) {
  std::vector<float> tv(steps);
  float t = 0.0f;
  const float dt = 1.0f / (float)steps;
  for (int s = 0; s < steps; ++s) {
    tv[s] = t;
    t += dt;  // accumulated in float like run_cfm_euler_cpu
  }
  return tv;
}

void Engine::enqueue_tables(const TableBufs& tb, int S) {
  Weights& W = *w_;
  for (int i = 0; i < 2; ++i) {
    float* out = i == 0 ? tb.t1 : tb.t2;
    HIP_OK(launch_timestep_embedding(tb.tvals, W.te_freqs[i], S, tb.temb, stream_));
    HIP_OK(launch_linear_small(tb.temb, S, 256, W.te_w0[i], W.te_b0[i], 512, 0, 1, tb.th, 512, stream_));
    HIP_OK(launch_linear_small(tb.th, S, 512, W.te_w2[i], W.te_b2[i], 512, 0, 0, out, 512, stream_));
  }
  HIP_OK(launch_linear_small(tb.t1, S, 512, W.proj_w, W.proj_b, 27 * 1024, 0, 0, tb.tab,
                             kTcondPerStep, stream_));
  HIP_OK(launch_linear_small(tb.t1, S, 512, W.ada_w, W.ada_b, 1024, 1, 0, tb.tab + kFinalSsOff,
                             kTcondPerStep, stream_));
  HIP_OK(launch_linear_small(tb.t2, S, 512, W.wnc_w, W.wnc_b, 8192, 0, 0, tb.tab + kWnCondOff,
                             kTcondPerStep, stream_));
  enqueue_norm_bias(tb, S);
}

// Column biases of the folded AdaRMSNorms (ab . W^T) for every layer and
// step slot of tb.tab.
void Engine::enqueue_norm_bias(const TableBufs& tb, int S) {
  Weights& W = *w_;
  for (int l = 0; l < 13; ++l) {
    HIP_OK(launch_norm_bias(tb.tab + l * 1024 + 512, kTcondPerStep, S, W.qkv_w[l], 1536,
                            tb.nbq + l * 1536, 13 * 1536, stream_));
    HIP_OK(launch_norm_bias(tb.tab + (13 + l) * 1024 + 512, kTcondPerStep, S, W.w13_w[l], 3072,
                            tb.nbw + l * 3072, 13 * 3072, stream_));
  }
}

// The tables of a `steps`-step Euler decode (t = 0, dt, 2 dt, ... accumulated
// in fp32).  They depend only on the step count, so each context computes
// them once per count, outside any captured graph, and every later decode
// reads them: the reference caches the same tables per step count in a
// process-wide map (dit_cfm_bigvgan.cpp:2954-2959); here the cache is per
// context, so it needs no lock.
const TableBufs& Engine::decode_tables(int steps) {
  auto it = table_cache_.find(steps);
  if (it != table_cache_.end()) return it->second->bufs;
  auto set = std::make_unique<TableSet>();
  const size_t S = (size_t)steps;
  size_t bytes = 0;
  const size_t counts[8] = {S, S * 256, S * 512, S * 512, S * 512, S * kTcondPerStep, S * 13 * 1536,
                            S * 13 * 3072};
  for (size_t c : counts) bytes += (c * 4 + 255) / 256 * 256;
  set->arena.reserve(bytes);
  auto F = [&](size_t n) { return static_cast<float*>(set->arena.take(n * 4)); };
  TableBufs& tb = set->bufs;
  tb.tvals = F(counts[0]); tb.temb = F(counts[1]); tb.th = F(counts[2]); tb.t1 = F(counts[3]);
  tb.t2 = F(counts[4]); tb.tab = F(counts[5]); tb.nbq = F(counts[6]); tb.nbw = F(counts[7]);
  const std::vector<float> tv = euler_times(steps);
  HIP_OK(hipMemcpyAsync(tb.tvals, tv.data(), tv.size() * 4, hipMemcpyHostToDevice, stream_));
  enqueue_tables(tb, steps);
  HIP_OK(hipStreamSynchronize(stream_));  // tv outlives the copy
  return table_cache_.emplace(steps, std::move(set)).first->second->bufs;
}

// One transformer block (dit_cfm_bigvgan.cpp:816-832 / pass version :1901-1996):
//   [l > 6] x = skip_in([x | skip]);  h = x + wo . Attn(RoPE(wqkv . AdaRMS(x)));
//   out = h + w2 . SwiGLU(w13 . AdaRMS(h)).
// Both AdaRMSNorms are folded into GEMM pairs (see GemmArgs): the GEMM that
// produces a normed row block also writes ws.n16 = f16(x * aw * gamma) and
// the row's partial sums of squares ws.ssq; the QKV / w13 GEMM scales by
// rs and adds ab . W^T (nbq / nbw, this step's slot).
// cur holds x on entry and out on exit (fp32).  On entry ws.n16 / ws.ssq
// hold block l's attention-norm operand when l <= 6 (written by the merge
// GEMM or block l-1); x16 must hold f16(x) when l > 6.  out16 receives
// f16(out); for l < 6 the w2 GEMM also leaves block l+1's operand.
// Within the stack, a block l in 6..11 is followed by block l+1's skip-in,
// which is linear in out = h + w2 . g: given next_skip16 (block l+1's skip
// input), the w2 GEMM is replaced by that skip-in over [f16(h) | g | skip]
// with the folded weight (Weights::fold_w), so cur leaves as block l+1's x
// with its attention-norm operand, and block l+1 runs with skip_in_done.
void Engine::enqueue_layer(int l, int B, int T, const float* tab, const float* nbq,
                           const float* nbw, float* cur, float* hbuf, const half_t* skip16,
                           half_t* out16, bool skip_in_done, const half_t* next_skip16) {
  Weights& W = *w_;
  Workspace& ws = *ws_;
  hipStream_t s = stream_;
  const int R = B * T;
  const int Tpad = (T + 63) / 64 * 64;
  auto norm_out = [&](GemmArgs& g, int norm_id) {
    g.C16s = ws.n16; g.ldc16s = 512;
    g.sc_a = tab + norm_id * 1024; g.sc_g = W.gamma[norm_id];
    g.ssq_out = ws.ssq;
  };
  if (l > 6 && !skip_in_done) {
    GemmArgs g;
    g.M = R; g.N = 512; g.K = 1024; g.K1 = 512;
    g.A = ws.x16; g.lda = 512; g.A2 = skip16; g.lda2 = 512;
    g.W = W.si_w[l]; g.ldw = 1024; g.bias = W.si_b[l]; g.colperm = 1;
    g.C32 = cur; g.ldc32 = 512;
    norm_out(g, l);
    apply_rows(row_skip_, g);
    HIP_OK(launch_gemm(g, A_CONCAT, EPI_F32, s));
  }
  {
    GemmArgs g;
    g.M = R; g.N = 1536; g.K = 512; g.A = ws.n16; g.lda = 512;
    g.W = W.qkv_w[l]; g.ldw = 512; g.T = T;
    g.bias = nbq + l * 1536; g.ssq_in = ws.ssq;
    g.rope = ws.rope; g.q = ws.q; g.k = ws.k; g.vt = ws.vt; g.Tpad = Tpad;
    apply_rows(row_skip_, g);
    HIP_OK(launch_gemm(g, A_PLAIN, EPI_QKV, s));
  }
  HIP_OK(launch_attention(ws.q, ws.k, ws.vt, ws.kbias, ws.o16, B, T, Tpad, s, branch_keys_,
                          row_skip_.nb > 0));
  {
    GemmArgs g;
    g.M = R; g.N = 512; g.K = 512; g.A = ws.o16; g.lda = 512;
    g.W = W.wo_w[l]; g.ldw = 512; g.res = cur; g.ldres = 512; g.colperm = 1;
    if (next_skip16) {
      g.C16 = ws.hg16; g.ldc16 = kHgLd;  // h is read only by the folded skip-in, in f16
    } else {
      g.C32 = hbuf; g.ldc32 = 512;
    }
    norm_out(g, 13 + l);
    apply_rows(row_skip_, g);
    HIP_OK(launch_gemm(g, A_PLAIN, EPI_F32, s));
  }
  {
    GemmArgs g;
    g.M = R; g.N = 3072; g.K = 512; g.A = ws.n16; g.lda = 512;
    g.W = W.w13_w[l]; g.ldw = 512; g.C16 = ws.g16; g.ldc16 = kHgLd;
    g.bias = nbw + l * 3072; g.ssq_in = ws.ssq;
    apply_rows(row_skip_, g);
    HIP_OK(launch_gemm(g, A_PLAIN, EPI_SWIGLU, s));
  }
  if (next_skip16) {
    GemmArgs g;
    g.M = R; g.N = 512; g.K = 2560; g.K1 = kHgLd;
    g.A = ws.hg16; g.lda = kHgLd; g.A2 = next_skip16; g.lda2 = 512;
    g.W = W.fold_w[l + 1]; g.ldw = 2560; g.bias = W.si_b[l + 1]; g.colperm = 1;
    g.C32 = cur; g.ldc32 = 512;
    norm_out(g, l + 1);
    apply_rows(row_skip_, g);
    HIP_OK(launch_gemm(g, A_CONCAT, EPI_F32, s));
  } else {
    GemmArgs g;
    g.M = R; g.N = 512; g.K = 1536; g.A = ws.g16; g.lda = kHgLd;
    g.W = W.w2_w[l]; g.ldw = 1536; g.res = hbuf; g.ldres = 512; g.colperm = 1;
    g.C32 = cur; g.ldc32 = 512; g.C16 = out16; g.ldc16 = 512;
    if (l < 6) norm_out(g, l + 1);
    apply_rows(row_skip_, g);
    HIP_OK(launch_gemm(g, A_PLAIN, EPI_F32, s));
  }
}

// The 13-block U-ViT stack (dit_cfm_bigvgan.cpp:868-886): outputs of blocks
// 0..5 are kept (f16) as the skip inputs of blocks 12..7; the final AdaRMSNorm
// leaves f16(norm(x)) in ws.n16.  x enters in ws.xa, with block 0's folded
// norm operand in ws.n16 / ws.ssq.
void Engine::enqueue_transformer(int B, int T, const float* tab, const float* nbq,
                                 const float* nbw) {
  Weights& W = *w_;
  Workspace& ws = *ws_;
  for (int l = 0; l < 13; ++l)
    enqueue_layer(l, B, T, tab, nbq, nbw, ws.xa, ws.xb, l > 6 ? ws.skip16[12 - l] : nullptr,
                  l < 6 ? ws.skip16[l] : ws.x16, l > 6,
                  l >= 6 && l < 12 ? ws.skip16[11 - l] : nullptr);
  HIP_OK(launch_adarms(ws.xa, W.gamma[26], tab + 26 * 1024, tab + 26 * 1024 + 512, ws.n16, B * T,
                       stream_));
}

// ------------------------------------------------------------------ estimator body
// Runs the estimator from x (ws.xa, fp32, already merged) to the final
// layer's AdaLN output (ws.n16, f16) for B branches of T rows, using one
// step's tables; the caller applies the folded final linear + conv2.
void Engine::enqueue_estimator(int B, int T, const float* tab, const float* nbq, const float* nbw) {
  Weights& W = *w_;
  Workspace& ws = *ws_;
  const int R = B * T;
  hipStream_t s = stream_;

  enqueue_transformer(B, T, tab, nbq, nbw);
  {
    // conv1 | res_projection of skip_linear([x_normed | x_mel]) as one product
    GemmArgs g;
    g.M = R; g.N = 1024; g.K = 512 + kMelPad; g.K1 = 512;
    g.A = ws.n16; g.lda = 512; g.A2 = ws.xmel16; g.lda2 = kMelPad;
    g.W = W.post_w; g.ldw = 512 + kMelPad; g.bias = W.post_b;
    g.C32 = ws.wn_x; g.ldc32 = 512; g.C16 = ws.wn_x16; g.ldc16 = 512;
    g.C32b = ws.rp; g.ldc32b = 512;
    apply_rows(row_skip_, g);
    HIP_OK(launch_gemm(g, A_CONCAT, EPI_DUAL, s));
  }
  for (int l = 0; l < 8; ++l) {
    {
      GemmArgs g;
      g.M = R; g.N = 1024; g.K = 2560; g.A = ws.wn_x16; g.lda = 512; g.T = T; g.conv_c = 512;
      g.W = W.in_w[l]; g.ldw = 2560; g.bias = W.in_b[l]; g.cond = tab + kWnCondOff + l * 1024;
      g.C16 = ws.gate16; g.ldc16 = 512;
      apply_rows(row_skip_, g);
      HIP_OK(launch_gemm(g, A_CONV5, EPI_GATE, s));
    }
    GemmArgs g;
    g.M = R; g.K = 512; g.A = ws.gate16; g.lda = 512; g.W = W.rs_w[l]; g.ldw = 512;
    g.bias = W.rs_b[l]; g.mask = ws.mask;
    if (l < 7) {
      g.N = 1024; g.C32 = ws.wn_x; g.ldc32 = 512; g.C16 = ws.wn_x16; g.ldc16 = 512;
      g.C32b = ws.wn_out; g.ldc32b = 512; g.flag = l > 0;
      apply_rows(row_skip_, g);
      HIP_OK(launch_gemm(g, A_PLAIN, EPI_RESSKIP, s));
    } else {
      g.N = 512; g.C32b = ws.wn_out; g.ldc32b = 512; g.C32 = ws.fin; g.ldc32 = 512; g.rp = ws.rp;
      apply_rows(row_skip_, g);
      HIP_OK(launch_gemm(g, A_PLAIN, EPI_FINALSKIP, s));
    }
  }
  // The final layer's AdaLN output stays in ws.n16; its linear map is folded
  // into conv2 (W.c2f_w), which the caller applies.
  HIP_OK(launch_adaln(ws.fin, tab + kFinalSsOff, tab + kFinalSsOff + 512, ws.n16, R, s));
}

// Input merge constant part: cond projection into mc16[:, kMcContent:+512], then
// xin_const = mc16 . Wc^T + b_merge.
static void enqueue_merge_const(Weights& W, Workspace& ws, int R, hipStream_t s,
                                const RowSkip& rows = RowSkip()) {
  GemmArgs g;
  g.M = R; g.N = 512; g.K = 512; g.A = ws.cond16; g.lda = 512;
  g.W = W.cp_w; g.ldw = 512; g.bias = W.cp_b; g.C16 = ws.mc16 + kMcContent; g.ldc16 = kMcWidth;
  apply_rows(rows, g);
  HIP_OK(launch_gemm(g, A_PLAIN, EPI_F16, s));
  GemmArgs c;
  c.M = R; c.N = 512; c.K = kMcWidth; c.A = ws.mc16; c.lda = kMcWidth;
  c.W = W.mc_w; c.ldw = kMcWidth; c.bias = W.mc_b; c.C32 = ws.xin_const; c.ldc32 = 512;
  apply_rows(rows, c);
  HIP_OK(launch_gemm(c, A_PLAIN, EPI_F32, s));
}

// Per-step merge: x = xin_const + xmel16 . Wx^T.  With tab (the step's
// table row) it also leaves block 0's folded attention-norm operand in
// ws.n16 / ws.ssq.
static void enqueue_merge_step(Weights& W, Workspace& ws, int R, hipStream_t s,
                               const float* tab, const RowSkip& rows = RowSkip()) {
  GemmArgs g;
  g.M = R; g.N = 512; g.K = kMelPad; g.A = ws.xmel16; g.lda = kMelPad;
  g.W = W.mx_w; g.ldw = kMelPad; g.res = ws.xin_const; g.ldres = 512; g.C32 = ws.xa; g.ldc32 = 512;
  g.colperm = 1;
  if (tab) {
    g.C16s = ws.n16; g.ldc16s = 512; g.sc_a = tab; g.sc_g = W.gamma[0]; g.ssq_out = ws.ssq;
  }
  apply_rows(rows, g);
  HIP_OK(launch_gemm(g, A_PLAIN, EPI_F32, s));
}

void Engine::enqueue_decode(const float* x0, const float* prompt, const float* cond,
                            const float* style, int nreq, int T, int steps, float cfg,
                            float* vtrace, const TableBufs& tb) {
  Weights& W = *w_;
  Workspace& ws = *ws_;
  const int cfg_on = cfg > 0.0f ? 1 : 0;
  const int B = cfg_on ? 2 * nreq : nreq;
  const int R = B * T;
  const float dt = 1.0f / (float)steps;
  HIP_OK(launch_decode_prep(x0, prompt, cond, style, ws.P, nreq, T, cfg_on, ws.x_cur, ws.xmel16,
                            ws.cond16, ws.mc16, stream_));
  HIP_OK(launch_key_bias(ws.mask, B, T, (T + 63) / 64 * 64, ws.kbias, stream_));
  enqueue_merge_const(W, ws, R, stream_, row_skip_);
  for (int s = 0; s < steps; ++s) {
    const float* tab = tb.tab + (size_t)s * kTcondPerStep;
    enqueue_merge_step(W, ws, R, stream_, tab, row_skip_);
    enqueue_estimator(B, T, tab, tb.nbq + (size_t)s * 13 * 1536, tb.nbw + (size_t)s * 13 * 3072);
    HIP_OK(launch_conv2_euler(ws.n16, W.c2f_w, W.c2f_b, ws.P, nreq, T, cfg_on, cfg, dt, ws.x_cur,
                              ws.xmel16, vtrace ? vtrace + (size_t)s * nreq * T * 80 : nullptr,
                              stream_));
  }
}

void Engine::decode_device(const float* x0, const float* prompt, const float* cond,
                           const float* style, int nreq, int T, const uint32_t* valid_T,
                           const uint32_t* P, int steps, float cfg, float* x_out, float* vtrace) {
  if (nreq <= 0 || T <= 0 || steps <= 0 || !(cfg >= 0.0f))
    throw std::invalid_argument("decode: nreq, T and steps must be positive and cfg_rate >= 0");
  for (int r = 0; r < nreq; ++r) {
    if (valid_T[r] == 0 || valid_T[r] > (uint32_t)T)
      throw std::invalid_argument("decode: each request needs 1 <= valid length <= T");
    if (P[r] > valid_T[r]) throw std::invalid_argument("decode: prompt longer than the request");
  }
  HIP_OK(hipSetDevice(device_));
  const int cfg_on = cfg > 0.0f ? 1 : 0;
  const int B = cfg_on ? 2 * nreq : nreq;
  ensure_workspace(B, T, 1, nreq);
  last_B_ = B;
  last_T_ = T;
  Workspace& ws = *ws_;
  ensure_rope(T);
  const TableBufs& tb = decode_tables(steps);
  {
    // Key mask and prompt lengths: uploaded only when they differ from what
    // the workspace already holds, so back-to-back decodes of one shape never
    // wait for the device here.
    std::vector<uint32_t> mask((size_t)B * T);
    for (int b = 0; b < B; ++b) {
      const int r = cfg_on ? b / 2 : b;
      for (int t = 0; t < T; ++t) mask[(size_t)b * T + t] = (uint32_t)t < valid_T[r] ? 1u : 0u;
    }
    std::vector<uint32_t> pv(P, P + nreq);
    if (mask != ws.mask_host || pv != ws.P_host) {
      HIP_OK(hipMemcpyAsync(ws.mask, mask.data(), mask.size() * 4, hipMemcpyHostToDevice, stream_));
      HIP_OK(hipMemcpyAsync(ws.P, pv.data(), pv.size() * 4, hipMemcpyHostToDevice, stream_));
      HIP_OK(hipStreamSynchronize(stream_));  // the host vectors outlive the copies
      ws.mask_host = std::move(mask);
      ws.P_host = std::move(pv);
    }
  }

  // A batch with a request shorter than T lets the attention skip each
  // branch's key tiles after its last valid key (a different graph than a
  // full-length batch of the same shape; either is correct for both).
  bool ragged = false;
  for (int r = 0; r < nreq; ++r) ragged = ragged || valid_T[r] < (uint32_t)T;
  // With skipped padding each branch's rows are needed up to two past its
  // valid length: the k=5 WaveNet conv at the last valid rows reads them
  // (layer 0's input there is the transformer's output, not masked).
  RowSkip rows;
  const bool skip = skip_padding_ && ragged && B <= kMaxRowSeq;
  if (skip) {
    rows.T = T;
    rows.nb = B;
    for (int b = 0; b < B; ++b) rows.need[b] = std::min<int>(T, (int)valid_T[cfg_on ? b / 2 : b] + 2);
  }
  // The Euler state lives in ws.x_cur; x_out receives a copy at the end.
  auto enqueue_all = [&]() {
    branch_keys_ = ragged;
    row_skip_ = rows;
    try {
      enqueue_decode(x0, prompt, cond, style, nreq, T, steps, cfg, vtrace, tb);
    } catch (...) {
      branch_keys_ = false;
      row_skip_ = RowSkip();
      throw;
    }
    branch_keys_ = false;
    row_skip_ = RowSkip();
    HIP_OK(launch_copy_f32(ws.x_cur, x_out, (size_t)nreq * T * 80, stream_));
  };
  uint32_t cfg_bits;
  std::memcpy(&cfg_bits, &cfg, 4);
  auto key = std::make_tuple(nreq, T, steps, cfg_bits, (const void*)vtrace, (const void*)x0,
                             (const void*)prompt, (const void*)cond, (const void*)style,
                             (const void*)x_out, ragged, skip);
  run_graph(graphs_, key, enqueue_all);
}

void Engine::estimator_step_device(const float* x, const float* prompt_x, const float* cond,
                                   const float* style, const uint32_t* mask, float t, int B, int T,
                                   float* dphi) {
  if (B <= 0 || T <= 0) throw std::invalid_argument("estimator_step: B and T must be positive");
  HIP_OK(hipSetDevice(device_));
  ensure_workspace(B, T, 1, 1);
  Workspace& ws = *ws_;
  Weights& W = *w_;
  const int R = B * T;
  ensure_rope(T);
  HIP_OK(hipMemcpyAsync(ws.mask, mask, (size_t)R * 4, hipMemcpyDeviceToDevice, stream_));
  ws.mask_host.clear();
  HIP_OK(launch_key_bias(ws.mask, B, T, (T + 63) / 64 * 64, ws.kbias, stream_));
  HIP_OK(hipMemcpyAsync(ws.tvals, &t, 4, hipMemcpyHostToDevice, stream_));
  HIP_OK(hipStreamSynchronize(stream_));
  enqueue_tables(ws.one(), 1);
  HIP_OK(launch_step_prep(x, prompt_x, cond, style, B, T, ws.xmel16, ws.cond16, ws.mc16, stream_));
  enqueue_merge_const(W, ws, R, stream_);
  enqueue_merge_step(W, ws, R, stream_, ws.tab);
  enqueue_estimator(B, T, ws.tab, ws.nbq, ws.nbw);
  HIP_OK(launch_conv2_rows(ws.n16, W.c2f_w, W.c2f_b, R, dphi, stream_));
  HIP_OK(hipStreamSynchronize(stream_));
}

// ------------------------------------------------------------------ profiling hook
void Engine::profile_launch(int kernel, int count, double* flops, double* bytes, std::string* name) {
  if (last_B_ == 0) throw std::invalid_argument("profile_launch: run a decode first");
  const int B = last_B_, T = last_T_, R = B * T;
  const int Tpad = (T + 63) / 64 * 64;
  Weights& W = *w_;
  Workspace& ws = *ws_;
  const float* tab = ws.tab;
  double f = 0, by = 0;
  std::string nm;
  auto loop = [&](auto&& launch) {
    for (int i = 0; i < count; ++i) launch();
  };
  switch (kernel) {
    case 0: {  // FFN w1|w3 GEMM + SwiGLU (N = 3072, K = 512)
      GemmArgs g;
      g.M = R; g.N = 3072; g.K = 512; g.A = ws.n16; g.lda = 512;
      g.W = W.w13_w[0]; g.ldw = 512; g.C16 = ws.g16; g.ldc16 = kHgLd;
      g.bias = ws.nbw; g.ssq_in = ws.ssq;
      loop([&] { HIP_OK(launch_gemm(g, A_PLAIN, EPI_SWIGLU, stream_)); });
      f = 2.0 * R * 3072 * 512;
      by = 2.0 * R * 512 + 2.0 * 3072 * 512 + 2.0 * R * 1536;
      nm = "gemm_w13_swiglu";
      break;
    }
    case 1: {  // WaveNet k=5 conv as implicit GEMM + gate (N = 1024, K = 2560)
      GemmArgs g;
      g.M = R; g.N = 1024; g.K = 2560; g.A = ws.wn_x16; g.lda = 512; g.T = T; g.conv_c = 512;
      g.W = W.in_w[0]; g.ldw = 2560; g.bias = W.in_b[0]; g.cond = tab + kWnCondOff;
      g.C16 = ws.gate16; g.ldc16 = 512;
      loop([&] { HIP_OK(launch_gemm(g, A_CONV5, EPI_GATE, stream_)); });
      f = 2.0 * R * 1024 * 2560;
      by = 2.0 * R * 512 + 2.0 * 1024 * 2560 + 2.0 * R * 512;
      nm = "gemm_wavenet_conv_gate";
      break;
    }
    case 2: {  // QKV GEMM + RoPE (N = 1536, K = 512)
      GemmArgs g;
      g.M = R; g.N = 1536; g.K = 512; g.A = ws.n16; g.lda = 512; g.W = W.qkv_w[0]; g.ldw = 512;
      g.T = T; g.rope = ws.rope; g.q = ws.q; g.k = ws.k; g.vt = ws.vt; g.Tpad = Tpad;
      g.bias = ws.nbq; g.ssq_in = ws.ssq;
      loop([&] { HIP_OK(launch_gemm(g, A_PLAIN, EPI_QKV, stream_)); });
      f = 2.0 * R * 1536 * 512;
      by = 2.0 * R * 512 + 2.0 * 1536 * 512 + 2.0 * R * 1536;
      nm = "gemm_qkv_rope";
      break;
    }
    case 3: {  // FFN w2 GEMM + residual (N = 512, K = 1536)
      GemmArgs g;
      g.M = R; g.N = 512; g.K = 1536; g.A = ws.g16; g.lda = kHgLd; g.W = W.w2_w[0]; g.ldw = 1536;
      g.colperm = 1;
      g.res = ws.xb; g.ldres = 512; g.C32 = ws.stage_a; g.ldc32 = 512;
      loop([&] { HIP_OK(launch_gemm(g, A_PLAIN, EPI_F32, stream_)); });
      f = 2.0 * R * 512 * 1536;
      by = 2.0 * R * 1536 + 2.0 * 512 * 1536 + 8.0 * R * 512;
      nm = "gemm_w2_residual";
      break;
    }
    case 4: {  // masked flash attention
      loop([&] { HIP_OK(launch_attention(ws.q, ws.k, ws.vt, ws.kbias, ws.o16, B, T, Tpad, stream_)); });
      f = 4.0 * 64.0 * 8.0 * B * (double)T * (double)T;
      by = 2.0 * 3.0 * B * 8 * (double)T * 64 + 2.0 * R * 512 + 4.0 * R;
      nm = "attention";
      break;
    }
    case 5: {  // AdaRMSNorm row kernel
      loop([&] { HIP_OK(launch_adarms(ws.xa, W.gamma[0], tab, tab + 512, ws.n16, R, stream_)); });
      f = 0;
      by = 4.0 * R * 512 + 2.0 * R * 512 + 3.0 * 512 * 4;
      nm = "adarms";
      break;
    }
    case 6: {  // attention output projection wo + residual, folded-norm producer (N = K = 512)
      GemmArgs g;
      g.M = R; g.N = 512; g.K = 512; g.A = ws.o16; g.lda = 512;
      g.W = W.wo_w[0]; g.ldw = 512; g.res = ws.xa; g.ldres = 512; g.colperm = 1;
      g.C32 = ws.stage_a; g.ldc32 = 512;
      g.C16s = ws.n16; g.ldc16s = 512; g.sc_a = tab + 13 * 1024; g.sc_g = W.gamma[13];
      g.ssq_out = ws.ssq;
      loop([&] { HIP_OK(launch_gemm(g, A_PLAIN, EPI_F32, stream_)); });
      f = 2.0 * R * 512 * 512;
      by = 2.0 * R * 512 + 2.0 * 512 * 512 + 4.0 * R * 512 + 4.0 * R * 512 + 2.0 * R * 512 +
           4.0 * R * kSsqParts;
      nm = "gemm_wo_residual_norm";
      break;
    }
    case 7: {  // WaveNet res/skip k=1 GEMM with the masked update (N = 1024, K = 512)
      GemmArgs g;
      g.M = R; g.N = 1024; g.K = 512; g.A = ws.gate16; g.lda = 512; g.W = W.rs_w[0]; g.ldw = 512;
      g.bias = W.rs_b[0]; g.mask = ws.mask;
      g.C32 = ws.stage_a; g.ldc32 = 512; g.C16 = ws.x16; g.ldc16 = 512;
      g.C32b = ws.stage_b; g.ldc32b = 512; g.flag = 1;
      loop([&] { HIP_OK(launch_gemm(g, A_PLAIN, EPI_RESSKIP, stream_)); });
      f = 2.0 * R * 1024 * 512;
      by = 2.0 * R * 512 + 2.0 * 1024 * 512 + 4.0 * R * 512 * 2 + 4.0 * R * 512 * 2 +
           2.0 * R * 512 + 4.0 * R;
      nm = "gemm_wavenet_resskip";
      break;
    }
    default:
      throw std::invalid_argument("profile_launch: unknown kernel id");
  }
  if (flops) *flops = f;
  if (bytes) *bytes = by;
  if (name) *name = nm;
}

// ------------------------------------------------------------------ stages
namespace {
struct DevBuf {
  void* p = nullptr;
  explicit DevBuf(size_t bytes) { HIP_OK(hipMalloc(&p, bytes ? bytes : 4)); }
  ~DevBuf() { (void)hipFree(p); }
  template <typename T>
  T* as() const { return static_cast<T*>(p); }
};
void h2d(void* d, const void* h, size_t bytes, hipStream_t s) {
  HIP_OK(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s));
}
void d2h(void* h, const void* d, size_t bytes, hipStream_t s) {
  HIP_OK(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, s));
  HIP_OK(hipStreamSynchronize(s));
}
void to_f16(const float* in, half_t* out, size_t n, hipStream_t s) {
  HIP_OK(launch_f32_to_f16(in, out, n, 0, s));
}
}  // namespace

// Stage tables from explicit t1 / t2 vectors: row 0 of ws.tab.
void Engine::upload_stage_tables(const float* t1_host, const float* t2_host) {
  Weights& W = *w_;
  Workspace& ws = *ws_;
  if (t1_host) {
    h2d(ws.t1, t1_host, 512 * 4, stream_);
    HIP_OK(launch_linear_small(ws.t1, 1, 512, W.proj_w, W.proj_b, 27 * 1024, 0, 0, ws.tab,
                               kTcondPerStep, stream_));
    HIP_OK(launch_linear_small(ws.t1, 1, 512, W.ada_w, W.ada_b, 1024, 1, 0, ws.tab + kFinalSsOff,
                               kTcondPerStep, stream_));
    enqueue_norm_bias(ws.one(), 1);
  }
  if (t2_host) {
    h2d(ws.t2, t2_host, 512 * 4, stream_);
    HIP_OK(launch_linear_small(ws.t2, 1, 512, W.wnc_w, W.wnc_b, 8192, 0, 0, ws.tab + kWnCondOff,
                               kTcondPerStep, stream_));
  }
}

void Engine::stage_timestep_embedder(float t, int which, float* out512) {
  ensure_workspace(1, 1, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  const int i = which == 2 ? 1 : 0;
  h2d(ws.tvals, &t, 4, stream_);
  HIP_OK(launch_timestep_embedding(ws.tvals, W.te_freqs[i], 1, ws.temb, stream_));
  HIP_OK(launch_linear_small(ws.temb, 1, 256, W.te_w0[i], W.te_b0[i], 512, 0, 1, ws.th, 512, stream_));
  HIP_OK(launch_linear_small(ws.th, 1, 512, W.te_w2[i], W.te_b2[i], 512, 0, 0, ws.t1, 512, stream_));
  d2h(out512, ws.t1, 512 * 4, stream_);
}

void Engine::stage_input_merge(const float* x, const float* prompt_x, const float* cond,
                               const float* style, int B, int T, float* out) {
  ensure_workspace(B, T, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  const int R = B * T;
  h2d(ws.in_x, x, (size_t)R * 80 * 4, stream_);
  h2d(ws.in_prompt, prompt_x, (size_t)R * 80 * 4, stream_);
  h2d(ws.in_cond, cond, (size_t)R * 512 * 4, stream_);
  h2d(ws.in_style, style, (size_t)B * 192 * 4, stream_);
  HIP_OK(launch_step_prep(ws.in_x, ws.in_prompt, ws.in_cond, ws.in_style, B, T, ws.xmel16,
                          ws.cond16, ws.mc16, stream_));
  enqueue_merge_const(W, ws, R, stream_);
  enqueue_merge_step(W, ws, R, stream_, nullptr);
  d2h(out, ws.xa, (size_t)R * 512 * 4, stream_);
}

void Engine::stage_adaptive_norm(const float* in, const float* t1, int rows, int norm_id,
                                 float* out) {
  if (norm_id < 0 || norm_id > 26) throw std::invalid_argument("norm_id must be in [0, 26]");
  ensure_workspace(1, rows, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  upload_stage_tables(t1, nullptr);
  h2d(ws.stage_a, in, (size_t)rows * 512 * 4, stream_);
  HIP_OK(launch_adarms(ws.stage_a, W.gamma[norm_id], ws.tab + norm_id * 1024,
                       ws.tab + norm_id * 1024 + 512, ws.n16, rows, stream_));
  // widen the f16 result for the caller
  std::vector<_Float16> h((size_t)rows * 512);
  d2h(h.data(), ws.n16, h.size() * 2, stream_);
  for (size_t i = 0; i < h.size(); ++i) out[i] = (float)h[i];
}

void Engine::stage_attention_core(const float* in, const uint32_t* mask, int B, int T, int layer,
                                  float* out) {
  if (layer < 0 || layer > 12) throw std::invalid_argument("layer must be in [0, 12]");
  ensure_workspace(B, T, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  const int R = B * T;
  const int Tpad = (T + 63) / 64 * 64;
  ensure_rope(T);
  h2d(ws.mask, mask, (size_t)R * 4, stream_);
  ws.mask_host.clear();
  HIP_OK(launch_key_bias(ws.mask, B, T, (T + 63) / 64 * 64, ws.kbias, stream_));
  h2d(ws.stage_a, in, (size_t)R * 512 * 4, stream_);
  to_f16(ws.stage_a, ws.n16, (size_t)R * 512, stream_);
  GemmArgs g;
  g.M = R; g.N = 1536; g.K = 512; g.A = ws.n16; g.lda = 512; g.W = W.qkv_w[layer]; g.ldw = 512;
  g.T = T; g.rope = ws.rope; g.q = ws.q; g.k = ws.k; g.vt = ws.vt; g.Tpad = Tpad;
  HIP_OK(launch_gemm(g, A_PLAIN, EPI_QKV, stream_));
  // Per-branch key tiles: each branch stops after the key tile holding its
  // last unmasked key (the decode takes this form for ragged batches).
  HIP_OK(launch_attention(ws.q, ws.k, ws.vt, ws.kbias, ws.o16, B, T, Tpad, stream_, true));
  GemmArgs o;
  o.M = R; o.N = 512; o.K = 512; o.A = ws.o16; o.lda = 512; o.W = W.wo_w[layer]; o.ldw = 512;
  o.colperm = 1;
  o.C32 = ws.stage_b; o.ldc32 = 512;
  HIP_OK(launch_gemm(o, A_PLAIN, EPI_F32, stream_));
  d2h(out, ws.stage_b, (size_t)R * 512 * 4, stream_);
}

void Engine::stage_feed_forward(const float* in, int rows, int layer, float* out) {
  if (layer < 0 || layer > 12) throw std::invalid_argument("layer must be in [0, 12]");
  ensure_workspace(1, rows, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  h2d(ws.stage_a, in, (size_t)rows * 512 * 4, stream_);
  to_f16(ws.stage_a, ws.n16, (size_t)rows * 512, stream_);
  GemmArgs g;
  g.M = rows; g.N = 3072; g.K = 512; g.A = ws.n16; g.lda = 512; g.W = W.w13_w[layer]; g.ldw = 512;
  g.C16 = ws.g16; g.ldc16 = kHgLd;
  HIP_OK(launch_gemm(g, A_PLAIN, EPI_SWIGLU, stream_));
  GemmArgs o;
  o.M = rows; o.N = 512; o.K = 1536; o.A = ws.g16; o.lda = kHgLd; o.W = W.w2_w[layer]; o.ldw = 1536;
  o.colperm = 1;
  o.C32 = ws.stage_b; o.ldc32 = 512;
  HIP_OK(launch_gemm(o, A_PLAIN, EPI_F32, stream_));
  d2h(out, ws.stage_b, (size_t)rows * 512 * 4, stream_);
}

void Engine::stage_block(const float* in, const float* t1, const uint32_t* mask, int B, int T,
                         int layer, const float* skip, float* out) {
  if (layer < 0 || layer > 12) throw std::invalid_argument("layer must be in [0, 12]");
  if ((layer > 6) != (skip != nullptr))
    throw std::invalid_argument("layers 7..12 take a skip input, layers 0..6 do not");
  ensure_workspace(B, T, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  const int R = B * T;
  ensure_rope(T);
  upload_stage_tables(t1, nullptr);
  h2d(ws.mask, mask, (size_t)R * 4, stream_);
  ws.mask_host.clear();
  HIP_OK(launch_key_bias(ws.mask, B, T, (T + 63) / 64 * 64, ws.kbias, stream_));
  h2d(ws.xa, in, (size_t)R * 512 * 4, stream_);
  if (skip) {
    h2d(ws.stage_a, skip, (size_t)R * 512 * 4, stream_);
    to_f16(ws.stage_a, ws.skip16[0], (size_t)R * 512, stream_);
    to_f16(ws.xa, ws.x16, (size_t)R * 512, stream_);
  }
  if (layer <= 6)  // block 0..6 inputs come straight from x here, not from a producer GEMM
    HIP_OK(launch_norm_prep(ws.xa, ws.tab + layer * 1024, W.gamma[layer], ws.n16, ws.ssq, R,
                            stream_));
  enqueue_layer(layer, B, T, ws.tab, ws.nbq, ws.nbw, ws.xa, ws.xb, ws.skip16[0], ws.skip16[1]);
  d2h(out, ws.xa, (size_t)R * 512 * 4, stream_);
}

void Engine::stage_stack(const float* in, const float* t1, const uint32_t* mask, int B, int T,
                         float* out) {
  Weights& W = *w_;
  ensure_workspace(B, T, 1, 1);
  Workspace& ws = *ws_;
  const int R = B * T;
  ensure_rope(T);
  upload_stage_tables(t1, nullptr);
  h2d(ws.mask, mask, (size_t)R * 4, stream_);
  ws.mask_host.clear();
  HIP_OK(launch_key_bias(ws.mask, B, T, (T + 63) / 64 * 64, ws.kbias, stream_));
  h2d(ws.xa, in, (size_t)R * 512 * 4, stream_);
  HIP_OK(launch_norm_prep(ws.xa, ws.tab, W.gamma[0], ws.n16, ws.ssq, R, stream_));
  enqueue_transformer(B, T, ws.tab, ws.nbq, ws.nbw);
  std::vector<_Float16> h((size_t)R * 512);
  d2h(h.data(), ws.n16, h.size() * 2, stream_);
  for (size_t i = 0; i < h.size(); ++i) out[i] = (float)h[i];
}

void Engine::stage_post(const float* xres, const float* xmel, int rows, float* long_skip,
                        float* conv1, float* res_proj) {
  ensure_workspace(1, rows, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  h2d(ws.stage_a, xres, (size_t)rows * 512 * 4, stream_);
  to_f16(ws.stage_a, ws.n16, (size_t)rows * 512, stream_);
  // xmel16 rows (80 + zero pad): reuse step prep with zero prompt/cond/style.
  std::vector<float> zeros((size_t)rows * 512, 0.0f);
  h2d(ws.in_x, xmel, (size_t)rows * 80 * 4, stream_);
  h2d(ws.in_prompt, zeros.data(), (size_t)rows * 80 * 4, stream_);
  h2d(ws.in_cond, zeros.data(), (size_t)rows * 512 * 4, stream_);
  h2d(ws.in_style, zeros.data(), 192 * 4, stream_);
  HIP_OK(launch_step_prep(ws.in_x, ws.in_prompt, ws.in_cond, ws.in_style, 1, rows, ws.xmel16,
                          ws.cond16, ws.mc16, stream_));
  GemmArgs g;
  g.M = rows; g.N = 512; g.K = 512 + kMelPad; g.K1 = 512;
  g.A = ws.n16; g.lda = 512; g.A2 = ws.xmel16; g.lda2 = kMelPad;
  g.W = W.sl_w; g.ldw = 512 + kMelPad; g.bias = W.sl_b; g.C16 = ws.ls16; g.ldc16 = 512;
  HIP_OK(launch_gemm(g, A_CONCAT, EPI_F16, stream_));
  // conv1 / res_projection as the decode computes them: one product with the
  // folded weights (the long-skip output above is reported, not consumed).
  GemmArgs c;
  c.M = rows; c.N = 1024; c.K = 512 + kMelPad; c.K1 = 512;
  c.A = ws.n16; c.lda = 512; c.A2 = ws.xmel16; c.lda2 = kMelPad;
  c.W = W.post_w; c.ldw = 512 + kMelPad; c.bias = W.post_b;
  c.C32 = ws.wn_x; c.ldc32 = 512; c.C16 = ws.wn_x16; c.ldc16 = 512; c.C32b = ws.rp; c.ldc32b = 512;
  HIP_OK(launch_gemm(c, A_CONCAT, EPI_DUAL, stream_));
  std::vector<_Float16> h((size_t)rows * 512);
  d2h(h.data(), ws.ls16, h.size() * 2, stream_);
  for (size_t i = 0; i < h.size(); ++i) long_skip[i] = (float)h[i];
  d2h(conv1, ws.wn_x, (size_t)rows * 512 * 4, stream_);
  d2h(res_proj, ws.rp, (size_t)rows * 512 * 4, stream_);
}

void Engine::stage_wavenet(const float* in, const float* t2, const uint32_t* mask, int B, int T,
                           float* out) {
  ensure_workspace(B, T, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  const int R = B * T;
  upload_stage_tables(nullptr, t2);
  h2d(ws.mask, mask, (size_t)R * 4, stream_);
  ws.mask_host.clear();
  h2d(ws.wn_x, in, (size_t)R * 512 * 4, stream_);
  to_f16(ws.wn_x, ws.wn_x16, (size_t)R * 512, stream_);
  // zero res_projection so FINALSKIP yields the bare WaveNet output
  HIP_OK(launch_zero(ws.rp, (size_t)R * 512 * 4, stream_));
  const float* tab = ws.tab;
  for (int l = 0; l < 8; ++l) {
    GemmArgs c;
    c.M = R; c.N = 1024; c.K = 2560; c.A = ws.wn_x16; c.lda = 512; c.T = T; c.conv_c = 512;
    c.W = W.in_w[l]; c.ldw = 2560; c.bias = W.in_b[l]; c.cond = tab + kWnCondOff + l * 1024;
    c.C16 = ws.gate16; c.ldc16 = 512;
    HIP_OK(launch_gemm(c, A_CONV5, EPI_GATE, stream_));
    GemmArgs g;
    g.M = R; g.K = 512; g.A = ws.gate16; g.lda = 512; g.W = W.rs_w[l]; g.ldw = 512;
    g.bias = W.rs_b[l]; g.mask = ws.mask;
    if (l < 7) {
      g.N = 1024; g.C32 = ws.wn_x; g.ldc32 = 512; g.C16 = ws.wn_x16; g.ldc16 = 512;
      g.C32b = ws.wn_out; g.ldc32b = 512; g.flag = l > 0;
      HIP_OK(launch_gemm(g, A_PLAIN, EPI_RESSKIP, stream_));
    } else {
      g.N = 512; g.C32b = ws.wn_out; g.ldc32b = 512; g.C32 = ws.fin; g.ldc32 = 512; g.rp = ws.rp;
      HIP_OK(launch_gemm(g, A_PLAIN, EPI_FINALSKIP, stream_));
    }
  }
  d2h(out, ws.fin, (size_t)R * 512 * 4, stream_);
}

void Engine::stage_final_layer(const float* in, const float* t1, int rows, float* out) {
  ensure_workspace(1, rows, 1, 1);
  Weights& W = *w_;
  Workspace& ws = *ws_;
  upload_stage_tables(t1, nullptr);
  h2d(ws.fin, in, (size_t)rows * 512 * 4, stream_);
  HIP_OK(launch_adaln(ws.fin, ws.tab + kFinalSsOff, ws.tab + kFinalSsOff + 512, ws.n16, rows, stream_));
  GemmArgs g;
  g.M = rows; g.N = 512; g.K = 512; g.A = ws.n16; g.lda = 512;
  g.W = W.fin_w; g.ldw = 512; g.bias = W.fin_b; g.C32 = ws.stage_b; g.ldc32 = 512;
  HIP_OK(launch_gemm(g, A_PLAIN, EPI_F32, stream_));
  d2h(out, ws.stage_b, (size_t)rows * 512 * 4, stream_);
}

void Engine::op_linear(const float* A, const float* Wt, const float* bias, int M, int N, int K,
                       float* out) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0 || N % 64 != 0)
    throw std::invalid_argument("op_linear: need M > 0, K % 128 == 0, N % 64 == 0");
  HIP_OK(hipSetDevice(device_));
  DevBuf a32((size_t)M * K * 4), w32((size_t)N * K * 4), a16((size_t)M * K * 2),
      w16((size_t)N * K * 2), b((size_t)N * 4), c((size_t)M * N * 4);
  h2d(a32.p, A, (size_t)M * K * 4, stream_);
  h2d(w32.p, Wt, (size_t)N * K * 4, stream_);
  if (bias) h2d(b.p, bias, (size_t)N * 4, stream_);
  to_f16(a32.as<float>(), a16.as<half_t>(), (size_t)M * K, stream_);
  to_f16(w32.as<float>(), w16.as<half_t>(), (size_t)N * K, stream_);
  GemmArgs g;
  g.M = M; g.N = N; g.K = K; g.A = a16.as<half_t>(); g.lda = K; g.W = w16.as<half_t>(); g.ldw = K;
  g.bias = bias ? b.as<float>() : nullptr; g.C32 = c.as<float>(); g.ldc32 = N;
  HIP_OK(launch_gemm(g, A_PLAIN, EPI_F32, stream_));
  d2h(out, c.p, (size_t)M * N * 4, stream_);
}

// ------------------------------------------------------------------ condition producer
bool Engine::has_length_regulator() const { return w_->has_lr; }

void Engine::set_f32(int stage, bool f32) {
  if (stage == 1) {
    lr_f32_ = f32;
  } else if (stage == 2) {
    if (!voc_) throw std::runtime_error("vocoder: the context has no bigvgan.* tensors");
    voc_->set_f32(f32);
  } else {
    throw std::invalid_argument("precision: stage must be 1 (length regulator) or 2 (vocoder)");
  }
}

bool Engine::f32(int stage) const {
  if (stage == 1) return lr_f32_;
  if (stage == 2 && voc_) return voc_->f32();
  throw std::invalid_argument("precision: stage must be 1 (length regulator) or 2 (vocoder, when present)");
}

int Engine::generated_frames(int codes) {
  // static_cast<uint32_t>(static_cast<float>(codes) * 1.72f), synthesis_pipeline.cpp:1012
  return (int)(uint32_t)((float)codes * 1.72f);
}

void Engine::ensure_lr(int in_tokens, int out_tokens, int cond_rows) {
  if (in_tokens <= lr_.cap_in && out_tokens <= lr_.cap_out && cond_rows <= lr_.cap_cond) return;
  HIP_OK(hipStreamSynchronize(stream_));
  destroy_graphs(cond_graphs_);  // captured on the old buffers
  const int ci = std::max(in_tokens, lr_.cap_in), co = std::max(out_tokens, lr_.cap_out);
  const int cc = std::max(cond_rows, lr_.cap_cond);
  size_t bytes = 0;
  auto f = [&](size_t n) { bytes += (n * 4 + 255) / 256 * 256; };
  auto h = [&](size_t n) { bytes += (n * 2 + 255) / 256 * 256; };
  // The f16 GEMM operands are split pairs: hi rows, then lo rows.
  f((size_t)ci * 1024); h((size_t)ci * 1024 * 2); h((size_t)ci * 512 * 2); h((size_t)(co + 1) * 512 * 2);
  f((size_t)co * 512); f((size_t)co * 16); f((size_t)co * 16); f((size_t)cc * 512);
  lr_.arena.reserve(bytes);
  Arena& a = lr_.arena;
  lr_.in32 = static_cast<float*>(a.take((size_t)ci * 1024 * 4));
  lr_.s16 = static_cast<half_t*>(a.take((size_t)ci * 1024 * 2 * 2));
  lr_.p16 = static_cast<half_t*>(a.take((size_t)ci * 512 * 2 * 2));
  lr_.x16 = static_cast<half_t*>(a.take((size_t)(co + 1) * 512 * 2 * 2));
  lr_.y32 = static_cast<float*>(a.take((size_t)co * 512 * 4));
  lr_.sum_p = static_cast<float*>(a.take((size_t)co * 16 * 4));
  lr_.ssq_p = static_cast<float*>(a.take((size_t)co * 16 * 4));
  lr_.out32 = static_cast<float*>(a.take((size_t)cc * 512 * 4));
  lr_.cap_in = ci;
  lr_.cap_out = co;
  lr_.cap_cond = cc;
}

// run_length_regulator_full (gpt.cpp:5271-5313):
//   content_in_proj GEMM (f16 out) -> nearest rows (+ the zero padding row)
//   -> 4 x [k=3 zero-padded conv GEMM writing fp32 rows and per-row partial
//      sums / sums of squares; GroupNorm, its statistics reduced in the same
//      kernel, + Mish -> f16]
//   -> k=1 conv GEMM into `out`.
// In the default fp32 mode every GEMM operand is a split pair (hi, lo), so
// the products carry fp32-level precision like the reference's fp32 path;
// the f16 mode uses the hi halves alone.
void Engine::length_regulator_device(const float* s_infer, int in_tokens, int out_tokens,
                                     float* out) {
  if (!w_->has_lr)
    throw std::runtime_error("length regulator: the context has no s2mel.net.length_regulator.* tensors");
  if (in_tokens <= 0 || out_tokens <= 0)
    throw std::invalid_argument("length regulator: token counts must be positive");
  HIP_OK(hipSetDevice(device_));
  ensure_lr(in_tokens, out_tokens, 0);
  const LrView v{lr_.s16, lr_.p16, lr_.x16, lr_.y32, lr_.sum_p, lr_.ssq_p, lr_.cap_in, lr_.cap_out};
  run_graph(cond_graphs_,
            std::make_tuple(in_tokens, out_tokens, 0, (const void*)s_infer, (const void*)nullptr,
                            (const void*)out, lr_f32_),
            [&] { length_regulator_on(v, s_infer, in_tokens, out_tokens, out); });
}

// The regulator's launches on the buffers of `lr` (enqueued on stream_).
void Engine::length_regulator_on(const LrView& lr, const float* s_infer, int in_tokens, int out_tokens,
                                 float* out) {
  Weights& W = *w_;
  hipStream_t s = stream_;
  const int sp = lr_f32_ ? W.lr_wsplit : 0;
  // lo-half offsets (elements) of the split operand buffers
  const size_t s16_lo = sp ? (size_t)lr.cap_in * 1024 : 0;
  const size_t p16_lo = sp ? (size_t)lr.cap_in * 512 : 0;
  const size_t x16_lo = sp ? (size_t)(lr.cap_out + 1) * 512 : 0;
  HIP_OK(launch_f32_to_f16(s_infer, lr.s16, (size_t)in_tokens * 1024, s16_lo, s));
  {
    GemmArgs g;
    g.M = in_tokens; g.N = 512; g.K = 1024; g.A = lr.s16; g.lda = 1024;
    g.W = W.lr_proj_w; g.ldw = 1024; g.bias = W.lr_proj_b; g.C16 = lr.p16; g.ldc16 = 512;
    g.split = sp; g.a_lo = s16_lo; g.w_lo = sp == 2 ? (size_t)512 * 1024 : 0; g.c16_lo = p16_lo;
    HIP_OK(launch_gemm(g, A_PLAIN, EPI_F16, s));
  }
  HIP_OK(launch_nearest_rows(lr.p16, in_tokens, out_tokens, (float)in_tokens / (float)out_tokens,
                             lr.x16, p16_lo, x16_lo, s));
  for (int b = 0; b < 4; ++b) {
    GemmArgs g;
    g.M = out_tokens; g.N = 512; g.K = 3 * 512; g.T = out_tokens; g.conv_c = 512;
    g.A = lr.x16; g.lda = 512;
    g.W = W.lr_conv_w[b]; g.ldw = 3 * 512; g.bias = W.lr_conv_b[b];
    g.C32 = lr.y32; g.ldc32 = 512; g.sum_out = lr.sum_p; g.ssq_out = lr.ssq_p;
    g.split = sp; g.a_lo = x16_lo; g.w_lo = sp == 2 ? (size_t)512 * 1536 : 0;
    HIP_OK(launch_gemm(g, A_CONV3Z, EPI_F32, s));
    HIP_OK(launch_gn_mish(lr.sum_p, lr.ssq_p, 1e-5f, lr.y32, W.lr_gn_w[b], W.lr_gn_b[b], out_tokens,
                          lr.x16, x16_lo, s));
  }
  GemmArgs g;
  g.M = out_tokens; g.N = 512; g.K = 512; g.A = lr.x16; g.lda = 512;
  g.W = W.lr_out_w; g.ldw = 512; g.bias = W.lr_out_b; g.C32 = out; g.ldc32 = 512;
  g.split = sp; g.a_lo = x16_lo; g.w_lo = sp == 2 ? (size_t)512 * 512 : 0;
  HIP_OK(launch_gemm(g, A_PLAIN, EPI_F32, s));
}

int Engine::condition_device(const float* s_infer, int codes, const float* prompt_cond,
                             int prompt_tokens, float* cond) {
  if (codes <= 0 || prompt_tokens <= 0)
    throw std::invalid_argument("condition: codes and prompt_tokens must be positive");
  const int gen = generated_frames(codes);
  if (gen <= 0) throw std::invalid_argument("condition: generated frame count is zero");
  if (!w_->has_lr)
    throw std::runtime_error("length regulator: the context has no s2mel.net.length_regulator.* tensors");
  HIP_OK(hipSetDevice(device_));
  ensure_lr(codes, gen, 0);
  const LrView v{lr_.s16, lr_.p16, lr_.x16, lr_.y32, lr_.sum_p, lr_.ssq_p, lr_.cap_in, lr_.cap_out};
  run_graph(cond_graphs_,
            std::make_tuple(codes, gen, prompt_tokens, (const void*)s_infer, (const void*)prompt_cond,
                            (const void*)cond, lr_f32_),
            [&] {
              HIP_OK(hipMemcpyAsync(cond, prompt_cond, (size_t)prompt_tokens * 512 * 4,
                                    hipMemcpyDeviceToDevice, stream_));
              length_regulator_on(v, s_infer, codes, gen, cond + (size_t)prompt_tokens * 512);
            });
  return gen;
}

// condition_device on the static scratch: no device or host memory is
// allocated, and nothing is cleared (every scratch value the kernels read is
// written earlier in the same call: the split operands, the zero padding
// row and the partial sums).
int Engine::condition_device_noalloc(const float* s_infer, int codes, const float* prompt_cond,
                                     int prompt_tokens, float* cond) {
  if (!w_->has_lr)
    throw std::runtime_error("length regulator: the context has no s2mel.net.length_regulator.* tensors");
  if (codes <= 0 || prompt_tokens <= 0)
    throw std::invalid_argument("condition: codes and prompt_tokens must be positive");
  if (codes > kNoAllocMaxCodes)
    throw std::invalid_argument("condition (no-alloc): codes exceeds the scratch limit of " +
                                std::to_string(kNoAllocMaxCodes));
  const int gen = generated_frames(codes);
  if (gen <= 0) throw std::invalid_argument("condition: generated frame count is zero");
  HIP_OK(hipSetDevice(device_));
  char* base = scratch_ptr(device_);
  if (!base) throw HipError("condition (no-alloc): no scratch address for this device");
  const LrView v{reinterpret_cast<half_t*>(base + kScrS16), reinterpret_cast<half_t*>(base + kScrP16),
                 reinterpret_cast<half_t*>(base + kScrX16), reinterpret_cast<float*>(base + kScrY32),
                 reinterpret_cast<float*>(base + kScrSum),  reinterpret_cast<float*>(base + kScrSsq),
                 kNoAllocMaxCodes, kNoAllocMaxFrames};
  // Calls on this GPU are ordered through its event, except while the stream
  // is being captured into a graph (a captured stream may not wait on work
  // outside the capture): replays of such a graph must not overlap other
  // calls on this GPU.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HIP_OK(hipStreamIsCapturing(stream_, &cs));
  const bool order = cs == hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(g_scratch_call_mu);
  if (order) HIP_OK(hipStreamWaitEvent(stream_, g_scratch_ev[device_], 0));
  HIP_OK(hipMemcpyAsync(cond, prompt_cond, (size_t)prompt_tokens * 512 * 4, hipMemcpyDeviceToDevice,
                        stream_));
  length_regulator_on(v, s_infer, codes, gen, cond + (size_t)prompt_tokens * 512);
  if (order) HIP_OK(hipEventRecord(g_scratch_ev[device_], stream_));
  return gen;
}

void Engine::length_regulator_host(const float* s_infer, int in_tokens, int out_tokens,
                                   float* out) {
  if (in_tokens <= 0 || out_tokens <= 0)
    throw std::invalid_argument("length regulator: token counts must be positive");
  HIP_OK(hipSetDevice(device_));
  ensure_lr(in_tokens, out_tokens, out_tokens);
  h2d(lr_.in32, s_infer, (size_t)in_tokens * 1024 * 4, stream_);
  length_regulator_device(lr_.in32, in_tokens, out_tokens, lr_.out32);
  d2h(out, lr_.out32, (size_t)out_tokens * 512 * 4, stream_);
}

int Engine::condition_host(const float* s_infer, int codes, const float* prompt_cond,
                           int prompt_tokens, float* cond) {
  if (codes <= 0 || prompt_tokens <= 0)
    throw std::invalid_argument("condition: codes and prompt_tokens must be positive");
  const int gen = generated_frames(codes);
  if (gen <= 0) throw std::invalid_argument("condition: generated frame count is zero");
  HIP_OK(hipSetDevice(device_));
  ensure_lr(codes, gen, prompt_tokens + gen);
  h2d(lr_.in32, s_infer, (size_t)codes * 1024 * 4, stream_);
  h2d(lr_.out32, prompt_cond, (size_t)prompt_tokens * 512 * 4, stream_);
  length_regulator_device(lr_.in32, codes, gen, lr_.out32 + (size_t)prompt_tokens * 512);
  d2h(cond, lr_.out32, (size_t)(prompt_tokens + gen) * 512 * 4, stream_);
  return gen;
}

void Engine::normal_noise_device(size_t n, uint64_t seed, float temperature, float* out) {
  if (n == 0) throw std::invalid_argument("noise: empty shape");
  HIP_OK(hipSetDevice(device_));
  HIP_OK(launch_normal_noise(n, seed, temperature, out, stream_));
}

}  // namespace mit2hip

// ------------------------------------------------------------------ vocoder
namespace mit2hip {

static Vocoder& need_vocoder(const std::unique_ptr<Vocoder>& v) {
  if (!v) throw std::runtime_error("vocoder: the context has no bigvgan.* tensors");
  return *v;
}

void Engine::vocode_device(const float* mel, int tokens, float* wav) {
  HIP_OK(hipSetDevice(device_));
  need_vocoder(voc_).vocode_device(mel, tokens, wav);
}

void Engine::vocode_host(const float* mel, int tokens, float* wav) {
  HIP_OK(hipSetDevice(device_));
  Vocoder& v = need_vocoder(voc_);
  if (tokens <= 0) throw std::invalid_argument("vocoder: tokens must be positive");
  const size_t need = (size_t)tokens * (80 + 256);
  if (need > voc_io_floats_) {
    HIP_OK(hipStreamSynchronize(stream_));
    if (voc_io_) HIP_OK(hipFree(voc_io_));
    voc_io_ = nullptr;
    HIP_OK(hipMalloc(&voc_io_, need * sizeof(float)));
    voc_io_floats_ = need;
  }
  float* dmel = voc_io_;
  float* dwav = voc_io_ + (size_t)tokens * 80;
  HIP_OK(hipMemcpyAsync(dmel, mel, (size_t)tokens * 80 * sizeof(float), hipMemcpyHostToDevice, stream_));
  v.vocode_device(dmel, tokens, dwav);
  HIP_OK(hipMemcpyAsync(wav, dwav, (size_t)tokens * 256 * sizeof(float), hipMemcpyDeviceToHost, stream_));
  HIP_OK(hipStreamSynchronize(stream_));
}

int Engine::acoustic_device(const float* s_infer, int codes, const float* prompt_cond,
                            const float* prompt_mel, int prompt_tokens, const float* style,
                            uint64_t seed, float temperature, int steps, float cfg, float* wav,
                            float* mel) {
  if (codes <= 0 || prompt_tokens <= 0 || steps <= 0)
    throw std::invalid_argument("acoustic: codes, prompt_tokens and steps must be positive");
  need_vocoder(voc_);
  if (!w_->has_lr)
    throw std::runtime_error("acoustic: the context has no s2mel.net.length_regulator.* tensors");
  const int gen = generated_frames(codes);
  if (gen <= 0) throw std::invalid_argument("acoustic: generated frame count is zero");
  const int T = prompt_tokens + gen;
  HIP_OK(hipSetDevice(device_));
  if (T > ac_cap_) {
    HIP_OK(hipStreamSynchronize(stream_));
    clear_graphs();  // graphs captured on the old buffers
    ac_.reserve((size_t)T * (512 + 80 + 80) * sizeof(float) + 3 * 256);
    ac_cond_ = static_cast<float*>(ac_.take((size_t)T * 512 * sizeof(float)));
    ac_x0_ = static_cast<float*>(ac_.take((size_t)T * 80 * sizeof(float)));
    ac_mel_ = static_cast<float*>(ac_.take((size_t)T * 80 * sizeof(float)));
    ac_cap_ = T;
  }
  condition_device(s_infer, codes, prompt_cond, prompt_tokens, ac_cond_);
  normal_noise_device((size_t)T * 80, seed, temperature, ac_x0_);
  const uint32_t vt = (uint32_t)T, pt = (uint32_t)prompt_tokens;
  decode_device(ac_x0_, prompt_mel, ac_cond_, style, 1, T, &vt, &pt, steps, cfg, ac_mel_, nullptr);
  voc_->vocode_device(ac_mel_ + (size_t)prompt_tokens * 80, gen, wav);
  if (mel)
    HIP_OK(hipMemcpyAsync(mel, ac_mel_, (size_t)T * 80 * sizeof(float), hipMemcpyDeviceToDevice, stream_));
  return gen;
}

size_t Engine::vocoder_stage_host(int stage, int index, const float* in, int tokens, float* out) {
  HIP_OK(hipSetDevice(device_));
  return need_vocoder(voc_).stage_host(stage, index, in, tokens, out);
}

}  // namespace mit2hip
