// rowops.h -- bandwidth-bound row kernels of the DiT-CFM decoder (gfx950).
#pragma once

#include "device_common.h"

namespace mit2hip {

// AdaRMSNorm: out16[m] = aw * (x[m] * rsqrt(mean(x[m]^2) + 1e-5) * gamma) + ab  (width 512)
hipError_t launch_adarms(const float* x, const float* gamma, const float* aw, const float* ab,
                         half_t* out16, int rows, hipStream_t s);
// The producer half of a folded AdaRMSNorm for a row block that no GEMM
// produced (stage entry points): n16[m] = f16(x[m] * aw * gamma) and the
// row's 16 partial sums of squares over 32-column blocks, ssq[m][16].
hipError_t launch_norm_prep(const float* x, const float* aw, const float* gamma, half_t* n16,
                            float* ssq, int rows, hipStream_t s);
// Column bias of a folded AdaRMSNorm, per step: out[s][n] = sum_k ab_s[k] *
// W[n][k] (K = 512, W f16 [N][512] as resident), ab_s = ab + s * ab_ld.
hipError_t launch_norm_bias(const float* ab, int ab_ld, int S, const half_t* W, int N, float* out,
                            int out_ld, hipStream_t s);
// Final-layer AdaLN: LayerNorm (no affine, eps 1e-6), then * (1 + scale) + shift (width 512)
hipError_t launch_adaln(const float* x, const float* shift, const float* scale, half_t* out16,
                        int rows, hipStream_t s);
// Masked attention (attention.hip).  kbias [B][Tpad]: 0 for a valid key,
// -inf for a masked or padding key, followed by B int32 key counts (one past
// each branch's last valid key), as launch_key_bias builds them from the
// [B][T] 0/1 key mask into a buffer of B * Tpad + B words.  With
// branch_keys, a branch's key tiles after its last valid key are skipped
// (they are fully masked: the result is the same up to the split of the
// keys between the kernel's two groups); worth it for padded batches.  With
// qskip (implies branch_keys) the query rows from two past a branch's last
// valid key on are not computed: their outputs keep what they held.
hipError_t launch_attention(const half_t* Q, const half_t* K, const half_t* Vt,
                            const float* kbias, half_t* O, int B, int T, int Tpad,
                            hipStream_t stream, bool branch_keys = false, bool qskip = false);
hipError_t launch_key_bias(const uint32_t* mask, int B, int T, int Tpad, float* kbias,
                           hipStream_t stream);

// Decode set-up for nreq requests of T tokens (branches b = 2r (cond), 2r+1 (null)
// when cfg is on, b = r when off):
//   x_cur[r][t][80] = x0 with rows t < P[r] zeroed,
//   xmel16[b][t][kMelPad] = f16(x_cur) (cols 80.. zero),
//   cond16[b][t][512] = f16(cond[r]) for cond branches, 0 for null branches,
//   mc16[b][t][kMcWidth] = [prompt_x (zero pad) | . | style | 0]; the
//   cond-projection GEMM fills columns kMcContent..kMcContent+511 afterwards.
hipError_t launch_decode_prep(const float* x0, const float* prompt, const float* cond,
                              const float* style, const uint32_t* P, int nreq, int T, int cfg_on,
                              float* x_cur, half_t* xmel16, half_t* cond16, half_t* mc16,
                              hipStream_t s);

// Estimator-step set-up for B independent branches (caller supplies every branch):
//   xmel16[m][kMelPad] = f16(x[m]), cond16[m] = f16(cond[m]),
//   mc16[m] = [prompt_x[m] (zero pad) | . | style[b] | 0].
hipError_t launch_step_prep(const float* x, const float* prompt_x, const float* cond,
                            const float* style, int B, int T, half_t* xmel16, half_t* cond16,
                            half_t* mc16, hipStream_t s);

// conv2 (512 -> 80, k=1) + CFG blend + Euler update for nreq requests:
//   dphi_b = y16[b] . W2^T + bias2;  v = (1+cfg)*dphi_cond - cfg*dphi_null (cfg on) or dphi_cond;
//   x_cur += dt * v; rows t < P[r] set to 0; xmel16 of every branch refreshed.
// vtrace (optional) receives v as [nreq][T][80].
hipError_t launch_conv2_euler(const half_t* y16, const half_t* w2, const float* b2,
                              const uint32_t* P, int nreq, int T, int cfg_on, float cfg, float dt,
                              float* x_cur, half_t* xmel16, float* vtrace, hipStream_t s);
// conv2 only: dphi[m][80] = y16[m] . W2^T + bias2 for every row.
hipError_t launch_conv2_rows(const half_t* y16, const half_t* w2, const float* b2, int rows,
                             float* dphi, hipStream_t s);

// Timestep-conditioning tables (fp32):
//   temb[s][256] = [cos(1000 t_s f_i) | sin(1000 t_s f_i)], i < 128
hipError_t launch_timestep_embedding(const float* tvals, const float* freqs, int S, float* temb,
                                     hipStream_t s);
// out[s][n] = bias[n] + sum_k W[n][k] * act(in[s][k]), act = SiLU when silu_in, then
// SiLU on the result when silu_out.  ldout is the row stride of out.
hipError_t launch_linear_small(const float* in, int S, int K, const float* W, const float* bias,
                               int N, int silu_in, int silu_out, float* out, int ldout,
                               hipStream_t s);
// dst[i] = src[i], i < n (graph-friendly copy kernel).
hipError_t launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s);
// Fills n halves / floats with zero (graph-safe replacement for memset).
hipError_t launch_zero(void* p, size_t bytes, hipStream_t s);

}  // namespace mit2hip
