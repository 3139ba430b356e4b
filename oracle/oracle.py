"""ctypes binding of the CPU oracle (oracle/build/libcfm_oracle.so).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, to compare results with or as the timed CPU
baseline.
The product path never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "libcfm_oracle.so"

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_lib = None


class _GreedyResult(ctypes.Structure):
    _fields_ = [("n_predicted", ctypes.c_uint32), ("n_input", ctypes.c_uint32),
                ("first_stop_step", ctypes.c_int32)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, u32, i32, f32, u64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_float, ctypes.c_uint64
        sig = {
            "orc_set_threads": (None, [i32]),
            "orc_get_threads": (i32, []),
            "orc_half_to_float": (f32, [ctypes.c_uint16]),
            "orc_halves_to_floats": (None, [ctypes.POINTER(ctypes.c_uint16), ctypes.c_size_t, _f32p]),
            "orc_splitmix64_next": (u64, [ctypes.POINTER(ctypes.c_uint64)]),
            "orc_uniform_open01": (f32, [ctypes.POINTER(ctypes.c_uint64)]),
            "orc_normal_noise": (None, [u32, u32, u64, f32, _f32p]),
            "orc_layernorm": (None, [_f32p, _f32p, _f32p, u32, f32, _f32p]),
            "orc_rmsnorm": (None, [_f32p, _f32p, u32, f32, _f32p]),
            "orc_linear": (None, [_f32p, _f32p, _f32p, u32, u32, _f32p]),
            "orc_linear_rows": (None, [_f32p, _f32p, _f32p, u32, u32, u32, _f32p]),
            "orc_conv1d_same": (None, [_f32p, _f32p, _f32p, u32, u32, u32, u32, _f32p]),
            "orc_reflect_pad": (None, [_f32p, u32, u32, u32, u32, _f32p]),
            "orc_nearest_interpolate": (None, [_f32p, u32, u32, u32, _f32p]),
            "orc_groupnorm1": (None, [_f32p, _f32p, _f32p, u32, u32, f32, _f32p]),
            "orc_mish": (None, [_f32p, ctypes.c_size_t, _f32p]),
            "orc_length_regulator": (None, [_f32p, u32, u32, _f32p, _f32p, ctypes.POINTER(_f32p),
                                            ctypes.POINTER(_f32p), ctypes.POINTER(_f32p),
                                            ctypes.POINTER(_f32p), _f32p, _f32p, _f32p]),
            "orc_length_regulator_ex": (None, [_f32p, u32, u32, _f32p, _f32p, ctypes.POINTER(_f32p),
                                               ctypes.POINTER(_f32p), ctypes.POINTER(_f32p),
                                               ctypes.POINTER(_f32p), _f32p, _f32p, ctypes.c_int, _f32p]),
            "orc_groupnorm1_f64stats": (None, [_f32p, _f32p, _f32p, u32, u32, f32, _f32p]),
            "orc_conv1d_reflect_same": (None, [_f32p, _f32p, _f32p, u32, u32, u32, u32, _f32p]),
            "orc_conv1d_dilated_same": (None, [_f32p, _f32p, _f32p, u32, u32, u32, u32, u32, _f32p]),
            "orc_conv_transpose1d": (None, [_f32p, _f32p, _f32p, u32, u32, u32, u32, u32, u32, _f32p]),
            "orc_bigvgan_activation": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, u32, u32, _f32p]),
            "orc_timestep_embedding": (None, [_f32p, u32, _f32p, u32, f32, _f32p]),
            "orc_attention_head_masked": (None, [_f32p, _f32p, _f32p, _u32p, u32, u32, _f32p]),
            "orc_rope_inplace": (None, [_f32p, u32, u32, u32]),
            "orc_weight_norm_rowmajor": (None, [_f32p, _f32p, u32, u32, _f32p]),
            "orc_model_new": (vp, []),
            "orc_model_free": (None, [vp]),
            "orc_model_set": (i32, [vp, ctypes.c_char_p, _f32p, u64]),
            "orc_model_tensor_count": (i32, []),
            "orc_model_tensor_name": (ctypes.c_char_p, [i32]),
            "orc_model_tensor_elems": (u64, [i32]),
            "orc_model_missing": (i32, [vp]),
            "orc_last_error": (ctypes.c_char_p, []),
            "orc_timestep_embedder": (None, [vp, f32, i32, _f32p]),
            "orc_input_merge": (None, [vp, _f32p, _f32p, _f32p, _f32p, u32, _f32p]),
            "orc_adaptive_norm": (None, [vp, _f32p, _f32p, u32, i32, _f32p]),
            "orc_attention_core": (None, [vp, _f32p, _u32p, u32, u32, _f32p]),
            "orc_feed_forward": (None, [vp, _f32p, u32, u32, _f32p]),
            "orc_skip_in": (None, [vp, _f32p, _f32p, u32, u32, _f32p]),
            "orc_transformer_block": (None, [vp, _f32p, _f32p, _u32p, u32, u32, _f32p, _f32p]),
            "orc_transformer_stack": (None, [vp, _f32p, _f32p, _u32p, u32, _f32p]),
            "orc_post_transformer": (None, [vp, _f32p, _f32p, u32, _f32p, _f32p, _f32p]),
            "orc_wavenet": (None, [vp, _f32p, _f32p, _u32p, u32, _f32p]),
            "orc_final_layer": (None, [vp, _f32p, _f32p, u32, _f32p]),
            "orc_estimator_step": (None, [vp, _f32p, _f32p, _f32p, _f32p, f32, _u32p, u32, _f32p]),
            "orc_cfm_euler": (None, [vp, _f32p, _f32p, _f32p, _f32p, u32, u32, u32, f32]),
            "orc_cfm_euler_trace": (None, [vp, _f32p, _f32p, _f32p, _f32p, u32, u32, u32, f32,
                                           _f32p, _f32p]),
            "orc_cfm_euler_masked": (None, [vp, _f32p, _f32p, _f32p, _f32p, _u32p, u32, u32, u32,
                                            f32]),
            "orc_cfm_euler_partial": (None, [vp, _f32p, _f32p, _f32p, _f32p, u32, u32, u32, u32, f32,
                                             _f32p, _f32p]),
            "orc_gpt_new": (vp, [i32]),
            "orc_gpt_free": (None, [vp]),
            "orc_gpt_set": (i32, [vp, ctypes.c_char_p, _f32p, u64]),
            "orc_gpt_missing": (i32, [vp]),
            "orc_gpt_last_error": (ctypes.c_char_p, []),
            "orc_gelu_new": (None, [_f32p, ctypes.c_size_t, _f32p]),
            "orc_attention_single_query": (None, [_f32p, _f32p, _f32p, u32, u32, _f32p]),
            "orc_attention_causal": (None, [_f32p, _f32p, _f32p, u32, u32, _f32p]),
            "orc_gpt_layer_qkv": (None, [vp, _f32p, u32, u32, _f32p]),
            "orc_gpt_block": (None, [vp, _f32p, u32, u32, _f32p]),
            "orc_gpt_cached_block_current": (None, [vp, _f32p, _f32p, u32, _f32p, _f32p, u32, _f32p]),
            "orc_gpt_logits": (u32, [vp, _f32p, u32, _f32p, _f32p]),
            "orc_gpt_cached_decode": (u32, [vp, _f32p, u32, _f32p, _f32p, _f32p]),
            "orc_gpt_kv_greedy": (i32, [vp, _f32p, u32, u32, i32, _u32p, _u32p, _f32p,
                                        ctypes.POINTER(_GreedyResult)]),
            "orc_gpt_greedy_full": (i32, [vp, _f32p, u32, u32, _u32p, _u32p, _f32p,
                                          ctypes.POINTER(_GreedyResult)]),
            "orc_gpt_sampling_processors": (i32, [_f32p, u32, _u32p, u32, f32, u32, f32, f32, _f32p]),
            "orc_gpt_sample_token": (u32, [_f32p, u32, ctypes.POINTER(u64)]),
            "orc_gpt_kv_sample": (i32, [vp, _f32p, u32, u32, i32, u64, f32, u32, f32, f32, _u32p, u32, _u32p,
                                        _u32p, _f32p, _f32p, ctypes.POINTER(_GreedyResult)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def P(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def PU(a: np.ndarray):
    return a.ctypes.data_as(_u32p)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def default_threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count() or 1))


# ---------------------------------------------------------------- primitives
def linear(w, b, x) -> np.ndarray:
    w, b, x = f32(w), f32(b), f32(x)
    rows, cols = w.shape
    x2 = x.reshape(-1, cols)
    out = np.empty((x2.shape[0], rows), np.float32)
    lib().orc_linear_rows(P(w), P(b), P(x2), x2.shape[0], rows, cols, P(out))
    return out.reshape(x.shape[:-1] + (rows,))


def rmsnorm(x, gamma, eps) -> np.ndarray:
    x, g = f32(x), f32(gamma)
    out = np.empty_like(x)
    n = x.shape[-1]
    for r in range(x.size // n):
        lib().orc_rmsnorm(P(x[r:r + 1].reshape(-1) if x.ndim > 1 else x), P(g), n, eps,
                          out.reshape(-1, n)[r:r + 1].ctypes.data_as(_f32p))
    return out


def layernorm(x, gamma, beta, eps) -> np.ndarray:
    x, g, b = f32(x), f32(gamma), f32(beta)
    n = x.shape[-1]
    x2 = x.reshape(-1, n)
    out = np.empty_like(x2)
    for r in range(x2.shape[0]):
        xr = np.ascontiguousarray(x2[r])
        o = np.empty(n, np.float32)
        lib().orc_layernorm(P(xr), P(g), P(b), n, eps, P(o))
        out[r] = o
    return out.reshape(x.shape)


def conv1d_same(x, w, b, kernel) -> np.ndarray:
    x, w, b = f32(x), f32(w), f32(b)
    tokens, cin = x.shape
    cout = b.size
    out = np.empty((tokens, cout), np.float32)
    lib().orc_conv1d_same(P(x), P(w), P(b), tokens, cin, cout, kernel, P(out))
    return out


def nearest_interpolate(x, out_tokens) -> np.ndarray:
    x = f32(x)
    in_tokens, width = x.shape
    out = np.empty((out_tokens, width), np.float32)
    lib().orc_nearest_interpolate(P(x), in_tokens, out_tokens, width, P(out))
    return out


def groupnorm1(x, gamma, beta, eps=1e-5, f64_stats: bool = False) -> np.ndarray:
    x, g, b = f32(x), f32(gamma), f32(beta)
    tokens, channels = x.shape
    out = np.empty_like(x)
    fn = lib().orc_groupnorm1_f64stats if f64_stats else lib().orc_groupnorm1
    fn(P(x), P(g), P(b), tokens, channels, eps, P(out))
    return out


def mish(x) -> np.ndarray:
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_mish(P(x), x.size, P(out))
    return out


LR_PREFIX = "s2mel.net.length_regulator."


def length_regulator(tensors: dict, s_infer, out_tokens: int, f64_stats: bool = False) -> np.ndarray:
    """run_length_regulator_full_cpu (gpt.cpp:5298): s_infer [in_tokens, 1024]
    -> [out_tokens, 512]; tensors holds the s2mel.net.length_regulator.* weights.
    f64_stats: the GroupNorm statistics in double instead of the reference's
    sequential float sums (a checker, not the reference's arithmetic)."""
    t = {k[len(LR_PREFIX):]: f32(v) for k, v in tensors.items() if k.startswith(LR_PREFIX)}
    x = f32(s_infer)
    in_tokens = x.shape[0]
    conv = [t[f"model.{i}.weight"] for i in (0, 3, 6, 9)]
    conv_b = [t[f"model.{i}.bias"] for i in (0, 3, 6, 9)]
    gn = [t[f"model.{i}.weight"] for i in (1, 4, 7, 10)]
    gn_b = [t[f"model.{i}.bias"] for i in (1, 4, 7, 10)]
    arrs = lambda lst: (_f32p * 4)(*[P(a) for a in lst])
    out = np.empty((out_tokens, 512), np.float32)
    lib().orc_length_regulator_ex(P(x), in_tokens, out_tokens, P(t["content_in_proj.weight"]),
                                  P(t["content_in_proj.bias"]), arrs(conv), arrs(conv_b), arrs(gn),
                                  arrs(gn_b), P(t["model.12.weight"]), P(t["model.12.bias"]),
                                  1 if f64_stats else 0, P(out))
    return out


def conv1d_reflect_same(x, w, b, kernel) -> np.ndarray:
    x, w, b = f32(x), f32(w), f32(b)
    tokens, cin = x.shape
    cout = b.size
    out = np.empty((tokens, cout), np.float32)
    lib().orc_conv1d_reflect_same(P(x), P(w), P(b), tokens, cin, cout, kernel, P(out))
    return out


def reflect_pad(x, left, right) -> np.ndarray:
    x = f32(x)
    tokens, ch = x.shape
    out = np.empty((tokens + left + right, ch), np.float32)
    lib().orc_reflect_pad(P(x), tokens, ch, left, right, P(out))
    return out


def timestep_embedding(t, freqs, scale=1000.0) -> np.ndarray:
    t, fr = f32(np.atleast_1d(t)), f32(freqs)
    out = np.empty((t.size, 2 * fr.size), np.float32)
    lib().orc_timestep_embedding(P(t), t.size, P(fr), fr.size, scale, P(out))
    return out


def attention_head(q, k, v, mask) -> np.ndarray:
    q, k, v, m = f32(q), f32(k), f32(v), u32(mask)
    tokens, hd = q.shape
    out = np.empty_like(q)
    lib().orc_attention_head_masked(P(q), P(k), P(v), PU(m), tokens, hd, P(out))
    return out


def rope(x, heads, head_dim) -> np.ndarray:
    x = f32(x).copy()
    tokens = x.size // (heads * head_dim)
    lib().orc_rope_inplace(P(x), tokens, heads, head_dim)
    return x


def weight_norm(g, v) -> np.ndarray:
    g, v = f32(g), f32(v)
    rows = g.size
    cols = v.size // rows
    out = np.empty((rows, cols), np.float32)
    lib().orc_weight_norm_rowmajor(P(g), P(v), rows, cols, P(out))
    return out


def normal_noise(tokens, channels, seed, temperature=1.0) -> np.ndarray:
    out = np.empty((tokens, channels), np.float32)
    lib().orc_normal_noise(tokens, channels, seed, temperature, P(out))
    return out


def half_to_float(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_halves_to_floats(h.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), h.size, P(out))
    return out


# ---------------------------------------------------------------- model
class Model:
    """Estimator weights widened to fp32 (tensor_as_f32) plus the stage functions."""

    def __init__(self, tensors: dict[str, np.ndarray]):
        L = lib()
        self._m = L.orc_model_new()
        for name, v in tensors.items():
            a = np.asarray(v)
            if a.dtype == np.float16:
                a = half_to_float(a.view(np.uint16))
            a = f32(a)
            if L.orc_model_set(self._m, name.encode(), P(a), a.size) != 0:
                raise ValueError(L.orc_last_error().decode())
        if L.orc_model_missing(self._m):
            raise ValueError(L.orc_last_error().decode())

    def close(self):
        if self._m:
            lib().orc_model_free(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def timestep_embedder(self, t, which):
        out = np.empty(512, np.float32)
        lib().orc_timestep_embedder(self._m, t, which, P(out))
        return out

    def input_merge(self, x, prompt_x, cond, style):
        x = f32(x)
        T = x.shape[0]
        out = np.empty((T, 512), np.float32)
        lib().orc_input_merge(self._m, P(x), P(f32(prompt_x)), P(f32(cond)), P(f32(style)), T, P(out))
        return out

    def adaptive_norm(self, x, t1, norm_id):
        x = f32(x)
        T = x.size // 512
        out = np.empty((T, 512), np.float32)
        lib().orc_adaptive_norm(self._m, P(x), P(f32(t1)), T, norm_id, P(out))
        return out

    def attention_core(self, x, mask, layer):
        x, m = f32(x), u32(mask)
        T = m.size
        out = np.empty((T, 512), np.float32)
        lib().orc_attention_core(self._m, P(x), PU(m), T, layer, P(out))
        return out

    def feed_forward(self, x, layer):
        x = f32(x)
        T = x.size // 512
        out = np.empty((T, 512), np.float32)
        lib().orc_feed_forward(self._m, P(x), T, layer, P(out))
        return out

    def block(self, x, t1, mask, layer, skip=None):
        x, m = f32(x), u32(mask)
        T = m.size
        out = np.empty((T, 512), np.float32)
        sk = None if skip is None else f32(skip)
        lib().orc_transformer_block(self._m, P(x), P(f32(t1)), PU(m), T, layer,
                                    None if sk is None else P(sk), P(out))
        return out

    def stack(self, x, t1, mask):
        x, m = f32(x), u32(mask)
        T = m.size
        out = np.empty((T, 512), np.float32)
        lib().orc_transformer_stack(self._m, P(x), P(f32(t1)), PU(m), T, P(out))
        return out

    def post(self, xres, xmel):
        xres = f32(xres)
        T = xres.size // 512
        ls, c1, rp = (np.empty((T, 512), np.float32) for _ in range(3))
        lib().orc_post_transformer(self._m, P(xres), P(f32(xmel)), T, P(ls), P(c1), P(rp))
        return ls, c1, rp

    def wavenet(self, x, t2, mask):
        x, m = f32(x), u32(mask)
        T = m.size
        out = np.empty((T, 512), np.float32)
        lib().orc_wavenet(self._m, P(x), P(f32(t2)), PU(m), T, P(out))
        return out

    def final_layer(self, x, t1):
        x = f32(x)
        T = x.size // 512
        out = np.empty((T, 512), np.float32)
        lib().orc_final_layer(self._m, P(x), P(f32(t1)), T, P(out))
        return out

    def estimator_step(self, x, prompt_x, cond, style, t, mask):
        x, m = f32(x), u32(mask)
        T = m.size
        out = np.empty((T, 80), np.float32)
        lib().orc_estimator_step(self._m, P(x), P(f32(prompt_x)), P(f32(cond)), P(f32(style)), t,
                                 PU(m), T, P(out))
        return out

    def cfm_euler(self, x0, prompt, cond, style, steps, cfg, trace=False):
        x = f32(x0).copy()
        T = x.size // 80
        pr = f32(prompt)
        Pn = pr.size // 80
        if not trace:
            lib().orc_cfm_euler(self._m, P(x), P(pr) if Pn else None, P(f32(cond)), P(f32(style)), T,
                                Pn, steps, cfg)
            return x.reshape(T, 80)
        xt = np.empty((steps, T, 80), np.float32)
        vt = np.empty((steps, T, 80), np.float32)
        lib().orc_cfm_euler_trace(self._m, P(x), P(pr) if Pn else None, P(f32(cond)), P(f32(style)),
                                  T, Pn, steps, cfg, P(xt), P(vt))
        return x.reshape(T, 80), xt, vt

    def cfm_euler_partial(self, x0, prompt, cond, style, steps, run_steps, cfg):
        """The first run_steps Euler steps of the steps-step schedule: (state after
        them, states before each, guided velocities of each)."""
        x = f32(x0).copy()
        T = x.size // 80
        pr = f32(prompt)
        Pn = pr.size // 80
        xt = np.empty((run_steps, T, 80), np.float32)
        vt = np.empty((run_steps, T, 80), np.float32)
        lib().orc_cfm_euler_partial(self._m, P(x), P(pr) if Pn else None, P(f32(cond)), P(f32(style)),
                                    T, Pn, steps, run_steps, cfg, P(xt), P(vt))
        return x.reshape(T, 80), xt, vt

    def cfm_euler_masked(self, x0, prompt, cond, style, mask, steps, cfg):
        """Euler decode at the padded length with key mask (one request)."""
        x = f32(x0).copy()
        m = u32(mask)
        T = m.size
        pr = f32(prompt)
        Pn = pr.size // 80
        lib().orc_cfm_euler_masked(self._m, P(x), P(pr) if Pn else None, P(f32(cond)), P(f32(style)),
                                   PU(m), T, Pn, steps, cfg)
        return x.reshape(T, 80)


def rel_l2(got, ref) -> float:
    """metal_indextts2/metrics.py:40-54 relative_l2_error."""
    g = np.asarray(got, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    return float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))


# ---------------------------------------------------------------- BigVGAN vocoder
def conv1d_dilated_same(x, w, b, kernel, dilation) -> np.ndarray:
    """cpu_conv1d_dilated_same (tokenizer_tests.cpp:3739): x [tokens, in], w [out, in, kernel]."""
    x, w, b = f32(x), f32(w), f32(b)
    tokens, cin = x.shape
    out = np.empty((tokens, b.size), np.float32)
    lib().orc_conv1d_dilated_same(P(x), P(w), P(b), tokens, cin, b.size, kernel, dilation, P(out))
    return out


def conv_transpose1d(x, w, b, kernel, stride, padding) -> np.ndarray:
    """cpu_conv_transpose1d (tokenizer_tests.cpp:3760): x [tokens, in], w [in, out, kernel]."""
    x, w, b = f32(x), f32(w), f32(b)
    tokens, cin = x.shape
    out_tokens = (tokens - 1) * stride + kernel - 2 * padding
    out = np.empty((out_tokens, b.size), np.float32)
    lib().orc_conv_transpose1d(P(x), P(w), P(b), tokens, cin, b.size, kernel, stride, padding, P(out))
    return out


def bigvgan_activation(x, up_filter, down_filter, alpha_log, beta_log) -> np.ndarray:
    """cpu_bigvgan_activation (tokenizer_tests.cpp:3811): anti-aliased SnakeBeta, x [tokens, C]."""
    x, up, down, a, bt = f32(x), f32(up_filter), f32(down_filter), f32(alpha_log), f32(beta_log)
    tokens, channels = x.shape
    out = np.empty_like(x)
    lib().orc_bigvgan_activation(P(x), P(up), P(down), P(a), P(bt), tokens, channels, P(out))
    return out


# kBigVGANUpsamplers (dit_cfm_bigvgan.cpp:3681-3688): prefix, in, out, kernel, stride, padding.
BIGVGAN_UPSAMPLERS = [("bigvgan.ups.0.0", 1536, 768, 8, 4, 2), ("bigvgan.ups.1.0", 768, 384, 8, 4, 2),
                      ("bigvgan.ups.2.0", 384, 192, 4, 2, 1), ("bigvgan.ups.3.0", 192, 96, 4, 2, 1),
                      ("bigvgan.ups.4.0", 96, 48, 4, 2, 1), ("bigvgan.ups.5.0", 48, 24, 4, 2, 1)]
# kBigVGANResblocks (dit_cfm_bigvgan.cpp:3960-3979): prefix, channels, kernel.
BIGVGAN_RESBLOCKS = [(f"bigvgan.resblocks.{3 * g + i}", 768 >> g, (3, 7, 11)[i])
                     for g in range(6) for i in range(3)]
BIGVGAN_DILATIONS = (1, 3, 5)


class BigVGAN:
    """The reference's fp32 CPU vocoder (dit_cfm_bigvgan.cpp:3606-4062) composed from the
    oracle primitives; element-wise adds, the /3 average and the clamp are float32 numpy
    operations in the reference's order.  tensors: the bigvgan.* weights (any float dtype)."""

    def __init__(self, tensors: dict):
        self.t = {k: f32(v) for k, v in tensors.items() if k.startswith("bigvgan.")}
        self._wn = {}

    def conv_weight(self, prefix, out_ch, in_ch, kernel):
        """weight_norm_conv_weight (gpt.cpp:5126): rows = output channels."""
        if prefix not in self._wn:
            w = weight_norm(self.t[prefix + ".weight_g"].reshape(out_ch),
                            self.t[prefix + ".weight_v"].reshape(out_ch, in_ch * kernel))
            self._wn[prefix] = w.reshape(out_ch, in_ch, kernel)
        return self._wn[prefix]

    def conv_transpose_weight(self, prefix, in_ch, out_ch, kernel):
        """weight_norm_conv_transpose_weight (gpt.cpp:5132): rows = input channels."""
        if prefix not in self._wn:
            w = weight_norm(self.t[prefix + ".weight_g"].reshape(in_ch),
                            self.t[prefix + ".weight_v"].reshape(in_ch, out_ch * kernel))
            self._wn[prefix] = w.reshape(in_ch, out_ch, kernel)
        return self._wn[prefix]

    def conv_pre(self, mel):
        """run_bigvgan_conv_pre_cpu (:3606): conv k=7 zero-padded, 80 -> 1536."""
        return conv1d_same(mel, self.conv_weight("bigvgan.conv_pre", 1536, 80, 7),
                           self.t["bigvgan.conv_pre.bias"], 7)

    def upsample(self, x, i):
        """run_bigvgan_upsample_cpu (:3690)."""
        prefix, cin, cout, k, stride, pad = BIGVGAN_UPSAMPLERS[i]
        return conv_transpose1d(x, self.conv_transpose_weight(prefix, cin, cout, k),
                                self.t[prefix + ".bias"], k, stride, pad)

    def activation(self, prefix, x):
        """run_bigvgan_activation_cpu (:3810)."""
        t = self.t
        return bigvgan_activation(x, t[prefix + ".upsample.filter"].reshape(-1),
                                  t[prefix + ".downsample.lowpass.filter"].reshape(-1),
                                  t[prefix + ".act.alpha"], t[prefix + ".act.beta"])

    def resblock_pair(self, prefix, x, pair, kernel, dilation):
        """run_bigvgan_resblock_pair_cpu (:3885): act, dilated conv, act, conv, + x."""
        c = x.shape[1]
        xt = self.activation(f"{prefix}.activations.{2 * pair}", x)
        xt = conv1d_dilated_same(xt, self.conv_weight(f"{prefix}.convs1.{pair}", c, c, kernel),
                                 self.t[f"{prefix}.convs1.{pair}.bias"], kernel, dilation)
        xt = self.activation(f"{prefix}.activations.{2 * pair + 1}", xt)
        xt = conv1d_dilated_same(xt, self.conv_weight(f"{prefix}.convs2.{pair}", c, c, kernel),
                                 self.t[f"{prefix}.convs2.{pair}.bias"], kernel, 1)
        return xt + f32(x)

    def resblock(self, prefix, x, kernel):
        """run_bigvgan_resblock_cpu (:3939): dilations 1, 3, 5."""
        for i, d in enumerate(BIGVGAN_DILATIONS):
            x = self.resblock_pair(prefix, x, i, kernel, d)
        return x

    def resblock_group(self, x, group):
        """run_bigvgan_resblock_group_cpu (:3982): out += rb / 3 over the three kernels."""
        out = np.zeros_like(f32(x))
        for prefix, _, kernel in BIGVGAN_RESBLOCKS[3 * group:3 * group + 3]:
            out += self.resblock(prefix, x, kernel) / np.float32(3.0)
        return out

    def body(self, mel):
        """run_bigvgan_body_cpu (:4008): conv_pre, then 6 x (upsampler, resblock group)."""
        x = self.conv_pre(mel)
        for i in range(6):
            x = self.resblock_group(self.upsample(x, i), i)
        return x

    def post(self, x):
        """run_bigvgan_post_cpu (:4030): activation_post, conv k=7 24 -> 1 (zero bias), clamp."""
        x = self.activation("bigvgan.activation_post", x)
        x = conv1d_same(x, self.conv_weight("bigvgan.conv_post", 1, 24, 7), np.zeros(1, np.float32), 7)
        return np.clip(x, np.float32(-1.0), np.float32(1.0))

    def vocoder(self, mel):
        """run_bigvgan_vocoder_cpu (:4058): mel [tokens, 80] -> waveform [256 * tokens]."""
        return self.post(self.body(mel)).reshape(-1)


# ---------------------------------------------------------------- GPT decoder
GPT_W, GPT_VOCAB = 1280, 8194


def gelu_new(x) -> np.ndarray:
    """cpu_gelu_new (tokenizer_tests.cpp:3931)."""
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_gelu_new(P(x), x.size, P(out))
    return out


def attention_single_query(q, k, v) -> np.ndarray:
    """cpu_attention_single_query (tokenizer_tests.cpp:4034): q [D], k/v [N, D]."""
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty(q.size, np.float32)
    lib().orc_attention_single_query(P(q), P(k), P(v), k.shape[0], q.size, P(out))
    return out


def attention_causal(q, k, v) -> np.ndarray:
    """cpu_attention_single_head_causal (tokenizer_tests.cpp:4003): q/k/v [T, D]."""
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty_like(q)
    lib().orc_attention_causal(P(q), P(k), P(v), q.shape[0], q.shape[1], P(out))
    return out


def gpt_sampling_processors(logits, history, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0):
    """apply_gpt_sampling_processors (gpt.cpp:1618)."""
    x = f32(logits)
    h = u32(history)
    out = np.empty_like(x)
    if lib().orc_gpt_sampling_processors(P(x), x.size, PU(h), h.size, temperature, top_k, top_p,
                                         repetition_penalty, P(out)) != 0:
        raise ValueError("invalid sampling setting")
    return out


def gpt_sample_token(processed, rng_state):
    """sample_gpt_token_from_logits (gpt.cpp:1720); rng_state is a one-element
    numpy uint64 array, advanced in place."""
    x = f32(processed)
    st = ctypes.c_uint64(int(rng_state[0]))
    tok = lib().orc_gpt_sample_token(P(x), x.size, ctypes.byref(st))
    rng_state[0] = st.value
    return int(tok)


class GPT:
    """The reference's fp32 CPU GPT decoder (runtime/impl/gpt.cpp) over the given
    gpt.* tensors (checkpoint layouts; layers 0..L-1 present)."""

    def __init__(self, tensors: dict):
        layers = 0
        while f"gpt.gpt.h.{layers}.ln_1.weight" in tensors:
            layers += 1
        self.layers = layers
        self._h = lib().orc_gpt_new(layers)
        if not self._h:
            raise ValueError("GPT oracle: bad layer count")
        for name, v in tensors.items():
            if not name.startswith("gpt."):
                continue
            a = f32(v)
            if lib().orc_gpt_set(self._h, name.encode(), P(a), a.size) != 0:
                raise ValueError(lib().orc_gpt_last_error().decode())
        if lib().orc_gpt_missing(self._h):
            raise ValueError(f"GPT oracle: {lib().orc_gpt_missing(self._h)} tensors missing")

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h and _lib is not None:
            _lib.orc_gpt_free(h)

    def layer_qkv(self, x, layer):
        """run_gpt_layer_qkv_cpu (gpt.cpp:1060): [T, 1280] -> [T, 3840]."""
        x = f32(x).reshape(-1, GPT_W)
        out = np.empty((x.shape[0], 3 * GPT_W), np.float32)
        lib().orc_gpt_layer_qkv(self._h, P(x), x.shape[0], layer, P(out))
        return out

    def block(self, x, layer):
        """run_gpt_transformer_block_cpu_layer (gpt.cpp:658)."""
        x = f32(x).reshape(-1, GPT_W)
        out = np.empty_like(x)
        lib().orc_gpt_block(self._h, P(x), x.shape[0], layer, P(out))
        return out

    def cached_block_current(self, cache_k, cache_v, current, current_qkv, layer):
        """run_gpt_cached_block_current_cpu (gpt.cpp:1180)."""
        ck, cv = f32(cache_k).reshape(-1, GPT_W), f32(cache_v).reshape(-1, GPT_W)
        cur, cq = f32(current), f32(current_qkv)
        out = np.empty(GPT_W, np.float32)
        lib().orc_gpt_cached_block_current(self._h, P(ck), P(cv), ck.shape[0], P(cur), P(cq), layer, P(out))
        return out

    def logits(self, x):
        """run_gpt_logits_cpu (gpt.cpp:1310): (final_norm [T, 1280], logits [T, 8194], last argmax)."""
        x = f32(x).reshape(-1, GPT_W)
        fn = np.empty_like(x)
        lg = np.empty((x.shape[0], GPT_VOCAB), np.float32)
        am = lib().orc_gpt_logits(self._h, P(x), x.shape[0], P(fn), P(lg))
        return fn, lg, int(am)

    def cached_decode(self, rows, prefix_tokens):
        """run_gpt_cached_decode_cpu (gpt.cpp:1400): (ln_f, final_norm, logits, argmax)."""
        x = f32(rows).reshape(-1, GPT_W)
        ln_f = np.empty(GPT_W, np.float32)
        fn = np.empty(GPT_W, np.float32)
        lg = np.empty(GPT_VOCAB, np.float32)
        am = lib().orc_gpt_cached_decode(self._h, P(x), prefix_tokens, P(ln_f), P(fn), P(lg))
        return ln_f, fn, lg, int(am)

    def _greedy(self, fn, prefix, steps, *extra):
        x = f32(prefix).reshape(-1, GPT_W)
        pred = np.zeros(max(steps, 1), np.uint32)
        inp = np.zeros(steps + 1, np.uint32)
        lg = np.zeros(GPT_VOCAB, np.float32)
        r = _GreedyResult()
        rc = fn(self._h, P(x), x.shape[0], steps, *extra, PU(pred), PU(inp), P(lg), ctypes.byref(r))
        if rc != 0:
            raise ValueError("GPT oracle: position beyond the mel position table")
        return {"predicted": pred[:r.n_predicted].copy(), "input_tokens": inp[:r.n_input].copy(),
                "first_stop_step": int(r.first_stop_step), "last_logits": lg if steps > 0 else None}

    def kv_greedy(self, prefix, steps, hf_generate_positions=False):
        """run_gpt_kv_greedy_cpu (gpt.cpp:1877)."""
        return self._greedy(lib().orc_gpt_kv_greedy, prefix, steps, 1 if hf_generate_positions else 0)

    def kv_sample(self, prefix, steps, seed, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0,
                  hf_generate_positions=False, history=None):
        """The sampled cached loop (gpt.cpp:2221-2240); also returns
        last_processed_logits.  history: repetition_history_prefix (None: the
        start token; an empty list: an empty prefix, the predictions alone)."""
        hist = np.ascontiguousarray(np.asarray(history if history is not None else [], np.uint32))
        hbuf = np.zeros(max(hist.size, 1), np.uint32)  # a valid pointer for an empty prefix too
        hbuf[:hist.size] = hist
        x = f32(prefix).reshape(-1, GPT_W)
        pred = np.zeros(max(steps, 1), np.uint32)
        inp = np.zeros(steps + 1, np.uint32)
        lg = np.zeros(GPT_VOCAB, np.float32)
        lp = np.zeros(GPT_VOCAB, np.float32)
        r = _GreedyResult()
        rc = lib().orc_gpt_kv_sample(self._h, P(x), x.shape[0], steps, 1 if hf_generate_positions else 0, seed,
                                     temperature, top_k, top_p, repetition_penalty,
                                     PU(hbuf) if history is not None else None, hist.size, PU(pred), PU(inp), P(lg),
                                     P(lp), ctypes.byref(r))
        if rc != 0:
            raise ValueError("GPT oracle: invalid sampling setting or position beyond the table")
        return {"predicted": pred[:r.n_predicted].copy(), "input_tokens": inp[:r.n_input].copy(),
                "first_stop_step": int(r.first_stop_step), "last_logits": lg if steps > 0 else None,
                "last_processed_logits": lp if steps > 0 else None}

    def greedy_full(self, prefix, steps):
        """run_gpt_greedy_cpu (gpt.cpp:1833): the uncached loop (no stop)."""
        return self._greedy(lib().orc_gpt_greedy_full, prefix, steps)
