"""Python binding of the gfx950 DiT-CFM decoder (ctypes over include/mit2cfm.h).

Mirrors the reference's entry points for this path -- run_cfm_euler_metal
(runtime/impl/dit_cfm_bigvgan.cpp:3121), run_dit_estimator_step_metal (:2778)
and the per-stage test harnesses (:74-2860) -- with numpy arrays in place of
std::vector<float>.  All compute goes through build/libmit2cfm.so; when that
library is missing every call raises instead of falling back to anything.
"""
from __future__ import annotations

import concurrent.futures
import ctypes
import os
import re
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "build" / "libmit2cfm.so"
HEADER_PATH = PKG_DIR.parent / "include" / "mit2cfm.h"
PREFIX = "s2mel.net.cfm.estimator."

OK, E_ARG, E_MODEL, E_HIP, E_INTERNAL = 0, 1, 2, 3, 4
DTYPE_F32, DTYPE_F16 = 0, 1
FLAG_SYNC = 1
STAGES = {"length_regulator": 1, "vocoder": 2}  # MIT2CFM_STAGE_*
PRECISIONS = {"f16": 0, "f32": 1}  # MIT2CFM_PREC_*
PADDING = {"compute": 0, "skip": 1}  # MIT2CFM_PADDING_*
NOALLOC_MAX_CODES = 1024  # MIT2CFM_NOALLOC_MAX_CODES

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_lib = None


class Mit2CfmError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"mit2cfm status {status}: {message}")
        self.status = status


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("data", ctypes.c_void_p),
                ("elems", ctypes.c_uint64), ("dtype", ctypes.c_int32)]


def lib() -> ctypes.CDLL:
    """Loads build/libmit2cfm.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
    L = ctypes.CDLL(str(LIB_PATH))
    st = ctypes.c_int32
    vp = ctypes.c_void_p
    u32, u64, i32, f32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32, ctypes.c_float
    sig = {
        "mit2cfm_abi_version": (i32, []),
        "mit2cfm_last_error": (ctypes.c_char_p, [vp]),
        "mit2cfm_create": (st, [ctypes.POINTER(_Tensor), u32, i32, ctypes.POINTER(vp)]),
        "mit2cfm_create_from_bundle": (st, [ctypes.c_char_p, i32, ctypes.POINTER(vp)]),
        "mit2cfm_create_synthetic": (st, [u64, f32, i32, ctypes.POINTER(vp)]),
        "mit2cfm_destroy": (None, [vp]),
        "mit2cfm_decode": (st, [vp, _f32p, _f32p, _f32p, _f32p, u32, u32, u32, f32, _f32p]),
        "mit2cfm_decode_device": (st, [vp, vp, vp, vp, vp, u32, u32, u32, f32, vp, u32]),
        "mit2cfm_decode_trace": (st, [vp, _f32p, _f32p, _f32p, _f32p, u32, u32, u32, f32, _f32p, _f32p]),
        "mit2cfm_decode_batched": (st, [vp, u32, u32, _u32p, _u32p, _f32p, _f32p, _f32p, _f32p,
                                        u32, f32, _f32p]),
        "mit2cfm_decode_batched_device": (st, [vp, u32, u32, _u32p, _u32p, vp, vp, vp, vp, u32, f32, vp, u32]),
        "mit2cfm_estimator_step": (st, [vp, _f32p, _f32p, _f32p, _f32p, _u32p, f32, u32, u32, _f32p]),
        "mit2cfm_stream": (vp, [vp]),
        "mit2cfm_synchronize": (st, [vp]),
        "mit2cfm_set_graph": (st, [vp, i32]),
        "mit2cfm_set_padding": (st, [vp, i32]),
        "mit2cfm_get_padding": (st, [vp, ctypes.POINTER(ctypes.c_int32)]),
        "mit2cfm_set_precision": (st, [vp, i32, i32]),
        "mit2cfm_decode_graph_count": (st, [vp, _u32p, _u32p]),
        "mit2cfm_get_precision": (st, [vp, i32, ctypes.POINTER(i32)]),
        "mit2cfm_stage_timestep_embedder": (st, [vp, f32, i32, _f32p]),
        "mit2cfm_stage_input_merge": (st, [vp, _f32p, _f32p, _f32p, _f32p, u32, u32, _f32p]),
        "mit2cfm_stage_adaptive_norm": (st, [vp, _f32p, _f32p, u32, i32, _f32p]),
        "mit2cfm_stage_attention_core": (st, [vp, _f32p, _u32p, u32, u32, i32, _f32p]),
        "mit2cfm_stage_feed_forward": (st, [vp, _f32p, u32, i32, _f32p]),
        "mit2cfm_stage_block": (st, [vp, _f32p, _f32p, _u32p, u32, u32, i32, _f32p, _f32p]),
        "mit2cfm_stage_stack": (st, [vp, _f32p, _f32p, _u32p, u32, u32, _f32p]),
        "mit2cfm_stage_post": (st, [vp, _f32p, _f32p, u32, _f32p, _f32p, _f32p]),
        "mit2cfm_stage_wavenet": (st, [vp, _f32p, _f32p, _u32p, u32, u32, _f32p]),
        "mit2cfm_stage_final_layer": (st, [vp, _f32p, _f32p, u32, _f32p]),
        "mit2cfm_op_linear": (st, [vp, _f32p, _f32p, _f32p, u32, u32, u32, _f32p]),
        "mit2cfm_normal_noise": (st, [u32, u32, u64, f32, _f32p]),
        "mit2cfm_synthetic_tensor_count": (u32, []),
        "mit2cfm_synthetic_tensor_info": (st, [u32, ctypes.POINTER(ctypes.c_char_p), _u32p,
                                               ctypes.POINTER(ctypes.c_int64),
                                               ctypes.POINTER(ctypes.c_int32),
                                               ctypes.POINTER(ctypes.c_uint64)]),
        "mit2cfm_synthetic_tensor_fill": (st, [u32, u64, f32, vp]),
        "mit2cfm_write_synthetic_bundle": (st, [ctypes.c_char_p, u64, f32]),
        "mit2cfm_profile_launch": (st, [vp, i32, u32, ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_char_p)]),
        "mit2cfm_inspect_bundle": (st, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.POINTER(ctypes.c_uint64), u32]),
        "mit2cfm_length_regulator": (st, [vp, _f32p, u32, u32, _f32p]),
        "mit2cfm_condition": (st, [vp, _f32p, u32, _f32p, u32, _f32p, _u32p]),
        "mit2cfm_condition_device": (st, [vp, vp, u32, vp, u32, vp, _u32p, u32]),
        "mit2cfm_condition_device_noalloc": (st, [vp, vp, u32, vp, u32, vp, _u32p, u32]),
        "mit2cfm_generated_frames": (u32, [u32]),
        "mit2cfm_noise_device": (st, [vp, u32, u32, u64, f32, vp, u32]),
        "mit2cfm_bigvgan": (st, [vp, _f32p, u32, _f32p]),
        "mit2cfm_bigvgan_device": (st, [vp, vp, u32, vp, u32]),
        "mit2cfm_bigvgan_stage": (st, [vp, i32, i32, _f32p, u32, _f32p, u64]),
        "mit2cfm_bigvgan_stage_floats": (u64, [i32, i32, u32, i32]),
        "mit2cfm_acoustic_device": (st, [vp, vp, u32, vp, vp, u32, vp, u64, f32, u32, f32, vp, vp, _u32p,
                                         u32]),
        "mit2cfm_synthetic_set_count": (u32, [i32]),
        "mit2cfm_synthetic_set_info": (st, [i32, u32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(u32),
                                            ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(i32),
                                            ctypes.POINTER(u64)]),
        "mit2cfm_synthetic_set_fill": (st, [i32, u32, u64, f32, vp]),
        "mit2cfm_create_synthetic_acoustic": (st, [u64, f32, i32, ctypes.POINTER(vp)]),
        "mit2cfm_write_image": (st, [vp, ctypes.c_char_p]),
        "mit2cfm_create_from_image": (st, [ctypes.c_char_p, i32, ctypes.POINTER(vp)]),
        "mit2cfm_gpt_layers": (st, [vp, _u32p]),
        "mit2cfm_gpt_kv_greedy": (st, [vp, _f32p, u32, u32, i32, _u32p, _u32p, _u32p, _u32p,
                                       ctypes.POINTER(i32), _f32p, ctypes.POINTER(ctypes.c_double)]),
        "mit2cfm_gpt_cached_decode": (st, [vp, _f32p, u32, _f32p, _f32p, _f32p, _u32p]),
        "mit2cfm_gpt_kv_sample": (st, [vp, _f32p, u32, u32, i32, ctypes.POINTER(_GptSampling), _u32p, u32, _u32p,
                                       _u32p, _u32p, _u32p, ctypes.POINTER(i32), _f32p, _f32p,
                                       ctypes.POINTER(ctypes.c_double)]),
        "mit2cfm_gpt_profile_launch": (st, [vp, i32, u32, ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_char_p)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class _GptSampling(ctypes.Structure):
    _fields_ = [("seed", ctypes.c_uint64), ("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("top_p", ctypes.c_float), ("repetition_penalty", ctypes.c_float)]


def declared_symbols() -> list[str]:
    """Function names declared in include/mit2cfm.h."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"\b(mit2cfm_[a-z0-9_]+)\s*\(", text)))


def _check(status: int, ctx=None) -> None:
    if status != OK:
        msg = lib().mit2cfm_last_error(ctx)
        raise Mit2CfmError(status, msg.decode() if msg else "")


def _f32(a, shape=None) -> np.ndarray:
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    if shape is not None and arr.size != int(np.prod(shape)):
        raise ValueError(f"expected {int(np.prod(shape))} elements, got {arr.size}")
    return arr


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def _p(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def _pu(a: np.ndarray):
    return a.ctypes.data_as(_u32p)


# ---------------------------------------------------------------- synthetic data
def normal_noise(tokens: int, channels: int, seed: int, temperature: float = 1.0) -> np.ndarray:
    """make_deterministic_normal_noise (tokenizer_tests.cpp:2121): [tokens, channels]."""
    out = np.empty((tokens, channels), np.float32)
    _check(lib().mit2cfm_normal_noise(tokens, channels, seed, temperature, _p(out)))
    return out


def synthetic_tensor_specs() -> list[tuple[str, tuple[int, ...], str]]:
    L = lib()
    specs = []
    for i in range(L.mit2cfm_synthetic_tensor_count()):
        name = ctypes.c_char_p()
        ndim = ctypes.c_uint32()
        shape = (ctypes.c_int64 * 4)()
        dt = ctypes.c_int32()
        n = ctypes.c_uint64()
        _check(L.mit2cfm_synthetic_tensor_info(i, ctypes.byref(name), ctypes.byref(ndim), shape,
                                               ctypes.byref(dt), ctypes.byref(n)))
        specs.append((name.value.decode(), tuple(shape[d] for d in range(ndim.value)),
                      "f16" if dt.value == DTYPE_F16 else "f32"))
    return specs


def synthetic_tensors(seed: int = 20240605, stddev: float = 0.02) -> dict[str, np.ndarray]:
    """Every estimator tensor, N(0, stddev) f16 from seed + (index in sorted-name order)."""
    L = lib()
    out = {}
    for i, (name, shape, dt) in enumerate(synthetic_tensor_specs()):
        arr = np.empty(shape, np.float16 if dt == "f16" else np.float32)
        _check(L.mit2cfm_synthetic_tensor_fill(i, seed, stddev, arr.ctypes.data_as(ctypes.c_void_p)))
        out[name] = arr
    return out


LR_PREFIX = "s2mel.net.length_regulator."


def generated_frames(codes: int) -> int:
    """floor(codes * 1.72f): frames the condition producer makes from `codes` tokens."""
    return int(lib().mit2cfm_generated_frames(codes))


SYNTH_ESTIMATOR, SYNTH_LENGTH_REGULATOR, SYNTH_BIGVGAN, SYNTH_GPT = 0, 1, 2, 3


def synthetic_set_specs(set_id: int) -> list[tuple[str, tuple[int, ...], str]]:
    """(name, shape, dtype) of every tensor of a synthetic set, sorted by name."""
    L = lib()
    specs = []
    for i in range(L.mit2cfm_synthetic_set_count(set_id)):
        name = ctypes.c_char_p()
        ndim = ctypes.c_uint32()
        shape = (ctypes.c_int64 * 4)()
        dt = ctypes.c_int32()
        n = ctypes.c_uint64()
        _check(L.mit2cfm_synthetic_set_info(set_id, i, ctypes.byref(name), ctypes.byref(ndim), shape,
                                            ctypes.byref(dt), ctypes.byref(n)))
        specs.append((name.value.decode(), tuple(shape[d] for d in range(ndim.value)),
                      "f16" if dt.value == DTYPE_F16 else "f32"))
    return specs


def synthetic_set(set_id: int, seed: int, stddev: float, keep=None) -> dict[str, np.ndarray]:
    """Every tensor of a synthetic set (or those whose name `keep` accepts),
    generated by the library (one generator for the C++ runtime, the tests and
    the bench)."""
    L = lib()
    out, jobs = {}, []
    for i, (name, shape, dt) in enumerate(synthetic_set_specs(set_id)):
        if keep is not None and not keep(name):
            continue
        arr = np.empty(shape, np.float16 if dt == "f16" else np.float32)
        out[name] = arr
        jobs.append((i, arr))

    def fill(job):  # ctypes releases the GIL, so tensors fill in parallel
        i, arr = job
        return L.mit2cfm_synthetic_set_fill(set_id, i, seed, stddev, arr.ctypes.data_as(ctypes.c_void_p))

    workers = max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else 4))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        for status in pool.map(fill, jobs):
            _check(status)
    return out


def length_regulator_specs() -> list[tuple[str, tuple[int, ...]]]:
    """The s2mel length regulator's tensors (gpt.cpp:5271-5340), sorted by name."""
    return [(n, shape) for n, shape, _ in synthetic_set_specs(SYNTH_LENGTH_REGULATOR)]


def synthetic_lr_tensors(seed: int = 20240606, stddev: float = 0.02) -> dict[str, np.ndarray]:
    """Length-regulator weights, f16: N(0, stddev) from seed + (index in sorted-name
    order); GroupNorm weights are 1 + N(0, stddev)."""
    return synthetic_set(SYNTH_LENGTH_REGULATOR, seed, stddev)


# BigVGAN v2 (22 kHz, 80 bands, 256x) as the reference runs it
# (dit_cfm_bigvgan.cpp:3606-4062): upsamplers (prefix, in, out, kernel, stride,
# padding) and resblocks (prefix, channels, kernel).
BIGVGAN_UPSAMPLERS = [("bigvgan.ups.0.0", 1536, 768, 8, 4, 2), ("bigvgan.ups.1.0", 768, 384, 8, 4, 2),
                      ("bigvgan.ups.2.0", 384, 192, 4, 2, 1), ("bigvgan.ups.3.0", 192, 96, 4, 2, 1),
                      ("bigvgan.ups.4.0", 96, 48, 4, 2, 1), ("bigvgan.ups.5.0", 48, 24, 4, 2, 1)]
BIGVGAN_RESBLOCKS = [(f"bigvgan.resblocks.{3 * g + i}", 768 >> g, (3, 7, 11)[i])
                     for g in range(6) for i in range(3)]


def bigvgan_specs() -> list[tuple[str, tuple[int, ...]]]:
    """The vocoder's tensors with their checkpoint shapes, sorted by name.  Convs are
    weight-normed (weight_g, weight_v); a transposed conv's weight_v is [in, out, kernel]
    and its weight_g [in, 1, 1]; each anti-aliased activation holds a 12-tap upsample
    and low-pass filter and SnakeBeta's log-scale alpha and beta."""
    return [(n, shape) for n, shape, _ in synthetic_set_specs(SYNTH_BIGVGAN)]


def kaiser_sinc_filter(kernel: int = 12, cutoff: float = 0.25, half_width: float = 0.3) -> np.ndarray:
    """The anti-aliasing filter of BigVGAN's alias-free activation for ratio 2: a
    Kaiser-windowed sinc low-pass, normalised to unit DC gain (Kaiser's
    empirical beta for the attenuation A = 2.285 (N/2 - 1) pi (4 half_width) + 7.95).
    numpy's own restatement, against which the library's filter is checked."""
    half = kernel // 2
    a = 2.285 * (half - 1) * np.pi * (4 * half_width) + 7.95
    if a > 50.0:
        beta = 0.1102 * (a - 8.7)
    elif a >= 21.0:
        beta = 0.5842 * (a - 21.0) ** 0.4 + 0.07886 * (a - 21.0)
    else:
        beta = 0.0
    window = np.kaiser(kernel, beta)
    time = (np.arange(-half, half) + 0.5) if kernel % 2 == 0 else (np.arange(kernel) - half)
    f = 2 * cutoff * window * np.sinc(2 * cutoff * time)
    return (f / f.sum()).astype(np.float32)


def synthetic_bigvgan_tensors(seed: int = 20240607, stddev: float = 0.02) -> dict[str, np.ndarray]:
    """Vocoder weights from the library's generator: weight_v and biases N(0, stddev)
    f16 from seed + (index in sorted-name order); weight_g = g (1 + N(0, stddev)) with
    g = 0.6 for the resblock convs (the per-row norm of the normalised weight, so the
    stack neither explodes nor vanishes), 1 for conv_pre and the upsamplers, 0.1 for
    conv_post; the filters the Kaiser-sinc low-pass (f32); SnakeBeta's log alpha and
    log beta N(0, 0.1) (f32)."""
    return synthetic_set(SYNTH_BIGVGAN, seed, stddev)


def bigvgan_flops(tokens: int) -> float:
    """Algorithmic conv FLOPs of the vocoder on `tokens` mel frames: 2 MACs per weight
    tap per output (conv_pre, the six transposed convs counted on their input,
    the 108 resblock convs, conv_post); the activations are element-wise work."""
    f = 2.0 * tokens * 1536 * 80 * 7
    t = tokens
    for (_, cin, cout, k, s, _), g in zip(BIGVGAN_UPSAMPLERS, range(6)):
        f += 2.0 * t * cin * cout * k
        t *= s
        c = cout
        f += sum(6 * 2.0 * t * c * c * kk for kk in (3, 7, 11))
    return f + 2.0 * t * 24 * 7


# The GPT-2 stack of IndexTTS2's mel-code decoder (gpt.cpp): width, heads,
# MLP width, vocabulary (8192 codes + start 8192 + stop 8193), position rows.
GPT_WIDTH, GPT_HEADS, GPT_MLP, GPT_VOCAB, GPT_POSITIONS = 1280, 20, 5120, 8194, 1818
GPT_START_TOKEN, GPT_STOP_TOKEN = 8192, 8193


def synthetic_gpt_tensors(layers: int = 24, seed: int = 20240608, stddev: float = 0.02) -> dict[str, np.ndarray]:
    """GPT decoder weights from the library's generator (checkpoint names and
    layouts, Conv1D weights [in][out], f16): N(0, stddev) from seed + (index in
    sorted-name order of the 24-layer set), LayerNorm weights 1 + N(0, stddev).
    `layers` < 24 keeps layers 0..layers-1 (a shallower model for fast tests)."""
    def keep(name: str) -> bool:
        if name.startswith("gpt.gpt.h."):
            return int(name.split(".")[3]) < layers
        return True
    return synthetic_set(SYNTH_GPT, seed, stddev, keep)


def gpt_step_bytes(layers: int = 24) -> float:
    """Algorithmic HBM bytes of one decode step's weights (f16): per layer
    c_attn, attn c_proj, c_fc, mlp c_proj; plus mel_head."""
    w = GPT_WIDTH
    return 2.0 * (layers * (3 * w * w + w * w + 2 * GPT_MLP * w) + GPT_VOCAB * w)


def write_synthetic_bundle(path: str | os.PathLike, seed: int = 20240605, stddev: float = 0.02) -> None:
    _check(lib().mit2cfm_write_synthetic_bundle(str(path).encode(), seed, stddev))


def inspect_bundle(path: str | os.PathLike, verify_sha256: bool = False) -> tuple[int, int]:
    """Opens a bundle with the C++ loader (all validation rules); returns
    (tensor count, payload bytes).  Raises Mit2CfmError on a bad bundle."""
    count = ctypes.c_uint64()
    nbytes = ctypes.c_uint64()
    _check(lib().mit2cfm_inspect_bundle(str(path).encode(), ctypes.byref(count), ctypes.byref(nbytes),
                                        1 if verify_sha256 else 0))
    return count.value, nbytes.value


# ---------------------------------------------------------------- context
class Context:
    """One GPU context with resident weights (mit2cfm_ctx)."""

    def __init__(self, tensors: dict[str, np.ndarray] | None = None, *, bundle=None, image=None,
                 synthetic_seed: int | None = None, stddev: float = 0.02, acoustic: bool = False,
                 device: int = 0):
        """From a tensor dict, an MIT2 bundle directory, a device image
        (write_image), or the library's synthetic weights (acoustic: also the
        length regulator's and the vocoder's, seeds synthetic_seed + 1, + 2)."""
        L = lib()
        handle = ctypes.c_void_p()
        if bundle is not None:
            _check(L.mit2cfm_create_from_bundle(str(bundle).encode(), device, ctypes.byref(handle)))
        elif image is not None:
            _check(L.mit2cfm_create_from_image(str(image).encode(), device, ctypes.byref(handle)))
        elif synthetic_seed is not None:
            create = L.mit2cfm_create_synthetic_acoustic if acoustic else L.mit2cfm_create_synthetic
            _check(create(synthetic_seed, stddev, device, ctypes.byref(handle)))
        else:
            if tensors is None:
                raise ValueError("need tensors, bundle or synthetic_seed")
            keep = []
            arr = (_Tensor * len(tensors))()
            for i, (name, v) in enumerate(tensors.items()):
                a = np.ascontiguousarray(v)
                if a.dtype == np.float16:
                    dt = DTYPE_F16
                else:
                    a = np.ascontiguousarray(a, dtype=np.float32)
                    dt = DTYPE_F32
                keep.append(a)
                arr[i] = _Tensor(name.encode(), a.ctypes.data, a.size, dt)
            _check(L.mit2cfm_create(arr, len(tensors), device, ctypes.byref(handle)))
        self._h = handle

    def write_image(self, path) -> None:
        """Saves the prepared device weights to a device image file."""
        self._c(lib().mit2cfm_write_image(self._h, str(path).encode()))

    # -- lifetime
    def close(self) -> None:
        if self._h:
            lib().mit2cfm_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _c(self, status: int) -> None:
        _check(status, self._h)

    # -- decode
    def decode(self, x0, prompt, cond, style, steps: int, cfg_rate: float) -> np.ndarray:
        """run_cfm_euler (dit_cfm_bigvgan.cpp:2908/3121): x0 [T,80], prompt [P,80],
        cond [T,512], style [192] -> x [T,80]."""
        x0 = _f32(x0)
        T = x0.size // 80
        prompt = _f32(prompt)
        P = prompt.size // 80
        cond = _f32(cond, (T, 512))
        style = _f32(style, (192,))
        out = np.empty((T, 80), np.float32)
        self._c(lib().mit2cfm_decode(self._h, _p(x0), _p(prompt) if P else None, _p(cond), _p(style),
                                     T, P, steps, cfg_rate, _p(out)))
        return out

    def decode_trace(self, x0, prompt, cond, style, steps: int, cfg_rate: float):
        """Decode plus the guided velocity of every step: (x [T,80], v [steps,T,80])."""
        x0 = _f32(x0)
        T = x0.size // 80
        prompt = _f32(prompt)
        P = prompt.size // 80
        cond = _f32(cond, (T, 512))
        style = _f32(style, (192,))
        out = np.empty((T, 80), np.float32)
        v = np.empty((steps, T, 80), np.float32)
        self._c(lib().mit2cfm_decode_trace(self._h, _p(x0), _p(prompt) if P else None, _p(cond),
                                           _p(style), T, P, steps, cfg_rate, _p(out), _p(v)))
        return out, v

    def decode_batched(self, tokens, prompt_tokens, x0, prompt, cond, style, steps: int,
                       cfg_rate: float) -> np.ndarray:
        """nreq right-padded requests: x0/prompt [nreq,Tmax,80], cond [nreq,Tmax,512],
        style [nreq,192], tokens/prompt_tokens [nreq] -> [nreq,Tmax,80]."""
        tokens = _u32(tokens)
        prompt_tokens = _u32(prompt_tokens)
        x0 = _f32(x0)
        nreq = tokens.size
        Tm = x0.size // (nreq * 80)
        prompt = _f32(prompt, (nreq, Tm, 80))
        cond = _f32(cond, (nreq, Tm, 512))
        style = _f32(style, (nreq, 192))
        out = np.empty((nreq, Tm, 80), np.float32)
        self._c(lib().mit2cfm_decode_batched(self._h, nreq, Tm, _pu(tokens), _pu(prompt_tokens),
                                             _p(x0), _p(prompt), _p(cond), _p(style), steps,
                                             cfg_rate, _p(out)))
        return out

    def decode_batched_device(self, tokens, prompt_tokens, x0_ptr: int, prompt_ptr: int, cond_ptr: int,
                              style_ptr: int, t_max: int, steps: int, cfg_rate: float, out_ptr: int,
                              sync: bool = False) -> None:
        """decode_batched on device buffers (raw addresses; tokens / prompt_tokens host arrays)."""
        tokens = _u32(tokens)
        prompt_tokens = _u32(prompt_tokens)
        self._c(lib().mit2cfm_decode_batched_device(self._h, tokens.size, t_max, _pu(tokens), _pu(prompt_tokens),
                                                    x0_ptr, prompt_ptr, cond_ptr, style_ptr, steps, cfg_rate,
                                                    out_ptr, FLAG_SYNC if sync else 0))

    def decode_device(self, x0_ptr: int, prompt_ptr: int, cond_ptr: int, style_ptr: int,
                      tokens: int, prompt_tokens: int, steps: int, cfg_rate: float, out_ptr: int,
                      sync: bool = False) -> None:
        """Decode on device buffers already in HBM (raw device addresses)."""
        self._c(lib().mit2cfm_decode_device(self._h, x0_ptr, prompt_ptr, cond_ptr, style_ptr,
                                            tokens, prompt_tokens, steps, cfg_rate, out_ptr,
                                            FLAG_SYNC if sync else 0))

    def estimator_step(self, x, prompt_x, cond, style, key_mask, t: float) -> np.ndarray:
        """run_dit_estimator_step (dit_cfm_bigvgan.cpp:1768) for B branches:
        x, prompt_x [B,T,80], cond [B,T,512], style [B,192], key_mask [B,T] -> [B,T,80]."""
        key_mask = _u32(key_mask)
        B, T = key_mask.shape
        x = _f32(x, (B, T, 80))
        prompt_x = _f32(prompt_x, (B, T, 80))
        cond = _f32(cond, (B, T, 512))
        style = _f32(style, (B, 192))
        out = np.empty((B, T, 80), np.float32)
        self._c(lib().mit2cfm_estimator_step(self._h, _p(x), _p(prompt_x), _p(cond), _p(style),
                                             _pu(key_mask), t, B, T, _p(out)))
        return out

    @property
    def stream(self) -> int:
        return lib().mit2cfm_stream(self._h) or 0

    def synchronize(self) -> None:
        self._c(lib().mit2cfm_synchronize(self._h))

    def set_graph(self, on: bool) -> None:
        self._c(lib().mit2cfm_set_graph(self._h, 1 if on else 0))

    def set_padding(self, mode: str) -> None:
        """Padded rows of a ragged batched decode: "compute" (default) or "skip"
        (rows from two past each request's valid length are not computed and
        come back unspecified; valid rows are bit-identical)."""
        self._c(lib().mit2cfm_set_padding(self._h, PADDING[mode]))

    def padding(self) -> str:
        m = ctypes.c_int32()
        self._c(lib().mit2cfm_get_padding(self._h, ctypes.byref(m)))
        return {v: k for k, v in PADDING.items()}[m.value]

    def graph_count(self) -> tuple[int, int]:
        """(decode graphs held now, capacity)."""
        n = np.zeros(1, np.uint32)
        c = np.zeros(1, np.uint32)
        self._c(lib().mit2cfm_decode_graph_count(self._h, _pu(n), _pu(c)))
        return int(n[0]), int(c[0])

    def set_precision(self, stage: str, mode: str) -> None:
        """Arithmetic of a stage the reference runs in fp32: stage "length_regulator" or
        "vocoder", mode "f32" (split f16 operand pairs, the default) or "f16"."""
        self._c(lib().mit2cfm_set_precision(self._h, STAGES[stage], PRECISIONS[mode]))

    def precision(self, stage: str) -> str:
        m = ctypes.c_int32()
        self._c(lib().mit2cfm_get_precision(self._h, STAGES[stage], ctypes.byref(m)))
        return {v: k for k, v in PRECISIONS.items()}[m.value]

    def profile_launch(self, kernel: int, count: int):
        """Enqueues `count` launches of decode kernel `kernel` on self.stream (no sync);
        returns (name, flops per launch, HBM bytes per launch)."""
        f = ctypes.c_double()
        b = ctypes.c_double()
        n = ctypes.c_char_p()
        self._c(lib().mit2cfm_profile_launch(self._h, kernel, count, ctypes.byref(f), ctypes.byref(b),
                                             ctypes.byref(n)))
        return n.value.decode(), f.value, b.value

    # -- condition and noise producer
    def length_regulator(self, s_infer, out_tokens: int) -> np.ndarray:
        """run_length_regulator_full (gpt.cpp:5298/5313): s_infer [in_tokens, 1024]
        -> [out_tokens, 512]."""
        x = _f32(s_infer)
        in_tokens = x.size // 1024
        out = np.empty((out_tokens, 512), np.float32)
        self._c(lib().mit2cfm_length_regulator(self._h, _p(x), in_tokens, out_tokens, _p(out)))
        return out

    def condition(self, s_infer, prompt_cond, prompt_tokens: int) -> np.ndarray:
        """The decode condition (synthesis_pipeline.cpp:1012-1035): [prompt_cond[:P];
        length_regulator(s_infer, floor(codes * 1.72))] -> [P + generated, 512]."""
        x = _f32(s_infer)
        codes = x.size // 1024
        pc = _f32(prompt_cond)
        if pc.size < prompt_tokens * 512:
            raise ValueError("prompt_cond holds fewer than prompt_tokens rows")
        gen = generated_frames(codes)
        out = np.empty((prompt_tokens + gen, 512), np.float32)
        g = np.zeros(1, np.uint32)
        self._c(lib().mit2cfm_condition(self._h, _p(x), codes, _p(pc), prompt_tokens, _p(out), _pu(g)))
        assert int(g[0]) == gen
        return out

    def condition_device(self, s_infer_ptr: int, codes: int, prompt_ptr: int, prompt_tokens: int,
                         cond_ptr: int, sync: bool = False) -> int:
        """The condition on device buffers (raw addresses); returns the generated frames."""
        g = np.zeros(1, np.uint32)
        self._c(lib().mit2cfm_condition_device(self._h, s_infer_ptr, codes, prompt_ptr, prompt_tokens,
                                               cond_ptr, _pu(g), FLAG_SYNC if sync else 0))
        return int(g[0])

    def condition_device_noalloc(self, s_infer_ptr: int, codes: int, prompt_ptr: int, prompt_tokens: int,
                                 cond_ptr: int, sync: bool = False) -> int:
        """condition_device on the library's static scratch (allocates nothing;
        codes <= NOALLOC_MAX_CODES); returns the generated frames."""
        g = np.zeros(1, np.uint32)
        self._c(lib().mit2cfm_condition_device_noalloc(self._h, s_infer_ptr, codes, prompt_ptr, prompt_tokens,
                                                       cond_ptr, _pu(g), FLAG_SYNC if sync else 0))
        return int(g[0])

    def noise_device(self, tokens: int, channels: int, seed: int, temperature: float, out_ptr: int,
                     sync: bool = False) -> None:
        """make_deterministic_normal_noise (tokenizer_tests.cpp:2121) into a device buffer."""
        self._c(lib().mit2cfm_noise_device(self._h, tokens, channels, seed, temperature, out_ptr,
                                           FLAG_SYNC if sync else 0))

    # -- BigVGAN vocoder
    def bigvgan(self, mel) -> np.ndarray:
        """run_bigvgan_vocoder (dit_cfm_bigvgan.cpp:4058/4196): mel [tokens, 80] -> wav [256 tokens]."""
        x = _f32(mel)
        tokens = x.size // 80
        out = np.empty(256 * tokens, np.float32)
        self._c(lib().mit2cfm_bigvgan(self._h, _p(x), tokens, _p(out)))
        return out

    def bigvgan_device(self, mel_ptr: int, tokens: int, wav_ptr: int, sync: bool = False) -> None:
        self._c(lib().mit2cfm_bigvgan_device(self._h, mel_ptr, tokens, wav_ptr, FLAG_SYNC if sync else 0))

    def acoustic_device(self, s_infer_ptr: int, codes: int, prompt_cond_ptr: int, prompt_mel_ptr: int,
                        prompt_tokens: int, style_ptr: int, seed: int, temperature: float, steps: int,
                        cfg: float, wav_ptr: int, mel_ptr: int = 0, sync: bool = False) -> int:
        """The whole acoustic stage on device buffers (raw addresses): condition,
        seeded noise, CFG decode, vocoder on the generated rows; returns the
        generated frame count (the waveform has 256 samples per frame)."""
        g = np.zeros(1, np.uint32)
        self._c(lib().mit2cfm_acoustic_device(self._h, s_infer_ptr, codes, prompt_cond_ptr, prompt_mel_ptr,
                                              prompt_tokens, style_ptr, seed, temperature, steps, cfg, wav_ptr,
                                              mel_ptr or None, _pu(g), FLAG_SYNC if sync else 0))
        return int(g[0])

    # -- GPT mel-code decoder
    def gpt_layers(self) -> int:
        """Layers of the context's GPT decoder (0: none)."""
        n = np.zeros(1, np.uint32)
        self._c(lib().mit2cfm_gpt_layers(self._h, _pu(n)))
        return int(n[0])

    def gpt_kv_greedy(self, prefix, steps: int, hf_generate_positions: bool = False) -> dict:
        """run_gpt_kv_greedy (gpt.cpp:1877): prefix [P, 1280] -> dict with
        predicted, input_tokens (uint32 arrays), first_stop_step, last_logits
        [8194] (None when steps == 0) and prefill_ms / decode_ms (device time)."""
        x = _f32(prefix).reshape(-1, GPT_WIDTH)
        P = x.shape[0]
        pred = np.zeros(max(steps, 1), np.uint32)
        inp = np.zeros(steps + 1, np.uint32)
        n_pred = np.zeros(1, np.uint32)
        n_in = np.zeros(1, np.uint32)
        stop = ctypes.c_int32()
        logits = np.zeros(GPT_VOCAB, np.float32)
        t = (ctypes.c_double * 2)()
        self._c(lib().mit2cfm_gpt_kv_greedy(self._h, _p(x) if P else None, P, steps,
                                            1 if hf_generate_positions else 0, _pu(pred), _pu(n_pred),
                                            _pu(inp), _pu(n_in), ctypes.byref(stop), _p(logits), t))
        return {"predicted": pred[:n_pred[0]].copy(), "input_tokens": inp[:n_in[0]].copy(),
                "first_stop_step": int(stop.value), "last_logits": logits if steps > 0 else None,
                "prefill_ms": float(t[0]), "decode_ms": float(t[1])}

    def gpt_kv_sample(self, prefix, steps: int, seed: int, temperature: float = 1.0, top_k: int = 0,
                      top_p: float = 1.0, repetition_penalty: float = 1.0,
                      hf_generate_positions: bool = False, history=None) -> dict:
        """The sampled loop (gpt.cpp:2221-2240); as gpt_kv_greedy plus
        last_processed_logits.  history: the repetition-history prefix
        (repetition_history_prefix, gpt.cpp:1918), e.g. the prefix's
        fake_inputs [1] * n + [8192]; None: the start token; []: an empty
        prefix (the history is the predictions alone)."""
        x = _f32(prefix).reshape(-1, GPT_WIDTH)
        P = x.shape[0]
        pred = np.zeros(max(steps, 1), np.uint32)
        inp = np.zeros(steps + 1, np.uint32)
        n_pred = np.zeros(1, np.uint32)
        n_in = np.zeros(1, np.uint32)
        stop = ctypes.c_int32()
        logits = np.zeros(GPT_VOCAB, np.float32)
        proc = np.zeros(GPT_VOCAB, np.float32)
        t = (ctypes.c_double * 2)()
        cfg = _GptSampling(seed, temperature, top_k, top_p, repetition_penalty)
        hist = _u32(history) if history is not None else None
        hbuf = None
        if hist is not None:  # a valid pointer for an empty prefix too
            hbuf = np.zeros(max(hist.size, 1), np.uint32)
            hbuf[:hist.size] = hist
        self._c(lib().mit2cfm_gpt_kv_sample(self._h, _p(x) if P else None, P, steps,
                                            1 if hf_generate_positions else 0, ctypes.byref(cfg),
                                            _pu(hbuf) if hbuf is not None else None,
                                            0 if hist is None else hist.size, _pu(pred),
                                            _pu(n_pred), _pu(inp), _pu(n_in), ctypes.byref(stop), _p(logits),
                                            _p(proc), t))
        return {"predicted": pred[:n_pred[0]].copy(), "input_tokens": inp[:n_in[0]].copy(),
                "first_stop_step": int(stop.value), "last_logits": logits if steps > 0 else None,
                "last_processed_logits": proc if steps > 0 else None,
                "prefill_ms": float(t[0]), "decode_ms": float(t[1])}

    def gpt_cached_decode(self, rows, prefix_tokens: int):
        """run_gpt_cached_decode (gpt.cpp:1400): rows [P + 1, 1280] -> (ln_f,
        final_norm, logits, argmax) of the last row."""
        x = _f32(rows).reshape(-1, GPT_WIDTH)
        if x.shape[0] != prefix_tokens + 1:
            raise ValueError(f"rows must hold prefix_tokens + 1 = {prefix_tokens + 1} rows, got {x.shape[0]}")
        ln_f = np.empty(GPT_WIDTH, np.float32)
        fn = np.empty(GPT_WIDTH, np.float32)
        logits = np.empty(GPT_VOCAB, np.float32)
        am = np.zeros(1, np.uint32)
        self._c(lib().mit2cfm_gpt_cached_decode(self._h, _p(x), prefix_tokens, _p(ln_f), _p(fn), _p(logits),
                                                _pu(am)))
        return ln_f, fn, logits, int(am[0])

    GPT_KERNELS = {"c_attn": 0, "attn_proj": 1, "c_fc": 2, "mlp_proj": 3, "mel_head": 4, "attention": 5}

    def gpt_profile_launch(self, kernel: int, count: int):
        """Enqueues `count` launches of one GPT decode kernel (ids in mit2cfm.h)
        on the context stream; returns (name, algorithmic bytes per launch)."""
        b = ctypes.c_double()
        nm = ctypes.c_char_p()
        self._c(lib().mit2cfm_gpt_profile_launch(self._h, kernel, count, ctypes.byref(b), ctypes.byref(nm)))
        return nm.value.decode(), float(b.value)

    BIGVGAN_STAGES = {"conv_pre": 0, "upsample": 1, "activation": 2, "resblock": 3, "group": 4, "post": 5,
                      "body": 6}

    def bigvgan_stage(self, stage: str, index: int, x) -> np.ndarray:
        """One vocoder stage (ids in mit2cfm.h); x is [tokens, channels]; returns
        [out_tokens, out_channels] (post: [tokens])."""
        sid = self.BIGVGAN_STAGES[stage]
        x = _f32(x)
        tokens = x.shape[0]
        n_in = lib().mit2cfm_bigvgan_stage_floats(sid, index, tokens, 0)
        n_out = lib().mit2cfm_bigvgan_stage_floats(sid, index, tokens, 1)
        if n_in != x.size:
            raise ValueError(f"stage {stage}[{index}] takes {n_in} floats for {tokens} tokens, got {x.size}")
        out = np.empty(n_out, np.float32)
        self._c(lib().mit2cfm_bigvgan_stage(self._h, sid, index, _p(x), tokens, _p(out), n_out))
        if stage == "post":
            return out
        if stage == "upsample":
            s = 4 if index < 2 else 2
            return out.reshape(tokens * s, -1)
        if stage == "body":
            return out.reshape(tokens * 256, 24)
        return out.reshape(tokens, -1)

    # -- stages (parity harness)
    def timestep_embedder(self, t: float, which: int) -> np.ndarray:
        out = np.empty(512, np.float32)
        self._c(lib().mit2cfm_stage_timestep_embedder(self._h, t, which, _p(out)))
        return out

    def input_merge(self, x, prompt_x, cond, style) -> np.ndarray:
        x = _f32(x)
        B, T = x.shape[0], x.shape[1]
        out = np.empty((B, T, 512), np.float32)
        self._c(lib().mit2cfm_stage_input_merge(
            self._h, _p(x), _p(_f32(prompt_x, (B, T, 80))), _p(_f32(cond, (B, T, 512))),
            _p(_f32(style, (B, 192))), B, T, _p(out)))
        return out

    def adaptive_norm(self, x, t1, norm_id: int) -> np.ndarray:
        x = _f32(x)
        rows = x.size // 512
        out = np.empty((rows, 512), np.float32)
        self._c(lib().mit2cfm_stage_adaptive_norm(self._h, _p(x), _p(_f32(t1, (512,))), rows,
                                                  norm_id, _p(out)))
        return out

    def attention_core(self, x, key_mask, layer: int) -> np.ndarray:
        key_mask = _u32(key_mask)
        B, T = key_mask.shape
        x = _f32(x, (B, T, 512))
        out = np.empty((B, T, 512), np.float32)
        self._c(lib().mit2cfm_stage_attention_core(self._h, _p(x), _pu(key_mask), B, T, layer,
                                                   _p(out)))
        return out

    def feed_forward(self, x, layer: int) -> np.ndarray:
        x = _f32(x)
        rows = x.size // 512
        out = np.empty((rows, 512), np.float32)
        self._c(lib().mit2cfm_stage_feed_forward(self._h, _p(x), rows, layer, _p(out)))
        return out

    def block(self, x, t1, key_mask, layer: int, skip=None) -> np.ndarray:
        key_mask = _u32(key_mask)
        B, T = key_mask.shape
        x = _f32(x, (B, T, 512))
        sk = None if skip is None else _f32(skip, (B, T, 512))
        out = np.empty((B, T, 512), np.float32)
        self._c(lib().mit2cfm_stage_block(self._h, _p(x), _p(_f32(t1, (512,))), _pu(key_mask), B,
                                          T, layer, None if sk is None else _p(sk), _p(out)))
        return out

    def stack(self, x, t1, key_mask) -> np.ndarray:
        key_mask = _u32(key_mask)
        B, T = key_mask.shape
        x = _f32(x, (B, T, 512))
        out = np.empty((B, T, 512), np.float32)
        self._c(lib().mit2cfm_stage_stack(self._h, _p(x), _p(_f32(t1, (512,))), _pu(key_mask), B,
                                          T, _p(out)))
        return out

    def post(self, xres, xmel):
        xres = _f32(xres)
        rows = xres.size // 512
        xmel = _f32(xmel, (rows, 80))
        ls = np.empty((rows, 512), np.float32)
        c1 = np.empty((rows, 512), np.float32)
        rp = np.empty((rows, 512), np.float32)
        self._c(lib().mit2cfm_stage_post(self._h, _p(xres), _p(xmel), rows, _p(ls), _p(c1), _p(rp)))
        return ls, c1, rp

    def wavenet(self, x, t2, key_mask) -> np.ndarray:
        key_mask = _u32(key_mask)
        B, T = key_mask.shape
        x = _f32(x, (B, T, 512))
        out = np.empty((B, T, 512), np.float32)
        self._c(lib().mit2cfm_stage_wavenet(self._h, _p(x), _p(_f32(t2, (512,))), _pu(key_mask), B,
                                            T, _p(out)))
        return out

    def final_layer(self, x, t1) -> np.ndarray:
        x = _f32(x)
        rows = x.size // 512
        out = np.empty((rows, 512), np.float32)
        self._c(lib().mit2cfm_stage_final_layer(self._h, _p(x), _p(_f32(t1, (512,))), rows, _p(out)))
        return out

    def linear(self, a, w, bias=None) -> np.ndarray:
        a = _f32(a)
        w = _f32(w)
        M, K = a.shape
        N = w.shape[0]
        out = np.empty((M, N), np.float32)
        b = None if bias is None else _f32(bias, (N,))
        self._c(lib().mit2cfm_op_linear(self._h, _p(a), _p(w), None if b is None else _p(b), M, N, K,
                                        _p(out)))
        return out


# Reference-named conveniences ------------------------------------------------
def run_cfm_euler(ctx: Context, x, prompt, cond, style, tokens: int, prompt_tokens: int,
                  steps: int, cfg_rate: float) -> np.ndarray:
    """run_cfm_euler_metal (dit_cfm_bigvgan.cpp:3121) signature."""
    x = _f32(x, (tokens, 80))
    prompt = _f32(prompt, (prompt_tokens, 80))
    return ctx.decode(x, prompt, cond, style, steps, cfg_rate)


def run_dit_estimator_step(ctx: Context, x, prompt_x, cond, style, timestep: float, mask,
                           tokens: int) -> np.ndarray:
    """run_dit_estimator_step_metal (dit_cfm_bigvgan.cpp:2778) signature, one branch."""
    return ctx.estimator_step(_f32(x, (tokens, 80))[None], _f32(prompt_x, (tokens, 80))[None],
                              _f32(cond, (tokens, 512))[None], _f32(style, (192,))[None],
                              _u32(mask).reshape(1, tokens), timestep)[0]
