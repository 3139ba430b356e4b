"""The C ABI (include/mit2cfm.h) on the CPU: the library loads, exports
exactly the functions the header declares, the header compiles as C and C++,
and calls that need no GPU validate their arguments (no compute calls here)."""
from __future__ import annotations

import ctypes
import re
import shutil
import subprocess

import numpy as np
import pytest


def test_every_declared_symbol_is_exported(mit2):
    L = mit2.lib()
    declared = mit2.declared_symbols()
    assert len(declared) >= 30
    for name in declared:
        assert hasattr(L, name), name


def test_exports_are_exactly_the_declared_functions(mit2):
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", str(mit2.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted({m for m in re.findall(r"\bT (mit2cfm_[a-z0-9_]+)$", out, re.M)})
    assert exported == mit2.declared_symbols()


def test_every_kernel_launch_stub_is_defined(mit2):
    """A kernel whose body the host compilation pass rejects (a GPU-only
    builtin or type reaching it) loses its launch stub without a build error;
    a shared library then links with the stub undefined and the first launch
    fails at load time."""
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-u", str(mit2.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    assert [s for s in out.split() if "__device_stub__" in s] == []


def test_abi_version_matches_header(mit2):
    text = mit2.HEADER_PATH.read_text()
    v = int(re.search(r"#define MIT2CFM_ABI_VERSION (\d+)", text).group(1))
    assert mit2.lib().mit2cfm_abi_version() == v


@pytest.mark.parametrize("lang,compiler", [("c", "gcc"), ("c++", "g++")])
def test_header_is_self_contained(mit2, lang, compiler, tmp_path):
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not available")
    src = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    src.write_text('#include "mit2cfm.h"\nint main(void) { return mit2cfm_abi_version() == '
                   'MIT2CFM_ABI_VERSION ? 0 : 1; }\n')
    std = "-std=c99" if lang == "c" else "-std=c++11"
    subprocess.run([compiler, std, "-Wall", "-Werror", "-pedantic", "-fsyntax-only",
                    f"-I{mit2.HEADER_PATH.parent}", str(src)], check=True)


def test_null_context_and_arguments_are_rejected(mit2):
    L = mit2.lib()
    buf = np.zeros(80, np.float32)
    p = buf.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    assert L.mit2cfm_decode(None, p, p, p, p, 1, 0, 1, 0.7, p) == mit2.E_ARG
    assert b"ctx" in L.mit2cfm_last_error(None)
    assert L.mit2cfm_synchronize(None) == mit2.E_ARG
    assert L.mit2cfm_create_from_bundle(None, 0, None) == mit2.E_ARG
    assert L.mit2cfm_normal_noise(2, 2, 1, 1.0, None) == mit2.E_ARG
    u = (ctypes.c_uint32 * 1)(8)
    assert L.mit2cfm_decode_batched_device(None, 1, 8, u, u, p, p, p, p, 1, 0.7, p, 0) == mit2.E_ARG
    assert L.mit2cfm_set_padding(None, 1) == mit2.E_ARG
    assert L.mit2cfm_get_padding(None, None) == mit2.E_ARG
    L.mit2cfm_destroy(None)  # a no-op


def test_missing_bundle_is_a_model_error(mit2, tmp_path):
    with pytest.raises(mit2.Mit2CfmError) as e:
        mit2.inspect_bundle(tmp_path / "nope")
    assert e.value.status == mit2.E_MODEL


def test_synthetic_inventory(mit2):
    """93 estimator tensors, sorted by name, with the hot path's shapes."""
    specs = mit2.synthetic_tensor_specs()
    names = [s[0] for s in specs]
    assert names == sorted(names)
    assert all(n.startswith(mit2.PREFIX) for n in names)
    d = {n[len(mit2.PREFIX):]: (shape, dt) for n, shape, dt in specs}
    assert d["transformer.layers.0.attention.wqkv.weight"] == ((1536, 512), "f16")
    assert d["wavenet.in_layers.3.conv.conv.weight_v"] == ((1024, 512, 5), "f16")
    assert d["wavenet.res_skip_layers.7.conv.conv.weight_v"] == ((512, 512, 1), "f16")
    assert d["t_embedder.freqs"] == ((128,), "f32")
    assert "transformer.layers.6.skip_in_linear.weight" not in d
    assert d["transformer.layers.7.skip_in_linear.weight"] == ((512, 1024), "f16")
    params = sum(int(np.prod(s)) for s, _ in d.values())
    assert params > 90_000_000


def test_synthetic_generator_is_seeded(mit2):
    a = mit2.synthetic_tensors(3, 0.02)
    b = mit2.synthetic_tensors(3, 0.02)
    c = mit2.synthetic_tensors(4, 0.02)
    k = mit2.PREFIX + "conv2.weight"
    assert np.array_equal(a[k], b[k]) and not np.array_equal(a[k], c[k])
    w = a[mit2.PREFIX + "transformer.layers.5.feed_forward.w2.weight"].astype(np.float64)
    assert abs(w.std() - 0.02) < 1e-3 and abs(w.mean()) < 1e-3


def test_gpt_entry_points_reject_a_null_context(mit2):
    """The GPT decoder's entry points check their context before anything else
    (no GPU is touched)."""
    L = mit2.lib()
    u = np.zeros(4, np.uint32)
    pu = u.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))
    i = ctypes.c_int32()
    f = np.zeros(8194, np.float32)
    pf = f.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    assert L.mit2cfm_gpt_layers(None, pu) == mit2.E_ARG
    assert L.mit2cfm_gpt_kv_greedy(None, None, 0, 1, 0, pu, pu, pu, pu, ctypes.byref(i), pf, None) == mit2.E_ARG
    cfg = mit2._GptSampling(1, 0.8, 30, 0.8, 10.0)
    assert L.mit2cfm_gpt_kv_sample(None, None, 0, 1, 0, ctypes.byref(cfg), None, 0, pu, pu, pu, pu, ctypes.byref(i),
                                   pf, pf, None) == mit2.E_ARG
    assert L.mit2cfm_gpt_cached_decode(None, pf, 0, pf, pf, pf, pu) == mit2.E_ARG
    assert L.mit2cfm_gpt_profile_launch(None, 0, 0, None, None) == mit2.E_ARG


def test_gpt_synthetic_set_inventory(mit2):
    specs = mit2.synthetic_set_specs(mit2.SYNTH_GPT)
    assert len(specs) == 24 * 12 + 8
    shapes = dict((n, s) for n, s, _ in specs)
    assert shapes["gpt.gpt.h.0.attn.c_attn.weight"] == (1280, 3840)  # Conv1D [in][out]
    assert shapes["gpt.mel_pos_embedding.emb.weight"] == (1818, 1280)
    assert shapes["gpt.mel_head.weight"] == (8194, 1280)
    assert abs(mit2.gpt_step_bytes(24) - 0.9647e9) < 1e6
