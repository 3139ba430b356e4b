"""The reference's own call shape and threading contract on the GPU.

* An MIT2 bundle on disk -> context -> decode (mit2::Bundle,
  runtime/include/mit2/bundle.hpp:46-79, then run_cfm_euler_metal(metal,
  bundle, ...), dit_cfm_bigvgan.cpp:3121): through the C ABI
  (mit2cfm_create_from_bundle) and through the C++ shim
  (mit2::HipContext(const Bundle&)) that the mtts-cfm CLI uses.  Both must
  give the same bits as a context built from the same tensors in memory, and
  the CLI's --test-cfm-euler[-cfg] harnesses (dit_cfm_bigvgan.cpp:3306-3409)
  are held against the CPU oracle's output for their inputs.
* One context per thread (the reference runs a second MetalContext on its
  AcousticWorker thread, synthesis_pipeline.cpp:1100-1225): two contexts
  decoding concurrently from two host threads give the serial runs' bits.
"""
from __future__ import annotations

import json
import subprocess
import threading

import numpy as np
import pytest

from conftest import sincos_series

pytestmark = pytest.mark.gpu

MEL_TOL = 1e-2  # final mel rel-L2 (the decode's parity bar)


@pytest.fixture(scope="module")
def bundle_dir(mit2, tmp_path_factory):
    d = tmp_path_factory.mktemp("mit2") / "synthetic_bundle"
    mit2.write_synthetic_bundle(d, 20240605, 0.02)  # the `tensors` fixture's weights
    return d


@pytest.fixture(scope="module")
def cli(mit2):
    exe = mit2.LIB_PATH.parent / "mtts-cfm"
    assert exe.exists(), f"{exe} not built"
    return str(exe)


def _inputs(mit2, T, P, seed):
    x0 = mit2.normal_noise(T, 80, seed)
    cond = mit2.normal_noise(T, 512, seed + 1)
    style = mit2.normal_noise(1, 192, seed + 2)[0]
    prompt = mit2.normal_noise(max(P, 1), 80, seed + 3, 2.0)[:P] - 5.0
    return x0, prompt, cond, style


def test_bundle_context_decode_equals_tensor_context(mit2, orc, model, tensors, bundle_dir):
    T, P, S, cfg = 96, 24, 4, 0.7
    inp = _inputs(mit2, T, P, 11)
    with mit2.Context(bundle=bundle_dir, device=0) as cb:
        got = cb.decode(*inp, S, cfg)
    with mit2.Context(tensors, device=0) as ct:
        ref_gpu = ct.decode(*inp, S, cfg)
    assert np.array_equal(got, ref_gpu)
    ref = model.cfm_euler(*inp, S, cfg)
    err = orc.rel_l2(got, ref)
    print(f"bundle context decode T={T} S={S}: rel-L2 {err:.3e} vs oracle", flush=True)
    assert err <= MEL_TOL


def test_cli_decode_on_bundle_equals_library(mit2, tensors, cli, bundle_dir, tmp_path):
    """mtts-cfm --decode BUNDLE (HipContext(const Bundle&)) writes the same mel
    as the library decode of the same seeded inputs from in-memory tensors."""
    T, P, S, seed = 60, 12, 12, 3
    out = tmp_path / "mel.f32"
    r = subprocess.run([cli, "--decode", str(bundle_dir), str(T), str(P), "--cfm_steps", str(S),
                        "--seed", str(seed), "--out", str(out)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    got = np.fromfile(out, np.float32).reshape(T, 80)
    x0 = mit2.normal_noise(T, 80, seed)
    prompt = mit2.normal_noise(P, 80, seed + 1, 2.0) - 5.0
    cond = mit2.normal_noise(T, 512, seed + 2)
    style = mit2.normal_noise(1, 192, seed + 3)[0]
    with mit2.Context(tensors, device=0) as c:
        ref = c.decode(x0, prompt, cond, style, S, 0.7)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("flag,steps,cfg", [("--test-cfm-euler", 3, 0.0), ("--test-cfm-euler-cfg", 25, 0.5)])
def test_cli_cfm_euler_harness_against_cpu_path(orc, model, cli, bundle_dir, tmp_path, flag, steps, cfg):
    """The reference's harness inputs (dit_cfm_bigvgan.cpp:3306-3326, T=5, P=2);
    the CPU path's result comes from the oracle through --expect."""
    T, P = 5, 2
    x = sincos_series(T * 80, 0.018, 0.011, 0.07, 0.03, 61).reshape(T, 80)
    i = np.arange(P * 80)
    prompt = (np.cos(i.astype(np.float32) * np.float32(0.022)) * np.float32(0.09)
              + np.sin((i % 37).astype(np.float32) * np.float32(0.019)) * np.float32(0.02)).astype(np.float32).reshape(P, 80)
    cond = sincos_series(T * 512, 0.009, 0.014, 0.08, 0.04, 109).reshape(T, 512)
    style = (np.cos(np.arange(192, dtype=np.float32) * np.float32(0.015)) * np.float32(0.18)).astype(np.float32)
    ref = model.cfm_euler(x, prompt, cond, style, steps, cfg)
    exp = tmp_path / "expect.f32"
    ref.astype(np.float32).tofile(exp)
    r = subprocess.run([cli, flag, str(bundle_dir), "--expect", str(exp)], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    d = json.loads(r.stdout)
    assert d["steps"] == steps and d["nonfinite"] == 0 and d["prompt_rows_max_abs"] == 0
    assert d["rel_l2_error"] <= MEL_TOL
    assert d["max_abs_error"] <= 1e-4 and d["meets_reference_bar"]  # the reference's own bar (:3340)


def test_two_contexts_on_two_threads(mit2, tensors):
    """Each thread drives its own context (its own stream) concurrently; every
    result equals the serial run bit for bit."""
    ca = mit2.Context(tensors, device=0)
    cb = mit2.Context(tensors, device=0)
    try:
        ia, ib = _inputs(mit2, 300, 60, 21), _inputs(mit2, 212, 40, 31)
        ra = ca.decode(*ia, 8, 0.7)
        rb = cb.decode(*ib, 8, 0.7)
        results, errors = {}, []

        def work(ctx, inp, key):
            try:
                results[key] = [ctx.decode(*inp, 8, 0.7) for _ in range(6)]
            except Exception as e:  # reported below
                errors.append(e)

        ts = [threading.Thread(target=work, args=(ca, ia, "a")), threading.Thread(target=work, args=(cb, ib, "b"))]
        for t in ts:
            t.start()
        for t in ts:
            t.join(timeout=240)
        assert not errors, errors
        assert not any(t.is_alive() for t in ts)
        assert all(np.array_equal(o, ra) for o in results["a"])
        assert all(np.array_equal(o, rb) for o in results["b"])
    finally:
        ca.close()
        cb.close()


def _reference_series(T, P):
    """The reference harnesses' inputs (dit_cfm_bigvgan.cpp:3306-3326, :3415-3422)."""
    x = sincos_series(T * 80, 0.018, 0.011, 0.07, 0.03, 61).reshape(T, 80)
    i = np.arange(P * 80)
    prompt = (np.cos(i.astype(np.float32) * np.float32(0.022)) * np.float32(0.09)
              + np.sin((i % 37).astype(np.float32) * np.float32(0.019)) * np.float32(0.02)).astype(np.float32).reshape(P, 80)
    cond = sincos_series(T * 512, 0.009, 0.014, 0.08, 0.04, 109).reshape(T, 512)
    style = (np.cos(np.arange(192, dtype=np.float32) * np.float32(0.015)) * np.float32(0.18)).astype(np.float32)
    return x, prompt, cond, style


def test_cli_cfm_euler_cfg_large_against_cpu_path(model, cli, bundle_dir, tmp_path):
    """--test-cfm-euler-cfg-large (dit_cfm_bigvgan.cpp:3411-3443): T=173, P=8,
    cfg 0.5, decoded with 1 and with 3 steps; the CPU path's two results come
    from the oracle through --expect, held to the reference's max-abs 3e-3."""
    T, P = 173, 8
    x, prompt, cond, style = _reference_series(T, P)
    ref = np.stack([model.cfm_euler(x, prompt, cond, style, s, 0.5) for s in (1, 3)])
    exp = tmp_path / "expect_large.f32"
    ref.astype(np.float32).tofile(exp)
    r = subprocess.run([cli, "--test-cfm-euler-cfg-large", str(bundle_dir), "--expect", str(exp)],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    d = json.loads(r.stdout)
    assert d["ok"] and [s["steps"] for s in d["steps"]] == [1, 3]
    for s in d["steps"]:
        assert s["pass"] and s["max_abs_error"] <= 3e-3 and s["repeat_max_abs_error"] == 0
        assert s["rel_l2_error"] <= MEL_TOL


def test_cli_s2mel_full_inputs_round_trips_config3(mit2, cli, bundle_dir, tmp_path):
    """--test-s2mel-full-inputs (dit_cfm_bigvgan.cpp:3516-3604) on the caller's
    tensor files: the T=128 (P=48) 12-step fixture's inputs, regenerated from
    its seeds, against the oracle's decode of them (tests/golden/config3), at
    the reference's max-abs 3e-3 over the full and the generated mel."""
    import json as _json
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden"
    meta = _json.loads((golden / "config3.json").read_text())
    with np.load(golden / "config3.npz") as z:
        expected = z["final"]
    T, P, S, cfg = meta["T"], meta["P"], meta["steps"], meta["cfg"]
    x0, prompt, cond, style = _inputs(mit2, T, P, meta["seed"])
    files = {}
    for name, arr in (("noise", x0), ("prompt", prompt), ("cond", cond), ("style", style), ("expected", expected)):
        files[name] = tmp_path / f"{name}.f32"
        np.ascontiguousarray(arr, np.float32).tofile(files[name])
    args = [cli, "--test-s2mel-full-inputs", str(bundle_dir), str(files["noise"]), str(files["prompt"]),
            str(files["cond"]), str(files["style"]), str(S), str(cfg), str(files["expected"])]
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    d = json.loads(r.stdout)
    assert d["ok"] and (d["tokens"], d["prompt_tokens"], d["generated_tokens"], d["steps"]) == (T, P, T - P, S)
    assert d["full_vs_expected_max_abs_error"] <= 3e-3 and d["generated_vs_expected_max_abs_error"] <= 3e-3
    assert d["full_vs_expected_rel_l2_error"] <= MEL_TOL


@pytest.mark.parametrize("tokens", [64, 300])
def test_cli_dit_attention_tokens_against_cpu_path(model, cli, bundle_dir, tmp_path, tokens):
    """--test-dit-attention-tokens (dit_cfm_bigvgan.cpp:584-638): the layer-0
    attention core on the reference's input series at N tokens, against the
    oracle's attention core through --expect (max-abs 1e-3), a batch of two
    whose first branch matches, and the reference's determinism gate (repeat
    error exactly 0)."""
    n = tokens * 512
    i = np.arange(n)
    x = (np.sin(i.astype(np.float32) * np.float32(0.017)) * np.float32(0.13)
         + np.cos((i % 97).astype(np.float32) * np.float32(0.011)) * np.float32(0.09)).astype(np.float32)
    ref = model.attention_core(x.reshape(tokens, 512), np.ones(tokens, np.uint32), 0)
    exp = tmp_path / "expect_attn.f32"
    ref.astype(np.float32).tofile(exp)
    r = subprocess.run([cli, "--test-dit-attention-tokens", str(bundle_dir), str(tokens), "--expect", str(exp)],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    d = json.loads(r.stdout)
    assert d["ok"] and d["tokens"] == tokens and d["batched_repeat_err"] == 0
    assert d["max_abs_error"] <= 1e-3 and d["batched_branch0_err"] <= 1e-3
