"""The mtts-cfm command line (the reference CLI's flags for this path,
runtime/main.cpp:57-88, :2925-2936, :3181-3187, :3293-3342): argument handling
on the CPU; the GPU harnesses (--decode, --test-cfm-euler, --bench-bigvgan,
--test-bigvgan-vocoder) on a GPU.  The file-driven harnesses against the CPU
oracle (--test-cfm-euler-cfg-large, --test-s2mel-full-inputs,
--test-dit-attention-tokens) are in test_gpu_bundle.py."""
from __future__ import annotations

import json
import subprocess

import pytest


@pytest.fixture(scope="module")
def cli(mit2):
    exe = mit2.LIB_PATH.parent / "mtts-cfm"
    if not exe.exists():
        pytest.fail(f"{exe} not built")
    return str(exe)


def _run(cli, *args, timeout=300):
    return subprocess.run([cli, *args], capture_output=True, text=True, timeout=timeout)


def test_usage_without_a_command(cli):
    r = _run(cli)
    assert r.returncode == 2
    assert "--bench-bigvgan" in r.stderr and "--test-gpt-kv-greedy" in r.stderr and "--cfm_steps" not in r.stdout


@pytest.mark.parametrize("steps", ["11", "26", "0"])
def test_cfm_steps_out_of_range_exits_1(cli, steps):
    """main.cpp:3181-3187: --cfm_steps outside 12..25 is an error (exit 1)."""
    r = _run(cli, "--cfm_steps", steps, "--decode", "synthetic", "8", "2")
    assert r.returncode == 1
    assert "between 12 and 25" in r.stderr


def test_s2mel_full_inputs_rejects_bad_shapes_before_the_gpu(cli, tmp_path):
    """--test-s2mel-full-inputs checks its files first (dit_cfm_bigvgan.cpp:3537-3559):
    a noise file that is not [tokens,80] and a style that is not [192] exit 1."""
    import numpy as np

    def f(name, n):
        p = tmp_path / f"{name}.f32"
        np.zeros(n, np.float32).tofile(p)
        return str(p)

    good = dict(noise=f("noise", 8 * 80), prompt=f("prompt", 2 * 80), cond=f("cond", 8 * 512),
                style=f("style", 192), expected=f("expected", 8 * 80))
    for bad, msg in ((dict(noise=f("noise_bad", 8 * 80 + 3)), "[tokens,80]"),
                     (dict(style=f("style_bad", 191)), "[192]"),
                     (dict(prompt=f("prompt_bad", 9 * 80)), "exceeds")):
        a = {**good, **bad}
        r = _run(cli, "--test-s2mel-full-inputs", "synthetic", a["noise"], a["prompt"], a["cond"], a["style"],
                 "2", "0.7", a["expected"])
        assert r.returncode == 1 and msg in r.stderr, r.stderr


def test_synthetic_bundle_roundtrip(mit2, cli, tmp_path):
    d = tmp_path / "bundle"
    assert _run(cli, "--write-synthetic-bundle", str(d), "7", "0.02").returncode == 0
    r = _run(cli, "--inspect-model-bundle", str(d))
    assert r.returncode == 0, r.stdout + r.stderr
    info = json.loads(r.stdout)
    assert info["ok"] is True and info["sha256_verified"] is True
    assert info["tensors"] == len(mit2.synthetic_tensor_specs())


@pytest.mark.gpu
def test_decode_and_invariant_harnesses(cli):
    r = _run(cli, "--decode", "synthetic", "40", "10", "--cfm_steps", "12")
    assert r.returncode == 0, r.stderr
    d = json.loads(r.stdout)
    assert d["tokens"] == 40 and d["steps"] == 12 and d["rms"] > 0
    for flag in ("--test-cfm-euler", "--test-cfm-euler-cfg"):
        r = _run(cli, flag, "synthetic")
        assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
def test_image_roundtrip_through_the_cli(cli, tmp_path):
    img = tmp_path / "m.mit2hip"
    r = _run(cli, "--write-image", "synthetic", str(img))
    assert r.returncode == 0, r.stderr
    a = _run(cli, "--test-bigvgan-vocoder", "synthetic")
    b = _run(cli, "--test-bigvgan-vocoder", f"image:{img}")
    assert a.returncode == 0 and b.returncode == 0, a.stderr + b.stderr
    assert json.loads(a.stdout)["peak_abs"] == json.loads(b.stdout)["peak_abs"]


@pytest.mark.gpu
def test_vocoder_harnesses(cli):
    r = _run(cli, "--test-bigvgan-vocoder", "synthetic")
    assert r.returncode == 0, r.stdout + r.stderr
    d = json.loads(r.stdout)
    assert d["samples"] == 256 and d["nonfinite"] == 0 and d["repeat_max_abs_error"] == 0
    r = _run(cli, "--bench-bigvgan", "synthetic", "16", "2")
    assert r.returncode == 0, r.stderr
    d = json.loads(r.stdout)
    assert d["samples"] == 16 * 256 and d["seconds_per_call"] > 0 and d["rtf_vocoder_only"] > 0


@pytest.mark.gpu
def test_gpt_harnesses(cli):
    r = _run(cli, "--test-gpt-kv-decode", "synthetic")
    assert r.returncode == 0, r.stdout + r.stderr
    d = json.loads(r.stdout)
    assert d["ok"] and d["nonfinite"] == 0 and d["repeat_max_abs_error"] == 0
    r = _run(cli, "--test-gpt-kv-greedy", "synthetic")
    assert r.returncode == 0, r.stdout + r.stderr
    d = json.loads(r.stdout)
    assert d["ok"] and len(d["predicted_tokens"]) == 3
    r = _run(cli, "--bench-gpt", "synthetic", "20", "16", "1")
    assert r.returncode == 0, r.stderr
    d = json.loads(r.stdout)
    assert d["codes"] == 16 and d["seconds_per_call"] > 0
