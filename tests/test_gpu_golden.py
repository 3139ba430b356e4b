"""GPU parity at the benchmark workloads' full sizes against committed oracle
fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

  config1  one estimator forward of the CFG pair, T=256, P=96, t=0.5
  config2  full decode T=860 (P=258), 25 steps, cfg 0.7 -- the headline decode
  config3  full decode T=128 (P=48), 12 steps, cfg 0.7

Inputs and synthetic weights are regenerated from the seeds stored beside each
fixture (splitmix64 + Box-Muller, bit-exact on any host); the weights digest
guards against a generator change.  Bars: velocity rel-L2 <= 2e-3 per step
(the GPU estimator pair on the oracle's own state of that step) and final mel
rel-L2 <= 1e-2 after the whole decode.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
VEL_TOL = 2e-3
MEL_TOL = 1e-2


def load(name):
    meta = json.loads((GOLDEN / f"{name}.json").read_text())
    with np.load(GOLDEN / f"{name}.npz") as z:
        data = {k: z[k] for k in z.files}
    return meta, data


@pytest.fixture(scope="module")
def golden_ctx(mit2, tensors):
    meta, _ = load("config1")
    assert (meta["weight_seed"], meta["weight_std"]) == (20240605, 0.02)
    h = hashlib.sha256()
    for name in sorted(tensors):
        h.update(name.encode())
        h.update(np.ascontiguousarray(tensors[name]).tobytes())
    assert h.hexdigest() == meta["weights_sha256"], "synthetic weight generator changed"
    c = mit2.Context(tensors, device=0)
    yield c
    c.close()


def inputs(mit2, T, P, seed):
    x0 = mit2.normal_noise(T, 80, seed)
    cond = mit2.normal_noise(T, 512, seed + 1)
    style = mit2.normal_noise(1, 192, seed + 2)[0]
    prompt = mit2.normal_noise(max(P, 1), 80, seed + 3, 2.0)[:P] - 5.0
    return x0, prompt, cond, style


def branches(x, prompt, cond, style, T, P):
    px = np.zeros((T, 80), np.float32)
    px[:P] = prompt
    return (np.stack([x, x]), np.stack([px, np.zeros_like(px)]),
            np.stack([cond, np.zeros_like(cond)]), np.stack([style, np.zeros_like(style)]))


def step_time(s, steps):
    """t of Euler step s: t accumulated in fp32 by dt = 1/steps."""
    t = np.float32(0.0)
    dt = np.float32(1.0 / steps)
    for _ in range(s):
        t = np.float32(t + dt)
    return float(t)


def test_config1_forward(mit2, orc, golden_ctx):
    meta, ref = load("config1")
    T, P = meta["T"], meta["P"]
    x0, prompt, cond, style = inputs(mit2, T, P, meta["seed"])
    x = x0.copy()
    x[:P] = 0
    X, PX, C, S = branches(x, prompt, cond, style, T, P)
    d = golden_ctx.estimator_step(X, PX, C, S, np.ones((2, T), np.uint32), meta["t"])
    for b, key in enumerate(("dphi_cond", "dphi_null")):
        err = orc.rel_l2(d[b], ref[key])
        print(f"config1 {key}: rel-L2 {err:.3e}", flush=True)
        assert err <= VEL_TOL


@pytest.mark.parametrize("name", ["config3", "config2"])
def test_decode_golden(mit2, orc, golden_ctx, name):
    meta, ref = load(name)
    T, P, steps, cfg = meta["T"], meta["P"], meta["steps"], meta["cfg"]
    x0, prompt, cond, style = inputs(mit2, T, P, meta["seed"])
    mask = np.ones((2, T), np.uint32)
    for s in meta["keep_steps"]:
        X, PX, C, S = branches(ref[f"x_step{s}"], prompt, cond, style, T, P)
        d = golden_ctx.estimator_step(X, PX, C, S, mask, step_time(s, steps))
        v = np.float32(1 + cfg) * d[0] - np.float32(cfg) * d[1]
        err = orc.rel_l2(v, ref[f"v_step{s}"])
        print(f"{name} step {s}: velocity rel-L2 {err:.3e}", flush=True)
        assert err <= VEL_TOL
    got = golden_ctx.decode(x0, prompt, cond, style, steps, cfg)
    err = orc.rel_l2(got, ref["final"])
    print(f"{name} final mel rel-L2 {err:.3e}", flush=True)
    assert err <= MEL_TOL
    assert np.all(got[:P] == 0)


def test_config2_batched_three_requests_properties(mit2, golden_ctx):
    """The headline T=860 request batched with two shorter ones: the T=860 row
    equals the single-request decode bit for bit (rows are independent and the
    padding keys are masked), at full size where the oracle is too slow."""
    meta, _ = load("config2")
    T, P, steps, cfg = meta["T"], meta["P"], meta["steps"], meta["cfg"]
    x0, prompt, cond, style = inputs(mit2, T, P, meta["seed"])
    single = golden_ctx.decode(x0, prompt, cond, style, steps, cfg)
    again = golden_ctx.decode(x0, prompt, cond, style, steps, cfg)
    assert np.array_equal(single, again), "decode is not deterministic"
    toks = [T, 400, 131]
    ptoks = [P, 100, 0]
    X0 = np.zeros((3, T, 80), np.float32)
    PR = np.zeros((3, T, 80), np.float32)
    CO = np.zeros((3, T, 512), np.float32)
    ST = np.zeros((3, 192), np.float32)
    for i, (t, p) in enumerate(zip(toks, ptoks)):
        a, b, c, s = inputs(mit2, t, p, 100 + i) if i else (x0, prompt, cond, style)
        X0[i, :t] = a
        PR[i, :p] = b
        CO[i, :t] = c
        ST[i] = s
    out = golden_ctx.decode_batched(toks, ptoks, X0, PR, CO, ST, steps, cfg)
    diff = np.abs(out[0, :T] - single)
    print(f"batched vs single T={T}: max |diff| {diff.max():.3e}, differing {np.count_nonzero(diff)}",
          flush=True)
    assert np.array_equal(out[0, :T], single)
    assert np.isfinite(out).all()
