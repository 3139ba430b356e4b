"""GPU parity at the benchmark workloads' full sizes against committed oracle
fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

  config1  one estimator forward of the CFG pair, T=256, P=96, t=0.5
  config2  full decode T=860 (P=258), 25 steps, cfg 0.7 -- the headline decode
  config3  full decode T=128 (P=48), 12 steps, cfg 0.7
  config4  T=3000 (P=258): CFG-pair velocity at three Euler states
  config4t T=3000: the first 2 Euler steps of the 25-step schedule (the decode's
           own trajectory against the oracle's)
  config5  8 right-padded requests (B=16 rows): masked velocity at t=0, and
           (config5t) the shortest and the longest request after a 2-step batched
           decode, with the padded rows computed and skipped

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


def _make_golden():
    """tests/golden/make_golden.py as a module (shared input recipes)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_config4_long_form_velocity(mit2, orc, golden_ctx):
    """T=3000 (P=258): the CFG-pair velocity at t=0 on x0 and at steps 12 and 24
    of 25 on flow states blended towards a mel-like field, against the oracle
    (the long-sequence attention: 47 key tiles in two groups)."""
    mg = _make_golden()
    meta, ref = load("config4")
    T, P, steps, cfg = meta["T"], meta["P"], meta["steps"], meta["cfg"]
    x0, prompt, cond, style = inputs(mit2, T, P, meta["seed"])
    mask = np.ones((2, T), np.uint32)
    tm = step_time(meta["mid_step"], steps)
    tl = step_time(meta["late_step"], steps)
    x = x0.copy()
    x[:P] = 0
    for key, state, t in (("v_t0", x, 0.0), ("v_mid", mg.mid_state(x0, T, P, meta["seed"], tm), tm),
                          ("v_late", mg.mid_state(x0, T, P, meta["seed"], tl), tl)):
        X, PX, C, S = branches(state, prompt, cond, style, T, P)
        d = golden_ctx.estimator_step(X, PX, C, S, mask, t)
        v = np.float32(1 + cfg) * d[0] - np.float32(cfg) * d[1]
        err = orc.rel_l2(v, ref[key])
        print(f"config4 {key} (t={t:.4f}): velocity rel-L2 {err:.3e}", flush=True)
        assert err <= VEL_TOL


def test_config4_long_form_decode_properties(mit2, golden_ctx):
    """The full 25-step T=3000 decode: finite, prompt rows zero, repeatable bit
    for bit, and unchanged when batched with a shorter request."""
    meta, _ = load("config4")
    T, P, steps, cfg = meta["T"], meta["P"], meta["steps"], meta["cfg"]
    x0, prompt, cond, style = inputs(mit2, T, P, meta["seed"])
    a = golden_ctx.decode(x0, prompt, cond, style, steps, cfg)
    b = golden_ctx.decode(x0, prompt, cond, style, steps, cfg)
    assert np.isfinite(a).all()
    assert np.all(a[:P] == 0)
    assert np.array_equal(a, b)
    X0 = np.zeros((2, T, 80), np.float32)
    PR = np.zeros((2, T, 80), np.float32)
    CO = np.zeros((2, T, 512), np.float32)
    ST = np.zeros((2, 192), np.float32)
    X0[0], PR[0, :P], CO[0], ST[0] = x0, prompt, cond, style
    s0, s1, s2, s3 = inputs(mit2, 900, 100, 77)
    X0[1, :900], PR[1, :100], CO[1, :900], ST[1] = s0, s1, s2, s3
    out = golden_ctx.decode_batched([T, 900], [P, 100], X0, PR, CO, ST, steps, cfg)
    assert np.array_equal(out[0], a)
    golden_ctx.set_padding("skip")
    try:
        skip = golden_ctx.decode_batched([T, 900], [P, 100], X0, PR, CO, ST, steps, cfg)
    finally:
        golden_ctx.set_padding("compute")
    assert np.array_equal(skip[0], a)
    assert np.array_equal(skip[1, :900], out[1, :900])


def test_config4_trajectory_first_steps(mit2, orc, golden_ctx):
    """T=3000 (P=258), the 25-step schedule: the guided velocity of steps 0 and 1
    along the decode's own trajectory (mit2cfm_decode_trace) against the oracle's
    trajectory, and the state after those two steps, rebuilt from the decode's
    velocities (x += dt v, prompt rows zeroed), against the oracle's."""
    meta, ref = load("config4t")
    T, P, steps, cfg = meta["T"], meta["P"], meta["steps"], meta["cfg"]
    x0, prompt, cond, style = inputs(mit2, T, P, meta["seed"])
    _, vt = golden_ctx.decode_trace(x0, prompt, cond, style, steps, cfg)
    x = x0.copy()
    x[:P] = 0
    dt = np.float32(1.0 / steps)
    for s in range(meta["run_steps"]):
        err = orc.rel_l2(vt[s], ref[f"v_step{s}"])
        print(f"config4t step {s}: velocity rel-L2 {err:.3e}", flush=True)
        assert err <= VEL_TOL
        x = (x + dt * vt[s]).astype(np.float32)
        x[:P] = 0
    err = orc.rel_l2(x, ref["x_after"])
    print(f"config4t state after {meta['run_steps']} steps: rel-L2 {err:.3e}", flush=True)
    assert err <= MEL_TOL


def test_config5_padded_batch_velocity(mit2, orc, golden_ctx):
    """8 right-padded requests (P=258, T_max=1348): the masked CFG-pair velocity
    at t=0 of the shortest and the longest request at the padded length, run as
    one B=4 forward, against the oracle's masked estimator."""
    mg = _make_golden()
    meta, ref = load("config5")
    c = dict(meta)
    toks, tmax, X0, PR, CO, ST = mg.padded_requests(c)
    assert toks == meta["tokens"] and tmax == meta["t_max"]
    P, cfg = meta["P"], meta["cfg"]
    Xs, PXs, Cs, Ss, Ms = [], [], [], [], []
    for r in meta["picked"]:
        x = X0[r].copy()
        x[:P] = 0
        X, PX, C, S = branches(x, PR[r][:P], CO[r], ST[r], tmax, P)
        m = (np.arange(tmax) < toks[r]).astype(np.uint32)
        Xs.append(X); PXs.append(PX); Cs.append(C); Ss.append(S); Ms += [m, m]
    d = golden_ctx.estimator_step(np.concatenate(Xs), np.concatenate(PXs), np.concatenate(Cs),
                                  np.concatenate(Ss), np.stack(Ms), 0.0)
    for i, r in enumerate(meta["picked"]):
        v = np.float32(1 + cfg) * d[2 * i] - np.float32(cfg) * d[2 * i + 1]
        err = orc.rel_l2(v[:toks[r]], ref[f"v_t0_req{r}"])
        print(f"config5 request {r} (T={toks[r]}): velocity rel-L2 {err:.3e}", flush=True)
        assert err <= VEL_TOL


@pytest.mark.parametrize("padding", ["compute", "skip"])
def test_config5_padded_batch_trajectory(mit2, orc, golden_ctx, padding):
    """The 8-request right-padded batch (B=16 rows, T_max=1348) decoded for 2
    Euler steps: the final mel of the shortest (T=624) and of the longest
    (T=1348) request against the oracle's masked decode of that request at the
    padded length, with the padded rows computed and with them skipped."""
    mg = _make_golden()
    meta, ref = load("config5t")
    toks, tmax, X0, PR, CO, ST = mg.padded_requests(dict(meta))
    assert toks == meta["tokens"] and tmax == meta["t_max"]
    P, steps, cfg = meta["P"], meta["steps"], meta["cfg"]
    golden_ctx.set_padding(padding)
    try:
        out = golden_ctx.decode_batched(toks, [P] * len(toks), X0, PR, CO, ST, steps, cfg)
    finally:
        golden_ctx.set_padding("compute")
    for r in meta["picked"]:
        err = orc.rel_l2(out[r, :toks[r]], ref[f"final_req{r}"])
        print(f"config5t request {r} (T={toks[r]}, {steps} steps, padding {padding}): final mel "
              f"rel-L2 {err:.3e}", flush=True)
        assert err <= MEL_TOL
        assert np.all(out[r, :P] == 0)


def test_config5_padded_batch_decode(mit2, golden_ctx):
    """The B=16 batched decode (16 steps): finite, prompt rows zero, and each
    checked request equal bit for bit to its own decode at the padded length."""
    mg = _make_golden()
    meta, _ = load("config5")
    toks, tmax, X0, PR, CO, ST = mg.padded_requests(dict(meta))
    P, steps, cfg = meta["P"], meta["steps"], meta["cfg"]
    n = len(toks)
    out = golden_ctx.decode_batched(toks, [P] * n, X0, PR, CO, ST, steps, cfg)
    assert out.shape == (n, tmax, 80)
    for r in range(n):
        assert np.isfinite(out[r, :toks[r]]).all()
        assert np.all(out[r, :P] == 0)
    for r in meta["picked"]:
        one = golden_ctx.decode_batched(toks[r:r + 1], [P], X0[r:r + 1], PR[r:r + 1], CO[r:r + 1],
                                        ST[r:r + 1], steps, cfg)
        assert np.array_equal(one[0], out[r])
    # The same decode from device buffers (mit2cfm_decode_batched_device), bit for bit.
    import torch

    dev = torch.device("cuda:0")
    d_in = [torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev) for a in (X0, PR, CO, ST)]
    d_out = torch.full((n, tmax, 80), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    golden_ctx.decode_batched_device(toks, [P] * n, d_in[0].data_ptr(), d_in[1].data_ptr(),
                                     d_in[2].data_ptr(), d_in[3].data_ptr(), tmax, steps, cfg,
                                     d_out.data_ptr(), sync=True)
    assert np.array_equal(d_out.cpu().numpy(), out)
    # Padded rows skipped (MIT2CFM_PADDING_SKIP): every request's valid rows are
    # the same bits; the padded rows are unspecified.
    golden_ctx.set_padding("skip")
    try:
        assert golden_ctx.padding() == "skip"
        skip = golden_ctx.decode_batched(toks, [P] * n, X0, PR, CO, ST, steps, cfg)
    finally:
        golden_ctx.set_padding("compute")
    for r in range(n):
        assert np.array_equal(skip[r, :toks[r]], out[r, :toks[r]]), f"request {r}"
