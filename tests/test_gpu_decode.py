"""GPU parity of the estimator forward and of the full CFG Euler decode, through
the C ABI, against the CPU oracle on identical seeded inputs.

Bars: per-step velocity rel-L2 <= 2e-3 (one estimator forward on
the oracle's own state for that step) and final mel rel-L2 <= 1e-2 after the
decode.  The f16 GEMM operands are the only source of difference (see
test_gpu_stages.py), so both bars are met with margin; the measured values
are printed.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import sincos_series

pytestmark = pytest.mark.gpu

VEL_TOL = 2e-3
MEL_TOL = 1e-2


@pytest.fixture(scope="module")
def ctx(mit2, tensors):
    c = mit2.Context(tensors, device=0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def ctx_unit(mit2, tensors_unit):
    c = mit2.Context(tensors_unit, device=0)
    yield c
    c.close()


def inputs(mit2, T, P, seed=1):
    """Seeded inputs: x0, content, style ~ N(0,1); prompt mel ~ N(-5, 2)."""
    x0 = mit2.normal_noise(T, 80, seed)
    cond = mit2.normal_noise(T, 512, seed + 1)
    style = mit2.normal_noise(1, 192, seed + 2)[0]
    prompt = mit2.normal_noise(max(P, 1), 80, seed + 3, 2.0)[:P] - 5.0
    return x0, prompt, cond, style


def cfg_branches(x, prompt, cond, style, T, P):
    """The (cond, null) branch pair of one Euler step (dit_cfm_bigvgan.cpp:2908-2926)."""
    px = np.zeros((T, 80), np.float32)
    px[:P] = prompt
    X = np.stack([x, x])
    PX = np.stack([px, np.zeros_like(px)])
    C = np.stack([cond, np.zeros_like(cond)])
    S = np.stack([style, np.zeros_like(style)])
    return X, PX, C, S


@pytest.mark.parametrize("which", ["baseline", "unit"])
def test_estimator_step_cfg_pair(mit2, orc, request, which):
    ctx = request.getfixturevalue("ctx" if which == "baseline" else "ctx_unit")
    model = request.getfixturevalue("model" if which == "baseline" else "model_unit")
    T, P, t = 40, 12, 0.37
    x0, prompt, cond, style = inputs(mit2, T, P, 11)
    x0[:P] = 0
    X, PX, C, S = cfg_branches(x0, prompt, cond, style, T, P)
    mask = np.ones((2, T), np.uint32)
    got = ctx.estimator_step(X, PX, C, S, mask, t)
    for b in range(2):
        ref = model.estimator_step(X[b], PX[b], C[b], S[b], t, mask[b])
        err = orc.rel_l2(got[b], ref)
        print(f"estimator {which} branch {b}: rel-L2 {err:.3e}")
        assert err <= VEL_TOL


def test_estimator_step_masked_reference_inputs(orc, model_unit, ctx_unit):
    """--test-dit-estimator-step shape: T=6, t=0.37, 4 valid tokens (:2829-2860)."""
    T = 6
    x = (np.sin(np.arange(T * 80, dtype=np.float32) * np.float32(0.021)) * 0.10
         + np.cos((np.arange(T * 80) % 53).astype(np.float32) * np.float32(0.017)) * 0.04).reshape(T, 80)
    px = (np.cos(np.arange(T * 80, dtype=np.float32) * np.float32(0.019)) * 0.08
          + np.sin((np.arange(T * 80) % 47).astype(np.float32) * np.float32(0.023)) * 0.03).reshape(T, 80)
    cond = sincos_series(T * 512, 0.010, 0.013, 0.09, 0.05, 127).reshape(T, 512)
    style = (np.cos(np.arange(192, dtype=np.float32) * np.float32(0.016)) * 0.20).astype(np.float32)
    mask = np.array([1, 1, 1, 1, 0, 0], np.uint32)
    got = ctx_unit.estimator_step(x[None], px[None], cond[None], style[None], mask[None], 0.37)[0]
    ref = model_unit.estimator_step(x, px, cond, style, 0.37, mask)
    err = orc.rel_l2(got, ref)
    print(f"estimator T=6 masked: rel-L2 {err:.3e}")
    assert err <= VEL_TOL


def test_config1_one_forward_T256(mit2, orc, model, ctx):
    """Config 1: B=2 CFG pair, T=256 (96 prompt), t=0.5, N(0,0.02) weights."""
    T, P, t = 256, 96, 0.5
    x0, prompt, cond, style = inputs(mit2, T, P, 1)
    x0[:P] = 0
    X, PX, C, S = cfg_branches(x0, prompt, cond, style, T, P)
    mask = np.ones((2, T), np.uint32)
    got = ctx.estimator_step(X, PX, C, S, mask, t)
    for b in range(2):
        ref = model.estimator_step(X[b], PX[b], C[b], S[b], t, mask[b])
        err = orc.rel_l2(got[b], ref)
        print(f"config1 branch {b}: rel-L2 {err:.3e}")
        assert err <= VEL_TOL


@pytest.mark.parametrize("steps,cfg", [(3, 0.0), (25, 0.5)])
def test_cfm_euler_reference_shape(orc, model_unit, ctx_unit, steps, cfg):
    """--test-cfm-euler / --test-cfm-euler-cfg: T=5, P=2 (dit_cfm_bigvgan.cpp:3306-3409)."""
    T, P = 5, 2
    x = sincos_series(T * 80, 0.018, 0.011, 0.07, 0.03, 61).reshape(T, 80)
    prompt = (np.cos(np.arange(P * 80, dtype=np.float32) * np.float32(0.022)) * 0.09
              + np.sin((np.arange(P * 80) % 37).astype(np.float32) * np.float32(0.019)) * 0.02).reshape(P, 80)
    cond = sincos_series(T * 512, 0.009, 0.014, 0.08, 0.04, 109).reshape(T, 512)
    style = (np.cos(np.arange(192, dtype=np.float32) * np.float32(0.015)) * 0.18).astype(np.float32)
    got = ctx_unit.decode(x, prompt, cond, style, steps, cfg)
    ref = model_unit.cfm_euler(x, prompt, cond, style, steps, cfg)
    err = orc.rel_l2(got, ref)
    print(f"cfm_euler T=5 steps={steps} cfg={cfg}: rel-L2 {err:.3e}")
    assert err <= MEL_TOL
    assert np.all(got[:P] == 0)


@pytest.mark.parametrize("which", ["baseline", "unit"])
def test_decode_per_step_velocity(mit2, orc, request, which):
    """Per-step velocity: the GPU estimator pair on the oracle's state of each
    step, blended with cfg, against the oracle's velocity of that step."""
    ctx = request.getfixturevalue("ctx" if which == "baseline" else "ctx_unit")
    model = request.getfixturevalue("model" if which == "baseline" else "model_unit")
    T, P, steps, cfg = 48, 12, 6, 0.7
    x0, prompt, cond, style = inputs(mit2, T, P, 21)
    ref_x, xt, vt = model.cfm_euler(x0, prompt, cond, style, steps, cfg, trace=True)
    mask = np.ones((2, T), np.uint32)
    tv = np.float32(0.0)
    for s in range(steps):
        X, PX, C, S = cfg_branches(xt[s], prompt, cond, style, T, P)
        d = ctx.estimator_step(X, PX, C, S, mask, float(tv))
        v = (np.float32(1 + cfg) * d[0] - np.float32(cfg) * d[1])
        err = orc.rel_l2(v, vt[s])
        print(f"{which} step {s}: velocity rel-L2 {err:.3e}")
        assert err <= VEL_TOL
        tv = np.float32(tv + np.float32(1.0 / steps))
    got = ctx.decode(x0, prompt, cond, style, steps, cfg)
    err = orc.rel_l2(got, ref_x)
    print(f"{which} final mel rel-L2 {err:.3e}")
    assert err <= MEL_TOL


def test_decode_trace_matches_decode(mit2, ctx):
    T, P = 40, 10
    x0, prompt, cond, style = inputs(mit2, T, P, 5)
    a = ctx.decode(x0, prompt, cond, style, 4, 0.7)
    b, v = ctx.decode_trace(x0, prompt, cond, style, 4, 0.7)
    assert np.array_equal(a, b)
    # x_final = zero-prompt( x0 + dt * sum_s v_s ) reconstructs the trajectory
    x = x0.copy()
    x[:P] = 0
    for s in range(4):
        x = x + np.float32(0.25) * v[s]
        x[:P] = 0
    assert np.allclose(x, a, rtol=0, atol=1e-5)


def test_decode_deterministic_and_graph_equal(mit2, ctx):
    T, P = 90, 20
    x0, prompt, cond, style = inputs(mit2, T, P, 7)
    a = ctx.decode(x0, prompt, cond, style, 5, 0.7)
    b = ctx.decode(x0, prompt, cond, style, 5, 0.7)
    ctx.set_graph(False)
    try:
        c = ctx.decode(x0, prompt, cond, style, 5, 0.7)
    finally:
        ctx.set_graph(True)
    assert np.array_equal(a, b)
    assert np.array_equal(a, c)


def test_decode_graph_cache_stays_bounded(mit2, tensors):
    """50 distinct lengths through one context (production T changes every
    segment): the captured decode graphs stay within the cache capacity (least
    recently used evicted), and results do not depend on the cache state: the
    first lengths decoded again after all 50 give the same bits, and so does a
    decode with graph replay off."""
    c = mit2.Context(tensors, device=0)
    try:
        first = {}
        n0, cap = c.graph_count()
        assert n0 == 0 and cap >= 1
        # the longest first: later lengths fit the workspace, so only the LRU evicts
        x0, prompt, cond, style = inputs(mit2, 70, 5, 110)
        c.decode(x0, prompt, cond, style, 2, 0.7)
        for i, T in enumerate(range(20, 70)):
            x0, prompt, cond, style = inputs(mit2, T, 5, 40 + T)
            out = c.decode(x0, prompt, cond, style, 2, 0.7)
            n, _ = c.graph_count()
            assert n == min(i + 2, cap)
            if i < 3:
                first[T] = out
        print(f"graph cache after 50 lengths: {c.graph_count()}", flush=True)
        for T, ref in first.items():
            x0, prompt, cond, style = inputs(mit2, T, 5, 40 + T)
            assert np.array_equal(c.decode(x0, prompt, cond, style, 2, 0.7), ref)
        c.set_graph(False)
        x0, prompt, cond, style = inputs(mit2, 20, 5, 60)
        assert np.array_equal(c.decode(x0, prompt, cond, style, 2, 0.7), first[20])
        assert c.graph_count()[0] <= cap
    finally:
        c.close()


def test_decode_cfg_zero_runs_cond_branch_only(mit2, orc, model, ctx):
    T, P = 24, 6
    x0, prompt, cond, style = inputs(mit2, T, P, 9)
    got = ctx.decode(x0, prompt, cond, style, 3, 0.0)
    ref = model.cfm_euler(x0, prompt, cond, style, 3, 0.0)
    assert orc.rel_l2(got, ref) <= MEL_TOL


def test_batched_requests_match_oracle(mit2, orc, model_unit, ctx_unit):
    """Right-padded batch (config 5 semantics at small size): 3 requests."""
    Tb = np.array([20, 33, 40], np.uint32)
    Pb = np.array([8, 8, 8], np.uint32)
    Tm, n, steps, cfg = 40, 3, 3, 0.7
    x0 = np.stack([mit2.normal_noise(Tm, 80, 100 + r) for r in range(n)])
    prompt = np.stack([mit2.normal_noise(Tm, 80, 200 + r, 2.0) - 5.0 for r in range(n)])
    cond = np.stack([mit2.normal_noise(Tm, 512, 300 + r) for r in range(n)])
    style = np.stack([mit2.normal_noise(1, 192, 400 + r)[0] for r in range(n)])
    got = ctx_unit.decode_batched(Tb, Pb, x0, prompt, cond, style, steps, cfg)
    for r in range(n):
        mask = (np.arange(Tm) < Tb[r]).astype(np.uint32)
        ref = model_unit.cfm_euler_masked(x0[r], prompt[r][:Pb[r]], cond[r], style[r], mask, steps, cfg)
        err = orc.rel_l2(got[r], ref)
        print(f"batched request {r} (T={Tb[r]}): rel-L2 {err:.3e}")
        assert err <= MEL_TOL
        single = ctx_unit.decode_batched(Tb[r:r + 1], Pb[r:r + 1], x0[r:r + 1], prompt[r:r + 1],
                                         cond[r:r + 1], style[r:r + 1], steps, cfg)
        assert np.array_equal(single[0], got[r])


def test_row_tiling_does_not_change_results(mit2, ctx):
    """A short request alone (B=2, M=256 rows: the GEMMs take 32-row tiles)
    and the same request in a batch of eight (M=2048: the wide tiles) give the
    same mel bit for bit -- the tile shape follows M, the K split does not."""
    T, P, steps, cfg = 128, 48, 4, 0.7
    n = 8
    reqs = [inputs(mit2, T, P, seed=500 + 10 * r) for r in range(n)]
    X0 = np.stack([q[0] for q in reqs])
    PR = np.zeros((n, T, 80), np.float32)
    for r in range(n):
        PR[r, :P] = reqs[r][1]
    CO = np.stack([q[2] for q in reqs])
    ST = np.stack([q[3] for q in reqs])
    batch = ctx.decode_batched([T] * n, [P] * n, X0, PR, CO, ST, steps, cfg)
    for r in (0, 5):
        alone = ctx.decode(X0[r], reqs[r][1], CO[r], ST[r], steps, cfg)
        diff = np.abs(alone - batch[r])
        print(f"request {r}: max |alone - batched| {diff.max():.3e}", flush=True)
        assert np.array_equal(alone, batch[r])


@pytest.mark.parametrize("toks", [[5, 63, 64, 130, 199, 200], [200, 5, 198], [40 + 17 * r for r in range(9)]],
                         ids=["edges", "first-full", "nine-requests"])
def test_skipped_padding_keeps_valid_rows(mit2, ctx, toks):
    """MIT2CFM_PADDING_SKIP at its edges: requests shorter than a row tile,
    of exactly a tile, one and two rows short of the padded length (their
    needed rows are clamped to it), a full-length request first, and nine
    requests (18 branches, more than the row skip covers: every row is
    computed).  Each request's valid rows equal the padding-computed decode's
    bit for bit."""
    T, P, steps, cfg = max(toks), 4, 2, 0.7
    n = len(toks)
    reqs = [inputs(mit2, T, P, seed=700 + 10 * r) for r in range(n)]
    X0 = np.stack([q[0] for q in reqs])
    PR = np.zeros((n, T, 80), np.float32)
    for r in range(n):
        PR[r, :P] = reqs[r][1]
    CO = np.stack([q[2] for q in reqs])
    ST = np.stack([q[3] for q in reqs])
    print(f"skipped padding: requests {toks}", flush=True)
    ref = ctx.decode_batched(toks, [P] * n, X0, PR, CO, ST, steps, cfg)
    ctx.set_padding("skip")
    try:
        got = ctx.decode_batched(toks, [P] * n, X0, PR, CO, ST, steps, cfg)
    finally:
        ctx.set_padding("compute")
    for r, t in enumerate(toks):
        assert np.isfinite(got[r, :t]).all()
        assert np.array_equal(got[r, :t], ref[r, :t]), f"request {r} (T={t})"


def test_single_token_decode_is_finite(mit2, ctx):
    """T=1: the reference CPU reflect pad never terminates for one token;
    the HIP path follows the reference GPU kernel (reflect index 0)."""
    x0, prompt, cond, style = inputs(mit2, 1, 0, 3)
    out = ctx.decode(x0, prompt, cond, style, 2, 0.7)
    assert np.isfinite(out).all()


def test_invalid_arguments_raise(mit2, ctx):
    x0, prompt, cond, style = inputs(mit2, 8, 2, 3)
    before = ctx.decode(x0, prompt, cond, style, 2, 0.7)

    def rejected(call):
        with pytest.raises(mit2.Mit2CfmError) as e:
            call()
        assert e.value.status == mit2.E_ARG

    rejected(lambda: ctx.decode(x0, np.zeros((9, 80), np.float32), cond, style, 2, 0.7))  # P > T
    rejected(lambda: ctx.decode(x0, prompt, cond, style, 0, 0.7))  # no steps
    rejected(lambda: ctx.decode(x0, prompt, cond, style, 2, -0.5))  # negative cfg_rate
    rejected(lambda: ctx.decode(x0, prompt, cond, style, 2, float("nan")))
    X0, PR, CO, ST = x0[None], np.zeros((1, 8, 80), np.float32), cond[None], style[None]
    rejected(lambda: ctx.decode_batched([0], [0], X0, PR, CO, ST, 2, 0.7))  # empty request
    rejected(lambda: ctx.decode_batched([9], [2], X0, PR, CO, ST, 2, 0.7))  # longer than T
    rejected(lambda: ctx.decode_batched([4], [5], X0, PR, CO, ST, 2, 0.7))  # prompt > request
    rejected(lambda: ctx.decode_batched_device([8], [2], 0, 0, 0, 0, 8, 2, 0.7, 0))  # NULL buffers
    rejected(lambda: ctx._c(mit2.lib().mit2cfm_set_padding(ctx._h, 7)))  # unknown padding mode
    assert ctx.padding() == "compute"
    # Rejected calls leave the context as it was: the same decode gives the same bits.
    assert np.array_equal(ctx.decode(x0, prompt, cond, style, 2, 0.7), before)
