"""Pins the oracle's estimator stages and Euler decode (CPU) against the
independent float64 torch restatement in torch_ref.py, on both synthetic
weight sets (the benchmark's N(0, 0.02) and the activation-preserving one,
where every stage carries O(1) signal).  fp32 vs float64: rel-L2 <= 1e-4.

Also pins the invariants the reference's own tests rely on: batched-vs-single
independence, cfg = 0 reducing to the cond-only decode, prompt rows held at
zero, and the U-ViT skip wiring (a stack with swapped skip order differs).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import sincos_series
from torch_ref import TorchEstimator, t64

TOL = 1e-4


@pytest.fixture(scope="module")
def tref(tensors):
    return TorchEstimator(tensors)


@pytest.fixture(scope="module")
def tref_unit(tensors_unit):
    return TorchEstimator(tensors_unit)


def _pick(request, which):
    if which == "unit":
        return request.getfixturevalue("model_unit"), request.getfixturevalue("tref_unit")
    return request.getfixturevalue("model"), request.getfixturevalue("tref")


def r(orc, got, ref):
    return orc.rel_l2(got, ref.detach().numpy() if isinstance(ref, torch.Tensor) else ref)


T6 = 6
MASK = np.array([1, 1, 1, 1, 0, 0], np.uint32)
X512 = sincos_series(T6 * 512, 0.019, 0.017, 0.12, 0.07, 113).reshape(T6, 512)
T1 = (np.cos(np.arange(512, dtype=np.float32) * np.float32(0.014)) * 0.25).astype(np.float32)


@pytest.mark.parametrize("which", ["baseline", "unit"])
def test_timestep_embedder(orc, request, which):
    m, t = _pick(request, which)
    for ts in (0.0, 0.37, 1.0):
        for w in (1, 2):
            assert r(orc, m.timestep_embedder(ts, w), t.timestep_embedder(ts, w)) <= TOL


@pytest.mark.parametrize("which", ["baseline", "unit"])
def test_stages(orc, request, which):
    m, t = _pick(request, which)
    x = t64(X512)
    t1 = t64(T1)
    assert r(orc, m.adaptive_norm(X512, T1, 3), t.adaptive_norm(x, t1, "transformer.layers.3.attention_norm")) <= TOL
    assert r(orc, m.adaptive_norm(X512, T1, 26), t.adaptive_norm(x, t1, "transformer.norm")) <= TOL
    assert r(orc, m.attention_core(X512, MASK, 5), t.attention_core(x, MASK, 5)) <= TOL
    assert r(orc, m.feed_forward(X512, 9), t.feed_forward(x, 9)) <= TOL
    skip = sincos_series(T6 * 512, 0.031, 0.019, 0.11, 0.05, 79).reshape(T6, 512)
    assert r(orc, m.block(X512, T1, MASK, 8, skip), t.block(x, t1, MASK, 8, t64(skip))) <= TOL
    assert r(orc, m.block(X512, T1, MASK, 2), t.block(x, t1, MASK, 2)) <= TOL
    xmel = sincos_series(T6 * 80, 0.031, 0.027, 0.18, 0.05, 43).reshape(T6, 80)
    for a, b in zip(m.post(X512, xmel), t.post(x, t64(xmel))):
        assert r(orc, a, b) <= TOL
    assert r(orc, m.wavenet(X512 * 0.5, T1, MASK), t.wavenet(x * 0.5, t1, MASK)) <= TOL
    assert r(orc, m.final_layer(X512, T1), t.final_layer(x, t1)) <= TOL
    style = (np.cos(np.arange(192, dtype=np.float32) * np.float32(0.02)) * 0.2).astype(np.float32)
    cond = sincos_series(T6 * 512, 0.011, 0.017, 0.15, 0.05, 127).reshape(T6, 512)
    assert r(orc, m.input_merge(xmel, xmel * 0.5, cond, style),
             t.input_merge(t64(xmel), t64(xmel * 0.5), t64(cond), t64(style))) <= TOL


@pytest.mark.parametrize("which", ["baseline", "unit"])
def test_stack(orc, request, which):
    m, t = _pick(request, which)
    assert r(orc, m.stack(X512, T1, MASK), t.stack(t64(X512), t64(T1), MASK)) <= TOL


def test_stack_skip_order_matters(model_unit, tref_unit, orc):
    """The LIFO skip schedule (layer 12 - l) is observable: pairing the skips
    first-in-first-out gives a different result from the oracle."""
    x, t1 = t64(X512), t64(T1)
    saved = []
    for layer in range(13):
        skip = saved.pop(0) if layer > 6 else None  # FIFO instead of LIFO
        x = tref_unit.block(x, t1, MASK, layer, skip)
        if layer < 6:
            saved.append(x)
    wrong = tref_unit.adaptive_norm(x, t1, "transformer.norm")
    assert r(orc, model_unit.stack(X512, T1, MASK), wrong) > 1e-2


@pytest.mark.parametrize("which", ["baseline", "unit"])
def test_estimator_step(mit2, orc, request, which):
    m, t = _pick(request, which)
    T = 8
    x = mit2.normal_noise(T, 80, 1)
    px = mit2.normal_noise(T, 80, 2)
    cond = mit2.normal_noise(T, 512, 3)
    style = mit2.normal_noise(1, 192, 4)[0]
    mask = np.array([1, 1, 1, 1, 1, 1, 0, 0], np.uint32)
    got = m.estimator_step(x, px, cond, style, 0.37, mask)
    ref = t.estimator_step(t64(x), t64(px), t64(cond), t64(style), 0.37, mask)
    assert r(orc, got, ref) <= TOL


@pytest.mark.parametrize("which", ["baseline", "unit"])
def test_cfm_euler(mit2, orc, request, which):
    m, t = _pick(request, which)
    T, P = 6, 2
    x0 = mit2.normal_noise(T, 80, 5)
    prompt = mit2.normal_noise(P, 80, 6, 2.0) - 5.0
    cond = mit2.normal_noise(T, 512, 7)
    style = mit2.normal_noise(1, 192, 8)[0]
    got = m.cfm_euler(x0, prompt, cond, style, 3, 0.5)
    ref = t.cfm_euler(t64(x0), t64(prompt), t64(cond), t64(style), 3, 0.5)
    assert r(orc, got, ref) <= TOL
    assert np.all(got[:P] == 0)


def test_cfg_zero_is_cond_only(mit2, model_unit):
    T, P = 6, 2
    x0 = mit2.normal_noise(T, 80, 5)
    prompt = mit2.normal_noise(P, 80, 6)
    cond = mit2.normal_noise(T, 512, 7)
    style = mit2.normal_noise(1, 192, 8)[0]
    got = model_unit.cfm_euler(x0, prompt, cond, style, 2, 0.0)
    # two explicit Euler steps with the cond branch only
    x = x0.copy()
    x[:P] = 0
    px = np.zeros((T, 80), np.float32)
    px[:P] = prompt
    t = np.float32(0)
    for _ in range(2):
        d = model_unit.estimator_step(x, px, cond, style, float(t), np.ones(T, np.uint32))
        x = (x + np.float32(0.5) * d).astype(np.float32)
        x[:P] = 0
        t = np.float32(t + np.float32(0.5))
    assert np.array_equal(got, x)


def test_masked_euler_with_all_ones_equals_unmasked(mit2, model):
    T, P = 6, 2
    x0 = mit2.normal_noise(T, 80, 15)
    prompt = mit2.normal_noise(P, 80, 16)
    cond = mit2.normal_noise(T, 512, 17)
    style = mit2.normal_noise(1, 192, 18)[0]
    a = model.cfm_euler(x0, prompt, cond, style, 2, 0.7)
    b = model.cfm_euler_masked(x0, prompt, cond, style, np.ones(T, np.uint32), 2, 0.7)
    assert np.array_equal(a, b)


def test_oracle_tensor_table_matches_synthetic_inventory(orc, mit2):
    """The oracle's required-tensor table (names, element counts) and the
    product's synthetic inventory are written independently; they must agree."""
    L = orc.lib()
    table = {L.orc_model_tensor_name(i).decode(): L.orc_model_tensor_elems(i)
             for i in range(L.orc_model_tensor_count())}
    inv = {name: int(np.prod(shape)) for name, shape, _ in mit2.synthetic_tensor_specs()}
    assert table == inv


def test_partial_euler_is_a_prefix_of_the_schedule(mit2, model_unit):
    """orc_cfm_euler_partial (the config-4 trajectory fixture): its k steps of the
    S-step schedule are the first k traced steps of the whole decode (same dt),
    not a k-step decode; k = S is the whole decode."""
    T, P, S = 6, 2, 5
    x0 = mit2.normal_noise(T, 80, 25)
    prompt = mit2.normal_noise(P, 80, 26, 2.0) - 5.0
    cond = mit2.normal_noise(T, 512, 27)
    style = mit2.normal_noise(1, 192, 28)[0]
    final, xt, vt = model_unit.cfm_euler(x0, prompt, cond, style, S, 0.7, trace=True)
    x2, xt2, vt2 = model_unit.cfm_euler_partial(x0, prompt, cond, style, S, 2, 0.7)
    assert np.array_equal(vt2, vt[:2]) and np.array_equal(xt2, xt[:2])
    assert np.array_equal(x2, xt[2])
    assert not np.array_equal(x2, model_unit.cfm_euler(x0, prompt, cond, style, 2, 0.7))
    xs, _, _ = model_unit.cfm_euler_partial(x0, prompt, cond, style, S, S, 0.7)
    assert np.array_equal(xs, final)
