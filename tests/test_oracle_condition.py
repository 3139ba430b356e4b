"""The oracle's length regulator (the condition producer before the decode)
against torch library operations, in float64.

Each oracle piece restates a reference CPU function (tokenizer_tests.cpp /
gpt.cpp, cited in oracle/cfm_oracle.c); here every one is pinned by an
independent library implementation of the same operator, and the checks are
chosen so a plausible mistake (layer norm per token instead of one group,
rounding the interpolation index, a dropped Mish term) fails them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle


def _t(a):
    return torch.from_numpy(np.asarray(a, np.float64))


@pytest.mark.parametrize("in_tokens,out_tokens", [(7, 12), (500, 860), (12, 7), (5, 5), (1, 9), (3, 1)])
def test_nearest_interpolate_matches_torch(in_tokens, out_tokens):
    rng = np.random.default_rng(in_tokens * 1000 + out_tokens)
    x = rng.standard_normal((in_tokens, 6)).astype(np.float32)
    got = oracle.nearest_interpolate(x, out_tokens)
    # float32 tensors: torch then forms the source index in float, as the reference does
    ref = F.interpolate(torch.from_numpy(x).T[None], size=out_tokens, mode="nearest")[0].T.numpy()
    assert np.array_equal(got, ref)


def test_nearest_interpolate_is_floor_not_round():
    # out_t = 1 of 3 -> 2 frames: floor(1 * 2/3) = 0, round would give 1
    x = np.array([[1.0], [2.0]], np.float32)
    assert oracle.nearest_interpolate(x, 3)[:, 0].tolist() == [1.0, 1.0, 2.0]


@pytest.mark.parametrize("tokens", [1, 9, 130])
def test_groupnorm1_matches_torch(tokens):
    rng = np.random.default_rng(tokens)
    x = (rng.standard_normal((tokens, 512)) * 3 + 0.7).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    got = oracle.groupnorm1(x, g, b)
    ref = F.group_norm(_t(x).T[None], 1, _t(g), _t(b), eps=1e-5)[0].T.numpy()
    assert np.abs(got - ref).max() <= 5e-5 * np.abs(ref).max()
    if tokens > 1:  # one group over the whole sequence, not a layer norm per token
        per_token = F.layer_norm(_t(x), (512,), _t(g), _t(b), eps=1e-5).numpy()
        assert np.abs(per_token - ref).max() > 1e-2


def test_mish_matches_torch():
    x = np.linspace(-30, 30, 20001, dtype=np.float32)
    got = oracle.mish(x)
    ref = F.mish(_t(x)).numpy()
    assert np.abs(got - ref).max() <= 2e-6 * max(1.0, np.abs(ref).max())
    assert np.abs(x * np.tanh(np.exp(x.astype(np.float64))) - ref).max() > 1e-2  # log1p matters


def _torch_length_regulator(t, s_infer, out_tokens):
    p = oracle.LR_PREFIX
    w = {k[len(p):]: _t(np.asarray(v, np.float32)) for k, v in t.items() if k.startswith(p)}
    x = F.linear(_t(s_infer), w["content_in_proj.weight"], w["content_in_proj.bias"])
    # source rows of the nearest interpolation, formed in float as the reference does
    src = F.interpolate(torch.arange(x.shape[0], dtype=torch.float32)[None, None], size=out_tokens,
                        mode="nearest")[0, 0].long()
    x = x[src].T[None]
    for ci, ni in ((0, 1), (3, 4), (6, 7), (9, 10)):
        x = F.conv1d(x, w[f"model.{ci}.weight"], w[f"model.{ci}.bias"], padding=1)
        x = F.group_norm(x, 1, w[f"model.{ni}.weight"], w[f"model.{ni}.bias"], eps=1e-5)
        x = F.mish(x)
    x = F.conv1d(x, w["model.12.weight"], w["model.12.bias"])
    return x[0].T.numpy()


@pytest.mark.parametrize("in_tokens,out_tokens,std", [(11, 18, 0.02), (7, 12, 0.05), (20, 34, 0.02)])
def test_length_regulator_matches_torch(mit2, in_tokens, out_tokens, std):
    t = mit2.synthetic_lr_tensors(100 + in_tokens, std)
    s_infer = mit2.normal_noise(in_tokens, 1024, 5 + in_tokens)
    got = oracle.length_regulator(t, s_infer, out_tokens)
    ref = _torch_length_regulator(t, s_infer, out_tokens)
    assert got.shape == (out_tokens, 512)
    assert oracle.rel_l2(got, ref) <= 1e-5
    # the interpolation is not a no-op: dropping it (first out_tokens rows) changes the result
    assert oracle.rel_l2(_torch_length_regulator(t, np.repeat(s_infer, 2, 0)[:in_tokens], out_tokens), ref) > 1e-3


def test_synthetic_lr_tensors_shapes(mit2):
    t = mit2.synthetic_lr_tensors()
    assert len(t) == 20
    assert t[oracle.LR_PREFIX + "model.0.weight"].shape == (512, 512, 3)
    assert abs(float(t[oracle.LR_PREFIX + "model.1.weight"].astype(np.float32).mean()) - 1.0) < 0.01


@pytest.mark.parametrize("tokens", [1, 9, 602])
def test_groupnorm1_f64stats_matches_torch(tokens):
    """The double-statistics variant is torch's float64 group_norm
    up to the final float rounding."""
    rng = np.random.default_rng(50 + tokens)
    x = (rng.standard_normal((tokens, 512)) * 3 + 0.7).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    got = oracle.groupnorm1(x, g, b, f64_stats=True)
    ref = F.group_norm(_t(x).T[None], 1, _t(g), _t(b), eps=1e-5)[0].T.numpy()
    assert np.abs(got - ref).max() <= 2e-6 * np.abs(ref).max()


def test_reference_groupnorm_statistics_drift_with_size():
    """The reference's sequential float sums of the GroupNorm statistics
    (tokenizer_tests.cpp:3874-3896) carry rounding error that grows with the
    element count: about 1e-6 of the output scale at 11 x 512 values, 1e-4 at
    602 x 512.  A GPU reduction in a different order cannot reproduce it; the
    GPU parity tests measure it with the f64-statistics checker and allow for it."""
    rng = np.random.default_rng(9)
    g = np.ones(512, np.float32)
    b = np.zeros(512, np.float32)
    drift = {}
    for tokens in (11, 602):
        x = (rng.standard_normal((tokens, 512)) * 1.3 + 0.2).astype(np.float32)
        ref = F.group_norm(_t(x).T[None], 1, _t(g), _t(b), eps=1e-5)[0].T.numpy()
        drift[tokens] = float(np.abs(oracle.groupnorm1(x, g, b) - ref).max())
        assert np.abs(oracle.groupnorm1(x, g, b, f64_stats=True) - ref).max() <= 2e-6 * np.abs(ref).max()
    assert drift[11] < 2e-5 and drift[602] > 2e-5


@pytest.mark.parametrize("in_tokens,out_tokens", [(7, 11), (20, 34)])
def test_length_regulator_f64stats_matches_torch(mit2, in_tokens, out_tokens):
    t = mit2.synthetic_lr_tensors(300 + in_tokens, 0.02)
    s_infer = mit2.normal_noise(in_tokens, 1024, 9 + in_tokens)
    got = oracle.length_regulator(t, s_infer, out_tokens, f64_stats=True)
    ref = _torch_length_regulator(t, s_infer, out_tokens)
    assert oracle.rel_l2(got, ref) <= 1e-5
