"""The oracle's BigVGAN vocoder (the consumer of the decoded mel) against torch
library operations in float64.

The oracle restates the reference's CPU primitives (tokenizer_tests.cpp:3739-3834)
with their index arithmetic; here each is pinned by torch's own operator
(F.conv1d with dilation, F.conv_transpose1d) or, for the anti-aliased SnakeBeta
activation, by the published alias-free algorithm written with torch operators
(replicate pad, depthwise transposed conv by 2, crop, snake, replicate pad,
depthwise strided conv).  The checks are chosen so a plausible mistake (a
transposed weight layout, an off-by-one crop or pad, the wrong snake term)
fails them.  The full vocoder is pinned by an independent torch composition.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle


def _t(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def _rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


@pytest.mark.parametrize("tokens,cin,cout,kernel,dilation", [(9, 8, 16, 3, 1), (20, 16, 8, 7, 3),
                                                              (33, 24, 24, 11, 5), (4, 8, 8, 11, 5),
                                                              (1, 8, 8, 3, 1)])
def test_conv1d_dilated_matches_torch(tokens, cin, cout, kernel, dilation):
    x, w, b = _rand((tokens, cin), 1), _rand((cout, cin, kernel), 2, 0.2), _rand((cout,), 3)
    got = oracle.conv1d_dilated_same(x, w, b, kernel, dilation)
    ref = F.conv1d(_t(x).T[None], _t(w), _t(b), padding=(kernel - 1) * dilation // 2,
                   dilation=dilation)[0].T.numpy()
    assert got.shape == (tokens, cout)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # dilation 1 is the plain zero-padded conv the oracle already has
    if dilation == 1:
        np.testing.assert_array_equal(got, oracle.conv1d_same(x, w, b, kernel))


@pytest.mark.parametrize("tokens,cin,cout,kernel,stride,padding", [(5, 16, 8, 8, 4, 2), (7, 8, 16, 4, 2, 1),
                                                                    (1, 8, 8, 8, 4, 2), (3, 24, 8, 4, 2, 1)])
def test_conv_transpose1d_matches_torch(tokens, cin, cout, kernel, stride, padding):
    x, w, b = _rand((tokens, cin), 4), _rand((cin, cout, kernel), 5, 0.2), _rand((cout,), 6)
    got = oracle.conv_transpose1d(x, w, b, kernel, stride, padding)
    ref = F.conv_transpose1d(_t(x).T[None], _t(w), _t(b), stride=stride, padding=padding)[0].T.numpy()
    assert got.shape == (tokens * stride, cout)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def _torch_alias_free_snake(x, filt_up, filt_down, alpha_log, beta_log):
    """Upstream alias-free activation (ratio 2, 12 taps) with SnakeBeta, float64."""
    c = x.shape[1]
    x = _t(x).T[None]
    fu = _t(filt_up).reshape(1, 1, 12).expand(c, 1, 12)
    fd = _t(filt_down).reshape(1, 1, 12).expand(c, 1, 12)
    y = F.pad(x, (5, 5), mode="replicate")
    y = 2.0 * F.conv_transpose1d(y, fu, stride=2, groups=c)
    y = y[..., 15:-15]
    a = torch.exp(_t(alpha_log))[None, :, None]
    b = torch.exp(_t(beta_log))[None, :, None]
    y = y + 1.0 / (b + 1e-9) * torch.sin(y * a) ** 2
    y = F.pad(y, (5, 6), mode="replicate")
    return F.conv1d(y, fd, stride=2, groups=c)[0].T.numpy()


@pytest.mark.parametrize("tokens,channels", [(1, 4), (2, 8), (17, 24), (64, 8)])
def test_bigvgan_activation_matches_alias_free_torch(mit2, tokens, channels):
    filt = mit2.kaiser_sinc_filter()
    x = _rand((tokens, channels), 7)
    al, bl = _rand((channels,), 8, 0.3), _rand((channels,), 9, 0.3)
    got = oracle.bigvgan_activation(x, filt, filt, al, bl)
    ref = _torch_alias_free_snake(x, filt, filt, al, bl)
    assert got.shape == (tokens, channels)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)
    # an asymmetric pair of filters catches swapped up/down roles
    fu = filt * np.linspace(0.5, 1.5, 12, dtype=np.float32)
    got2 = oracle.bigvgan_activation(x, fu, filt, al, bl)
    np.testing.assert_allclose(got2, _torch_alias_free_snake(x, fu, filt, al, bl), rtol=2e-5, atol=2e-5)
    if tokens > 2:  # (a constant, replicate-padded signal hides the order of the filters)
        assert np.abs(got2 - _torch_alias_free_snake(x, filt, fu, al, bl)).max() > 1e-3


def test_kaiser_sinc_filter_is_a_half_band_lowpass(mit2):
    f = mit2.kaiser_sinc_filter().astype(np.float64)
    assert f.shape == (12,)
    np.testing.assert_allclose(f, f[::-1], atol=1e-7)  # linear phase
    assert abs(f.sum() - 1.0) < 1e-6  # unit DC gain
    w = np.exp(-1j * np.pi * np.arange(12))
    assert abs((f * w).sum()) < 0.05  # Nyquist rejected
    # cutoff at a quarter of the sampling rate: gain at 0.25 cycles/sample near -6 dB
    h = abs((f * np.exp(-2j * np.pi * 0.25 * np.arange(12))).sum())
    assert 0.35 < h < 0.65


def test_library_filter_matches_numpy_kaiser(mit2, bv_tensors):
    """The library's synthetic filter (C++, std::cyl_bessel_i) equals numpy's
    np.kaiser-based restatement, and the synthetic sets are well formed."""
    lib_f = bv_tensors["bigvgan.resblocks.0.activations.0.upsample.filter"].reshape(-1)
    np.testing.assert_allclose(lib_f, mit2.kaiser_sinc_filter(), rtol=0, atol=2e-8)
    assert len(mit2.synthetic_set_specs(mit2.SYNTH_ESTIMATOR)) == len(mit2.synthetic_tensor_specs())
    assert len(mit2.synthetic_set_specs(mit2.SYNTH_LENGTH_REGULATOR)) == 20


def _torch_vocoder(T, mel):
    """Upstream BigVGAN forward in float64 from torch operators: conv_pre, then per
    stage a transposed-conv upsampler and the mean of three AMP resblocks, then the
    final activation, conv_post without bias and the clamp."""
    def wn(prefix):
        return torch._weight_norm(_t(T[prefix + ".weight_v"]), _t(T[prefix + ".weight_g"]), 0)

    def act(prefix, x):  # x [1, C, L]
        y = _torch_alias_free_snake(x[0].T.numpy(), T[prefix + ".upsample.filter"].reshape(-1),
                                    T[prefix + ".downsample.lowpass.filter"].reshape(-1),
                                    T[prefix + ".act.alpha"], T[prefix + ".act.beta"])
        return _t(y).T[None]

    x = F.conv1d(_t(mel).T[None], wn("bigvgan.conv_pre"), _t(T["bigvgan.conv_pre.bias"]), padding=3)
    for i, (prefix, _, _, k, s, p) in enumerate(oracle.BIGVGAN_UPSAMPLERS):
        x = F.conv_transpose1d(x, wn(prefix), _t(T[prefix + ".bias"]), stride=s, padding=p)
        acc = torch.zeros_like(x)
        for rb, _, k in oracle.BIGVGAN_RESBLOCKS[3 * i:3 * i + 3]:
            h = x
            for j, d in enumerate((1, 3, 5)):
                xt = act(f"{rb}.activations.{2 * j}", h)
                xt = F.conv1d(xt, wn(f"{rb}.convs1.{j}"), _t(T[f"{rb}.convs1.{j}.bias"]),
                              padding=(k - 1) * d // 2, dilation=d)
                xt = act(f"{rb}.activations.{2 * j + 1}", xt)
                xt = F.conv1d(xt, wn(f"{rb}.convs2.{j}"), _t(T[f"{rb}.convs2.{j}.bias"]), padding=(k - 1) // 2)
                h = xt + h
            acc = acc + h / 3.0
        x = acc
    x = act("bigvgan.activation_post", x)
    x = F.conv1d(x, wn("bigvgan.conv_post"), None, padding=3)
    return torch.clamp(x, -1.0, 1.0)[0, 0].numpy()


@pytest.fixture(scope="module")
def bv_tensors(mit2):
    return mit2.synthetic_bigvgan_tensors()


def test_synthetic_bigvgan_tensors(mit2, bv_tensors):
    assert len(bv_tensors) == len(mit2.bigvgan_specs()) == 783
    n = sum(v.size for v in bv_tensors.values())
    assert 112_000_000 < n < 112_500_000
    assert bv_tensors["bigvgan.ups.0.0.weight_v"].shape == (1536, 768, 8)
    assert bv_tensors["bigvgan.resblocks.17.convs2.2.weight_v"].shape == (24, 24, 11)
    assert "bigvgan.conv_post.bias" not in bv_tensors


def test_bigvgan_vocoder_matches_torch(bv_tensors):
    oracle.set_threads(oracle.default_threads())
    mel = (np.random.default_rng(11).standard_normal((2, 80)) * 2.0 - 5.0).astype(np.float32)
    bv = oracle.BigVGAN(bv_tensors)
    got = bv.vocoder(mel)
    ref = _torch_vocoder(bv_tensors, mel)
    assert got.shape == (512,)
    assert np.abs(got).max() < 1.0  # the synthetic weights keep the output inside the clamp
    assert oracle.rel_l2(got, ref) <= 1e-5
    # a group that averages instead over two of its resblocks must differ
    x = bv.upsample(bv.conv_pre(mel), 0)
    two = (bv.resblock("bigvgan.resblocks.0", x, 3) + bv.resblock("bigvgan.resblocks.1", x, 7)) / np.float32(2)
    assert oracle.rel_l2(two, bv.resblock_group(x, 0)) > 1e-2
