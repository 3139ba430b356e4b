"""Pins the oracle's primitives (CPU).

Each check compares the oracle's hand-written loop with something that does
not share its code: numpy/torch library routines in float64, published
known-answer values, or exhaustive enumeration.  A dropped term, a swapped
operand, a wrong sign or index in the oracle fails at least one of these.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F


def test_half_to_float_exhaustive(orc):
    """All 65536 f16 bit patterns (normals, subnormals, zeros, inf, NaN) against
    numpy's IEEE binary16 -> binary32 conversion (tokenizer_tests.cpp:4284)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.half_to_float(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_splitmix64_known_answers(orc):
    """splitmix64 from state 0: the published reference sequence
    (Vigna's splitmix64.c), the generator of tokenizer_tests.cpp:2102."""
    import ctypes

    state = ctypes.c_uint64(0)
    got = [orc.lib().orc_splitmix64_next(ctypes.byref(state)) for _ in range(5)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F,
                   0xF88BB8A8724C81EC, 0x1B39896A51A8749B]


def test_uniform_open01_from_top53_bits(orc):
    """u = (bits >> 11 + 0.5) / 2^53 computed exactly with Python integers from
    the known-answer splitmix64 outputs (tokenizer_tests.cpp:2109)."""
    import ctypes
    from fractions import Fraction

    s = ctypes.c_uint64(0)
    got = [orc.lib().orc_uniform_open01(ctypes.byref(s)) for _ in range(3)]
    raw = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    for g, r in zip(got, raw):
        exact = (Fraction(r >> 11) + Fraction(1, 2)) / Fraction(2 ** 53)
        assert np.float32(g) == np.float32(float(exact))


def test_normal_noise_distribution_and_pairs(orc):
    """Box-Muller output: N(0,1) moments and normality over 2^20 draws, and the
    pair structure x^2 + y^2 = -2 ln u1 of each (cos, sin) pair."""
    from scipy import stats

    z = orc.normal_noise(1 << 20, 1, 20240605)[:, 0].astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3
    assert stats.kstest(z, "norm").pvalue > 1e-3
    t = orc.normal_noise(1000, 1, 5, 3.0)[:, 0]
    assert abs(t.std() / 3.0 - 1) < 0.1  # temperature scales the draws
    import ctypes

    s = ctypes.c_uint64(77)
    u1 = orc.lib().orc_uniform_open01(ctypes.byref(s))
    pair = orc.normal_noise(1, 2, 77)[0].astype(np.float64)
    assert abs((pair ** 2).sum() - (-2 * np.log(np.float64(np.float32(u1))))) < 1e-4


def test_product_generator_matches_oracle(orc, mit2):
    for seed, shape, temp in [(1, (7, 80), 1.0), (20240605, (33, 512), 0.02), (9, (1, 1), 2.0)]:
        a = orc.normal_noise(*shape, seed, temp)
        b = mit2.normal_noise(*shape, seed, temp)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_linear_against_float64(orc):
    rng = np.random.default_rng(0)
    for rows, cols, n in [(7, 13, 1), (512, 864, 3), (1536, 512, 2), (80, 512, 5)]:
        w = rng.standard_normal((rows, cols)).astype(np.float32)
        b = rng.standard_normal(rows).astype(np.float32)
        x = rng.standard_normal((n, cols)).astype(np.float32)
        got = orc.linear(w, b, x)
        ref = x.astype(np.float64) @ w.astype(np.float64).T + b
        assert np.abs(got - ref).max() <= 1e-5 * np.sqrt(cols) * np.abs(ref).max()


def test_linear_thread_count_invariant(orc):
    """Row-parallel threads must not change any bit (the accumulation order of
    each output element is fixed)."""
    rng = np.random.default_rng(1)
    w = rng.standard_normal((512, 512)).astype(np.float32)
    b = rng.standard_normal(512).astype(np.float32)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    orc.set_threads(1)
    a = orc.linear(w, b, x)
    orc.set_threads(8)
    c = orc.linear(w, b, x)
    orc.set_threads(orc.default_threads())
    assert np.array_equal(a, c)


def test_rmsnorm_and_layernorm_against_torch(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 512)).astype(np.float32) * 3
    g = rng.standard_normal(512).astype(np.float32)
    bt = rng.standard_normal(512).astype(np.float32)
    ref = F.rms_norm(torch.from_numpy(x).double(), (512,), torch.from_numpy(g).double(), eps=1e-5).numpy()
    assert np.abs(orc.rmsnorm(x, g, 1e-5) - ref).max() < 1e-5
    ref = F.layer_norm(torch.from_numpy(x).double(), (512,), torch.from_numpy(g).double(),
                       torch.from_numpy(bt).double(), eps=1e-6).numpy()
    assert np.abs(orc.layernorm(x, g, bt, 1e-6) - ref).max() < 1e-5


@pytest.mark.parametrize("kernel", [1, 3, 5])
def test_conv1d_same_against_torch(orc, kernel):
    rng = np.random.default_rng(kernel)
    T, cin, cout = 9, 24, 16
    x = rng.standard_normal((T, cin)).astype(np.float32)
    w = rng.standard_normal((cout, cin, kernel)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    ref = F.conv1d(torch.from_numpy(x).double().T[None], torch.from_numpy(w).double(),
                   torch.from_numpy(b).double(), padding=kernel // 2)[0].T.numpy()
    assert np.abs(orc.conv1d_same(x, w, b, kernel) - ref).max() < 1e-4


@pytest.mark.parametrize("T", [2, 3, 6, 17])
def test_conv1d_reflect_same_against_torch(orc, T):
    rng = np.random.default_rng(T)
    cin, cout = 32, 24
    x = rng.standard_normal((T, cin)).astype(np.float32)
    w = rng.standard_normal((cout, cin, 5)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    xp = torch.from_numpy(x).double().T[None]
    if T > 2:
        xp = F.pad(xp, (2, 2), mode="reflect")
    else:  # torch requires pad < T; numpy's reflect repeats the mirror like the reference
        xp = torch.from_numpy(np.pad(x.astype(np.float64), ((2, 2), (0, 0)), mode="reflect")).T[None]
    ref = F.conv1d(xp, torch.from_numpy(w).double(), torch.from_numpy(b).double())[0].T.numpy()
    assert np.abs(orc.conv1d_reflect_same(x, w, b, 5) - ref).max() < 1e-4


@pytest.mark.parametrize("T", [2, 3, 5, 8])
def test_reflect_pad_against_numpy(orc, T):
    x = np.arange(T * 3, dtype=np.float32).reshape(T, 3)
    assert np.array_equal(orc.reflect_pad(x, 2, 2), np.pad(x, ((2, 2), (0, 0)), mode="reflect"))


def test_timestep_embedding_closed_form(orc):
    """[cos(1000 t f_i) | sin(1000 t f_i)] with cos first (tokenizer_tests.cpp:3947)."""
    freqs = np.exp(-np.log(10000.0) * np.arange(128) / 128).astype(np.float32)
    t = np.array([0.0, 0.125, 0.37, 1.0], np.float32)
    got = orc.timestep_embedding(t, freqs)
    arg = 1000.0 * t.astype(np.float64)[:, None] * freqs.astype(np.float64)[None]
    ref = np.concatenate([np.cos(arg), np.sin(arg)], axis=1)
    assert np.abs(got - ref).max() < 5e-4  # fp32 argument rounding at |arg| <= 1000
    assert np.array_equal(got[0], np.r_[np.ones(128), np.zeros(128)].astype(np.float32))


def test_attention_against_sdpa(orc):
    rng = np.random.default_rng(4)
    T, d = 11, 64
    q, k, v = (rng.standard_normal((T, d)).astype(np.float32) for _ in range(3))
    mask = (rng.random(T) > 0.3).astype(np.uint32)
    mask[0] = 1
    got = orc.attention_head(q, k, v, mask)
    t = lambda a: torch.from_numpy(a).double()[None]
    ref = F.scaled_dot_product_attention(t(q), t(k), t(v), attn_mask=torch.from_numpy(mask != 0)[None, None])[0].numpy()
    assert np.abs(got - ref).max() < 1e-5
    # keys that are masked never matter
    k2, v2 = k.copy(), v.copy()
    k2[mask == 0] = 1e3
    v2[mask == 0] = -7.0
    assert np.array_equal(orc.attention_head(q, k2, v2, mask), got)


def test_attention_fully_masked_row_is_nan_like_reference_cpu(orc):
    """cpu_attention_single_head_masked divides 0 by a zero denominator when no
    key is valid; the oracle keeps that (the GPU path returns 0 like the
    reference's Metal kernel, kernels.metal:2804-2806)."""
    q = np.ones((3, 64), np.float32)
    out = orc.attention_head(q, q, q, np.zeros(3, np.uint32))
    assert np.isnan(out).all()


def test_rope_against_complex_rotation(orc):
    rng = np.random.default_rng(5)
    T, H, D = 7, 8, 64
    x = rng.standard_normal((T, H * D)).astype(np.float32)
    got = orc.rope(x, H, D)
    xc = x.astype(np.float64).reshape(T, H, D // 2, 2)
    z = xc[..., 0] + 1j * xc[..., 1]
    theta = np.arange(T)[:, None] / 10000.0 ** (2 * np.arange(D // 2) / D)
    r = z * np.exp(1j * theta)[:, None, :]
    ref = np.stack([r.real, r.imag], -1).reshape(T, H * D)
    assert np.abs(got - ref).max() < 1e-5


def test_weight_norm_against_torch(orc):
    rng = np.random.default_rng(6)
    v = rng.standard_normal((16, 24, 5)).astype(np.float32)
    g = rng.standard_normal((16, 1, 1)).astype(np.float32)
    ref = torch._weight_norm(torch.from_numpy(v).double(), torch.from_numpy(g).double(), 0).numpy()
    assert np.abs(orc.weight_norm(g.reshape(-1), v.reshape(16, -1)) - ref.reshape(16, -1)).max() < 1e-6
