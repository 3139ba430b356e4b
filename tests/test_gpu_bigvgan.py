"""GPU parity of the BigVGAN vocoder (the consumer of the decoded mel,
dit_cfm_bigvgan.cpp:3606-4512) through the C ABI, stage by stage and end to
end, against the CPU oracle on identical seeded inputs.

The reference runs the vocoder in fp32 and holds its Metal path to max-abs
1e-3 against its CPU path (run_bigvgan_vocoder_test, :4469-4490, on a
one-frame mel of small amplitude; test_vocoder_reference_input repeats that
case).  In the default fp32 mode every conv runs on split f16 operand pairs
(hi + lo: fp32-level products, fp32 accumulation); the activations, residual
sums, the resblock mean and the clamp are fp32.  The whole waveform is held
to the reference's max-abs 1e-3 on loud mels up to 64 frames (16,384
samples), and each stage to rel-L2 bars two orders tighter than f16 operands
give.  The f16 mode (plain f16 operands) keeps its own, wider bars: measured
rel-L2 about 3e-4 per conv and 1e-3 on a loud waveform.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import sincos_series

pytestmark = pytest.mark.gpu

ACT_TOL = 1e-6       # fp32 activation (the GPU's sin), rel-L2
CONV_TOL = 1e-5      # one split-operand conv, rel-L2
BLOCK_TOL = 2e-5     # a resblock / group: six convs (residual), rel-L2
WAV_TOL = 5e-5       # the whole vocoder, rel-L2 ...
WAV_MAXABS = 1e-3    # ... and max-abs on a waveform in [-1, 1]: the reference's bar (:4489)
F16_CONV_TOL = 1e-3  # f16 mode: one conv, rel-L2
F16_WAV_TOL = 2e-3   # f16 mode: the whole vocoder, rel-L2 ...
F16_WAV_MAXABS = 2.5e-3  # ... and max-abs


@pytest.fixture(scope="module")
def bv_tensors(mit2):
    return mit2.synthetic_bigvgan_tensors()


@pytest.fixture(scope="module")
def ctx_bv(mit2, tensors, bv_tensors):
    c = mit2.Context({**tensors, **bv_tensors}, device=0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def bv(orc, bv_tensors):
    return orc.BigVGAN(bv_tensors)


def _x(tokens, channels, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal((tokens, channels)) * scale).astype(np.float32)


@pytest.mark.parametrize("index,tokens", [(0, 1), (0, 37), (20, 130), (58, 64), (75, 200), (90, 65),
                                          (107, 301), (108, 513)])
def test_activation(orc, ctx_bv, bv, index, tokens):
    j, a = divmod(index, 6)
    prefix = "bigvgan.activation_post" if index == 108 else f"bigvgan.resblocks.{j}.activations.{a}"
    C = 24 if index == 108 else 768 >> (j // 3)
    x = _x(tokens, C, index + tokens, 2.0)
    print(f"activation {index} ({prefix}) T={tokens} C={C}", flush=True)
    got = ctx_bv.bigvgan_stage("activation", index, x)
    ref = bv.activation(prefix, x)
    err = orc.rel_l2(got, ref)
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err <= ACT_TOL


@pytest.mark.parametrize("tokens", [1, 5, 70])
def test_conv_pre(orc, ctx_bv, bv, tokens):
    mel = sincos_series(tokens * 80, 0.017, 0.029, 2.0, 1.0, 71).reshape(tokens, 80) - 5.0
    got = ctx_bv.bigvgan_stage("conv_pre", 0, mel)
    ref = bv.conv_pre(mel)
    err = orc.rel_l2(got, ref)
    print(f"conv_pre T={tokens}: rel-L2 {err:.3e}", flush=True)
    assert err <= CONV_TOL


@pytest.mark.parametrize("index,tokens", [(0, 1), (0, 9), (1, 33), (2, 70), (3, 129), (4, 64), (5, 257)])
def test_upsample(orc, ctx_bv, bv, index, tokens):
    cin = [1536, 768, 384, 192, 96, 48][index]
    x = _x(tokens, cin, 100 + index)
    print(f"upsample {index} T={tokens} Cin={cin}", flush=True)
    got = ctx_bv.bigvgan_stage("upsample", index, x)
    ref = bv.upsample(x, index)
    assert got.shape == ref.shape
    err = orc.rel_l2(got, ref)
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err <= CONV_TOL


@pytest.mark.parametrize("index,tokens", [(0, 12), (2, 40), (4, 64), (8, 100), (10, 257), (14, 300),
                                          (17, 512)])
def test_resblock(orc, ctx_bv, bv, index, tokens):
    C = 768 >> (index // 3)
    k = (3, 7, 11)[index % 3]
    x = _x(tokens, C, 200 + index)
    print(f"resblock {index} T={tokens} C={C} k={k}", flush=True)
    got = ctx_bv.bigvgan_stage("resblock", index, x)
    ref = bv.resblock(f"bigvgan.resblocks.{index}", x, k)
    err = orc.rel_l2(got, ref)
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err <= BLOCK_TOL


# Lengths at which the fp32-level convs take the pipelined and the wider
# tiles (the 860-frame call's stages run at 3,440 / 13,760 / 27,520 / 55,040
# rows): 128 x 128 (768 channels at 2,816 rows; 384 at 6,000), 192 x 128 with
# a 2-stage ring (384 channels at 13,760 rows, k = 3), 64 x 192 (192 channels
# at 8,192 rows) and 128 x 96 (96 channels at 32,768 rows).
@pytest.mark.parametrize("index,tokens", [(0, 2816), (3, 6000), (3, 13760), (6, 8192), (9, 32768)])
def test_resblock_long(orc, ctx_bv, bv, index, tokens):
    C = 768 >> (index // 3)
    k = (3, 7, 11)[index % 3]
    x = _x(tokens, C, 400 + index)
    print(f"resblock {index} T={tokens} C={C} k={k}", flush=True)
    got = ctx_bv.bigvgan_stage("resblock", index, x)
    ref = bv.resblock(f"bigvgan.resblocks.{index}", x, k)
    err = orc.rel_l2(got, ref)
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err <= BLOCK_TOL


@pytest.mark.parametrize("index,tokens", [(0, 16), (3, 128), (5, 600)])
def test_resblock_group(orc, ctx_bv, bv, index, tokens):
    C = 768 >> index
    x = _x(tokens, C, 300 + index)
    print(f"group {index} T={tokens} C={C}", flush=True)
    got = ctx_bv.bigvgan_stage("group", index, x)
    ref = bv.resblock_group(x, index)
    err = orc.rel_l2(got, ref)
    print(f"  rel-L2 {err:.3e}", flush=True)
    assert err <= BLOCK_TOL


@pytest.mark.parametrize("tokens", [1, 256, 1000])
def test_post(orc, ctx_bv, bv, tokens):
    x = sincos_series(tokens * 24, 0.011, 0.021, 3.0, 1.0, 83).reshape(tokens, 24)
    got = ctx_bv.bigvgan_stage("post", 0, x)
    ref = bv.post(x).reshape(-1)
    err = float(np.abs(got - ref).max())
    print(f"post T={tokens}: max-abs {err:.3e}", flush=True)
    assert err <= 1e-5


@pytest.mark.parametrize("tokens,amp", [(1, 2.0), (3, 2.0), (8, 2.0), (64, 2.0), (64, 0.5)])
def test_vocoder_matches_oracle(orc, ctx_bv, bv, tokens, amp):
    """Loud mels (amp 2: log-mel -5 +- 3, the waveform reaches the clamp) and a
    quieter one, up to 64 frames, at the reference's max-abs bar."""
    mel = (sincos_series(tokens * 80, 0.017, 0.029, amp, amp / 2, 71).reshape(tokens, 80) - 5.0).astype(np.float32)
    print(f"vocoder T={tokens} amp={amp}", flush=True)
    got = ctx_bv.bigvgan(mel)
    ref = bv.vocoder(mel)
    assert got.shape == (256 * tokens,)
    err, mx = orc.rel_l2(got, ref), float(np.abs(got - ref).max())
    print(f"  rel-L2 {err:.3e}  max-abs {mx:.3e}  |wav| max {np.abs(ref).max():.3f}", flush=True)
    assert np.isfinite(got).all()
    assert err <= WAV_TOL and mx <= WAV_MAXABS


@pytest.fixture(scope="module")
def ctx_bv_stream(mit2, tensors, bv_tensors):
    """A context whose narrow convs stream every tap's rows (the window form
    off: MIT2CFM_CONV_WINDOW=0 is read when the vocoder is built)."""
    import os
    old = os.environ.get("MIT2CFM_CONV_WINDOW")
    os.environ["MIT2CFM_CONV_WINDOW"] = "0"
    try:
        c = mit2.Context({**tensors, **bv_tensors}, device=0)
    finally:
        if old is None:
            del os.environ["MIT2CFM_CONV_WINDOW"]
        else:
            os.environ["MIT2CFM_CONV_WINDOW"] = old
    yield c
    c.close()


# The narrow convs (192, 96, 48 and 24 channels, the upsamplers into them) read
# their operand from a row block's input window held in LDS; the products are
# the same MFMAs in the same K order as the streamed form's, so every output
# bit must match.  Cases: rows fewer than one tile, ragged last tiles, the
# 128-row tiles of the 96- and 48-channel convs (>= 256 row tiles), every
# kernel size (3, 7, 11) and dilation (1, 3, 5) through the resblocks, and a
# whole call.
@pytest.mark.parametrize("stage,index,tokens", [
    ("resblock", 9, 37), ("resblock", 10, 1000), ("resblock", 11, 32768 + 77),
    ("resblock", 12, 5), ("resblock", 13, 4099), ("resblock", 14, 40000 + 11),
    ("resblock", 15, 63), ("resblock", 16, 12345), ("resblock", 17, 65536 + 3),
    ("resblock", 6, 70), ("resblock", 7, 3001), ("resblock", 8, 27520 + 9),
    ("upsample", 3, 500), ("upsample", 4, 300), ("upsample", 5, 1031)])
def test_conv_window_same_bits(ctx_bv, ctx_bv_stream, stage, index, tokens):
    if stage == "resblock":
        C = 768 >> (index // 3)
    else:
        C = [1536, 768, 384, 192, 96, 48][index]
    x = _x(tokens, C, 500 + index)
    print(f"{stage} {index} T={tokens} C={C}", flush=True)
    got = ctx_bv.bigvgan_stage(stage, index, x)
    ref = ctx_bv_stream.bigvgan_stage(stage, index, x)
    assert got.shape == ref.shape
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_conv_window_same_bits_f16_mode(ctx_bv, ctx_bv_stream):
    """The window form in f16 mode (plain f16 operands): 128 x 96 tiles where
    the streamed form takes 64 x 32, the same bits all the same (one K part,
    so every tiling sums each output in one order)."""
    try:
        for c in (ctx_bv, ctx_bv_stream):
            c.set_precision("vocoder", "f16")
        for index, tokens in ((8, 3001), (10, 40000), (13, 4099), (16, 12345)):
            C = 768 >> (index // 3)
            x = _x(tokens, C, 700 + index)
            print(f"f16 resblock {index} T={tokens} C={C}", flush=True)
            got = ctx_bv.bigvgan_stage("resblock", index, x)
            ref = ctx_bv_stream.bigvgan_stage("resblock", index, x)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        mel = (sincos_series(97 * 80, 0.013, 0.031, 2.0, 1.0, 23).reshape(97, 80) - 5.0).astype(np.float32)
        assert np.array_equal(ctx_bv.bigvgan(mel).view(np.uint32), ctx_bv_stream.bigvgan(mel).view(np.uint32))
    finally:
        for c in (ctx_bv, ctx_bv_stream):
            c.set_precision("vocoder", "f32")


def test_conv_window_same_bits_vocoder(ctx_bv, ctx_bv_stream):
    tokens = 97
    mel = (sincos_series(tokens * 80, 0.013, 0.031, 2.0, 1.0, 19).reshape(tokens, 80) - 5.0).astype(np.float32)
    got = ctx_bv.bigvgan(mel)
    ref = ctx_bv_stream.bigvgan(mel)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.fixture(scope="module")
def ctx_bv16(mit2, tensors, bv_tensors):
    c = mit2.Context({**tensors, **bv_tensors}, device=0)
    c.set_precision("vocoder", "f16")
    yield c
    c.close()


@pytest.mark.parametrize("index,tokens", [(0, 33), (4, 64)])
def test_f16_mode_upsample(orc, ctx_bv16, bv, index, tokens):
    assert ctx_bv16.precision("vocoder") == "f16"
    cin = [1536, 768, 384, 192, 96, 48][index]
    x = _x(tokens, cin, 400 + index)
    err = orc.rel_l2(ctx_bv16.bigvgan_stage("upsample", index, x), bv.upsample(x, index))
    print(f"f16 mode upsample {index} T={tokens}: rel-L2 {err:.3e}", flush=True)
    assert err <= F16_CONV_TOL


@pytest.mark.parametrize("tokens", [3, 8])
def test_f16_mode_vocoder(orc, ctx_bv16, bv, tokens):
    mel = (sincos_series(tokens * 80, 0.017, 0.029, 2.0, 1.0, 71).reshape(tokens, 80) - 5.0).astype(np.float32)
    got = ctx_bv16.bigvgan(mel)
    ref = bv.vocoder(mel)
    err, mx = orc.rel_l2(got, ref), float(np.abs(got - ref).max())
    print(f"f16 mode vocoder T={tokens}: rel-L2 {err:.3e}  max-abs {mx:.3e}", flush=True)
    assert err <= F16_WAV_TOL and mx <= F16_WAV_MAXABS


def test_vocoder_reference_input(orc, ctx_bv, bv):
    """run_bigvgan_vocoder_test's input (dit_cfm_bigvgan.cpp:4469-4490): one mel
    frame, mel[i] = sin(0.017 i) 0.10 + cos(0.029 (i % 71)) 0.025; its bar max-abs 1e-3."""
    mel = sincos_series(80, 0.017, 0.029, 0.10, 0.025, 71).reshape(1, 80)
    got = ctx_bv.bigvgan(mel)
    ref = bv.vocoder(mel)
    mx = float(np.abs(got - ref).max())
    print(f"vocoder (reference input): max-abs {mx:.3e}  rel-L2 {orc.rel_l2(got, ref):.3e}", flush=True)
    assert mx <= 1e-3


def test_vocoder_device_matches_host_and_repeats(mit2, ctx_bv):
    torch = pytest.importorskip("torch")
    tokens = 40
    mel = (np.random.default_rng(5).standard_normal((tokens, 80)) * 2.0 - 5.0).astype(np.float32)
    host = ctx_bv.bigvgan(mel)
    d_mel = torch.from_numpy(mel).to("cuda:0")
    d_wav = torch.empty(256 * tokens, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    ctx_bv.bigvgan_device(d_mel.data_ptr(), tokens, d_wav.data_ptr(), sync=True)
    assert np.array_equal(d_wav.cpu().numpy(), host)
    # a longer call in between (the workspace grows) does not change a later short one
    ctx_bv.bigvgan(np.zeros((200, 80), np.float32) - 4.0)
    assert np.array_equal(ctx_bv.bigvgan(mel), host)


def test_missing_vocoder_is_a_model_error(mit2, tensors):
    c = mit2.Context(tensors, device=0)
    try:
        with pytest.raises(mit2.Mit2CfmError) as e:
            c.bigvgan(np.zeros((2, 80), np.float32))
        assert e.value.status == mit2.E_MODEL
        with pytest.raises(mit2.Mit2CfmError) as e:
            c.set_precision("vocoder", "f16")
        assert e.value.status == mit2.E_MODEL
    finally:
        c.close()
