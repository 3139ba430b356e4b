"""Device weight image (mit2cfm_write_image / mit2cfm_create_from_image): a
context created from the image of another computes, bit for bit, what the
original computes -- decode, condition producer and vocoder -- and malformed
images are refused before anything reaches the device."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx_src(mit2):
    c = mit2.Context(synthetic_seed=20240605, stddev=0.02, acoustic=True, device=0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def image(ctx_src, tmp_path_factory):
    p = tmp_path_factory.mktemp("img") / "model.mit2hip"
    ctx_src.write_image(p)
    return p


def test_image_context_matches_source(mit2, ctx_src, image):
    c = mit2.Context(image=image, device=0)
    try:
        T, P = 40, 12
        x0 = mit2.normal_noise(T, 80, 1)
        prompt = mit2.normal_noise(P, 80, 2, 2.0) - 5.0
        cond = mit2.normal_noise(T, 512, 3)
        style = mit2.normal_noise(1, 192, 4)[0]
        a = ctx_src.decode(x0, prompt, cond, style, 3, 0.7)
        b = c.decode(x0, prompt, cond, style, 3, 0.7)
        assert np.array_equal(a, b)
        s = mit2.normal_noise(20, 1024, 5)
        assert np.array_equal(ctx_src.length_regulator(s, 34), c.length_regulator(s, 34))
        mel = mit2.normal_noise(6, 80, 6, 2.0) - 5.0
        assert np.array_equal(ctx_src.bigvgan(mel), c.bigvgan(mel))
    finally:
        c.close()


def test_image_of_decoder_only_context(mit2, tensors, tmp_path):
    src = mit2.Context(tensors, device=0)
    p = tmp_path / "dec.mit2hip"
    try:
        src.write_image(p)
        c = mit2.Context(image=p, device=0)
        try:
            x0 = mit2.normal_noise(9, 80, 7)
            pr = mit2.normal_noise(3, 80, 8)
            cond = mit2.normal_noise(9, 512, 9)
            st = mit2.normal_noise(1, 192, 10)[0]
            assert np.array_equal(src.decode(x0, pr, cond, st, 2, 0.7), c.decode(x0, pr, cond, st, 2, 0.7))
            with pytest.raises(mit2.Mit2CfmError) as e:
                c.bigvgan(np.zeros((2, 80), np.float32))
            assert e.value.status == mit2.E_MODEL
        finally:
            c.close()
    finally:
        src.close()


def test_corrupt_images_are_model_errors(mit2, image, tmp_path):
    data = image.read_bytes()
    cases = {
        "truncated": data[: len(data) // 2],
        "flipped": data[:4096] + bytes([data[4096] ^ 0x40]) + data[4097:],
        "magic": b"XXXXXXXX" + data[8:],
        "empty": b"",
    }
    for name, blob in cases.items():
        p = tmp_path / f"{name}.mit2hip"
        p.write_bytes(blob)
        with pytest.raises(mit2.Mit2CfmError) as e:
            mit2.Context(image=p, device=0)
        assert e.value.status == mit2.E_MODEL, name


def test_image_with_gpt_decoder(mit2, tensors, tmp_path):
    """The GPT decoder's prepared weights travel in the image too (section 2)."""
    gpt = mit2.synthetic_gpt_tensors(layers=2)
    src = mit2.Context({**tensors, **gpt}, device=0)
    p = tmp_path / "gpt.mit2hip"
    try:
        src.write_image(p)
        c = mit2.Context(image=p, device=0)
        try:
            assert c.gpt_layers() == 2
            prefix = (np.random.default_rng(4).standard_normal((20, 1280)) * 0.05).astype(np.float32)
            a = src.gpt_kv_greedy(prefix, 6)
            b = c.gpt_kv_greedy(prefix, 6)
            assert a["predicted"].tolist() == b["predicted"].tolist()
            assert np.array_equal(a["last_logits"], b["last_logits"])
        finally:
            c.close()
    finally:
        src.close()
