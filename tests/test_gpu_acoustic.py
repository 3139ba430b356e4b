"""GPU check of the whole acoustic stage entry (mit2cfm_acoustic_device): the
condition producer, the seeded noise, the CFG decode and the vocoder chained on
the device (synthesis_pipeline.cpp:1012-1035, :1333, :1038-1097) give, bit for
bit, what the four entry points give when called one after another -- each of
which is checked against the oracle in its own test file."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx_all(mit2, tensors):
    c = mit2.Context({**tensors, **mit2.synthetic_lr_tensors(), **mit2.synthetic_bigvgan_tensors()}, device=0)
    yield c
    c.close()


@pytest.mark.parametrize("codes,P,steps,cfg", [(20, 6, 2, 0.7), (37, 16, 3, 0.0)])
def test_acoustic_stage_equals_its_parts(mit2, ctx_all, codes, P, steps, cfg):
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    gen = mit2.generated_frames(codes)
    T = P + gen
    seed = 1234 + codes
    s_infer = torch.from_numpy(mit2.normal_noise(codes, 1024, 31)).to(dev)
    prompt_cond = torch.from_numpy(mit2.normal_noise(P + 5, 512, 32)).to(dev)  # the voice holds >= P rows
    prompt_mel = torch.from_numpy(mit2.normal_noise(P, 80, 33, 2.0) - 5.0).to(dev)
    style = torch.from_numpy(mit2.normal_noise(1, 192, 34)[0]).to(dev)
    wav = torch.empty(256 * gen, dtype=torch.float32, device=dev)
    mel = torch.empty((T, 80), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    print(f"acoustic codes={codes} P={P} steps={steps} cfg={cfg}", flush=True)
    g = ctx_all.acoustic_device(s_infer.data_ptr(), codes, prompt_cond.data_ptr(), prompt_mel.data_ptr(), P,
                                style.data_ptr(), seed, 1.0, steps, cfg, wav.data_ptr(), mel.data_ptr(), sync=True)
    assert g == gen
    # the same chain from the separate entry points
    cond = torch.empty((T, 512), dtype=torch.float32, device=dev)
    x0 = torch.empty((T, 80), dtype=torch.float32, device=dev)
    mel2 = torch.empty((T, 80), dtype=torch.float32, device=dev)
    wav2 = torch.empty(256 * gen, dtype=torch.float32, device=dev)
    assert ctx_all.condition_device(s_infer.data_ptr(), codes, prompt_cond.data_ptr(), P, cond.data_ptr()) == gen
    ctx_all.noise_device(T, 80, seed, 1.0, x0.data_ptr())
    ctx_all.decode_device(x0.data_ptr(), prompt_mel.data_ptr(), cond.data_ptr(), style.data_ptr(), T, P, steps, cfg,
                          mel2.data_ptr(), sync=True)
    ctx_all.bigvgan_device(mel2[P:].contiguous().data_ptr(), gen, wav2.data_ptr(), sync=True)
    torch.cuda.synchronize()
    m, m2 = mel.cpu().numpy(), mel2.cpu().numpy()
    assert np.array_equal(m, m2)
    assert np.all(m[:P] == 0.0)
    w = wav.cpu().numpy()
    assert np.array_equal(w, wav2.cpu().numpy())
    assert np.isfinite(w).all() and np.abs(w).max() <= 1.0


def test_acoustic_stage_needs_all_weights(mit2, tensors):
    torch = pytest.importorskip("torch")
    c = mit2.Context(tensors, device=0)  # estimator only
    try:
        buf = torch.zeros(1 << 16, dtype=torch.float32, device="cuda:0")
        p = buf.data_ptr()
        with pytest.raises(mit2.Mit2CfmError) as e:
            c.acoustic_device(p, 4, p, p, 2, p, 1, 1.0, 2, 0.7, p)
        assert e.value.status == mit2.E_MODEL
    finally:
        c.close()
