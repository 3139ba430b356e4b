"""GPU check of mit2cfm_condition_device_noalloc, the allocation-free form of
mit2cfm_condition_device (no reference counterpart; for callers that cannot
allocate): called through the C ABI on device buffers, its condition must
equal the allocating entry point's bit for bit (the same kernels on the same
inputs, scratch from the library's static per-GPU array instead of the
context's workspace), on two calls in a row with the second smaller, in both
precision modes; a size past the scratch limit is an argument error."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx_na(mit2, tensors):
    c = mit2.Context({**tensors, **mit2.synthetic_lr_tensors(20240606, 0.02)}, device=0)
    yield c
    c.close()


def _pair(mit2, ctx, codes, P, seed):
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    gen = mit2.generated_frames(codes)
    s_infer = torch.from_numpy(mit2.normal_noise(codes, 1024, seed)).to(dev)
    prompt = torch.from_numpy(mit2.normal_noise(P, 512, seed + 1)).to(dev)
    ref = torch.full((P + gen, 512), float("nan"), dtype=torch.float32, device=dev)
    got = torch.full((P + gen, 512), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    g_ref, g_got = ctypes.c_uint32(0), ctypes.c_uint32(0)
    L = mit2.lib()
    print(f"no-alloc condition: codes={codes} P={P}", flush=True)
    st = L.mit2cfm_condition_device(ctx._h, s_infer.data_ptr(), codes, prompt.data_ptr(), P, ref.data_ptr(),
                                    ctypes.cast(ctypes.byref(g_ref), ctypes.POINTER(ctypes.c_uint32)),
                                    mit2.FLAG_SYNC)
    assert st == mit2.OK, L.mit2cfm_last_error(ctx._h)
    st = L.mit2cfm_condition_device_noalloc(ctx._h, s_infer.data_ptr(), codes, prompt.data_ptr(), P,
                                            got.data_ptr(),
                                            ctypes.cast(ctypes.byref(g_got), ctypes.POINTER(ctypes.c_uint32)),
                                            mit2.FLAG_SYNC)
    assert st == mit2.OK, L.mit2cfm_last_error(ctx._h)
    assert g_ref.value == g_got.value == gen
    r, g = ref.cpu().numpy(), got.cpu().numpy()
    assert np.isfinite(g).all()
    assert np.array_equal(g, r)
    return g


@pytest.mark.parametrize("mode", ["f32", "f16"])
def test_noalloc_condition_matches_allocating_entry_point(mit2, ctx_na, mode):
    ctx_na.set_precision("length_regulator", mode)
    try:
        _pair(mit2, ctx_na, 350, 258, 31)   # the bench's condition: 602 generated frames
        _pair(mit2, ctx_na, 40, 20, 41)     # a second, smaller call on the same scratch
        _pair(mit2, ctx_na, mit2.NOALLOC_MAX_CODES, 8, 51)  # the limit itself
    finally:
        ctx_na.set_precision("length_regulator", "f32")


def test_noalloc_condition_rejects_past_the_limit(mit2, ctx_na):
    torch = pytest.importorskip("torch")
    codes = mit2.NOALLOC_MAX_CODES + 1
    dev = torch.device("cuda:0")
    s_infer = torch.zeros((codes, 1024), dtype=torch.float32, device=dev)
    prompt = torch.zeros((4, 512), dtype=torch.float32, device=dev)
    out = torch.zeros((4 + mit2.generated_frames(codes), 512), dtype=torch.float32, device=dev)
    with pytest.raises(mit2.Mit2CfmError) as e:
        ctx_na.condition_device_noalloc(s_infer.data_ptr(), codes, prompt.data_ptr(), 4, out.data_ptr(), sync=True)
    assert e.value.status == mit2.E_ARG
    assert "MIT2CFM_NOALLOC_MAX_CODES" in str(e.value)
