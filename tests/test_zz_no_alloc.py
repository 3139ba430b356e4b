"""GPU check of mit2cfm_condition_device_noalloc, the allocation-free form of
mit2cfm_condition_device (no reference counterpart; for callers that cannot
allocate): called through the C ABI on device buffers, its condition must
equal the allocating entry point's bit for bit (the same kernels on the same
inputs, scratch from the library's static per-GPU array instead of the
context's workspace), on two calls in a row with the second smaller, in both
precision modes; a size past the scratch limit is an argument error.  The
first call on a fresh context leaves the GPU's free memory unchanged, and the
call captured into a HIP graph on the context's stream replays to the same
bits."""
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


def _inputs(mit2, codes, P, seed):
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    gen = mit2.generated_frames(codes)
    s_infer = torch.from_numpy(mit2.normal_noise(codes, 1024, seed)).to(dev)
    prompt = torch.from_numpy(mit2.normal_noise(P, 512, seed + 1)).to(dev)
    return gen, s_infer, prompt


def _call(mit2, ctx, name, s_infer, codes, prompt, P, out, flags):
    g = ctypes.c_uint32(0)
    fn = getattr(mit2.lib(), name)
    st = fn(ctx._h, s_infer.data_ptr(), codes, prompt.data_ptr(), P, out.data_ptr(),
            ctypes.cast(ctypes.byref(g), ctypes.POINTER(ctypes.c_uint32)), flags)
    assert st == mit2.OK, mit2.lib().mit2cfm_last_error(ctx._h)
    return g.value


def test_noalloc_first_call_on_a_fresh_context_allocates_nothing(mit2, tensors, ctx_na):
    """A context that has never run the condition producer calls the no-alloc
    entry point first: the GPU's free memory is the same before and after (the
    kernels' code was loaded by the module context's calls), and the condition
    equals the allocating entry point's on the module context, bit for bit."""
    torch = pytest.importorskip("torch")
    codes, P = 350, 258
    gen, s_infer, prompt = _inputs(mit2, codes, P, 61)
    ref = torch.full((P + gen, 512), float("nan"), dtype=torch.float32, device=s_infer.device)
    got = torch.full_like(ref, float("nan"))
    torch.cuda.synchronize()
    _call(mit2, ctx_na, "mit2cfm_condition_device", s_infer, codes, prompt, P, ref, mit2.FLAG_SYNC)
    fresh = mit2.Context({**tensors, **mit2.synthetic_lr_tensors(20240606, 0.02)}, device=0)
    try:
        fresh.synchronize()
        torch.cuda.synchronize()
        free_before, _ = torch.cuda.mem_get_info()
        print(f"no-alloc fresh context: codes={codes} P={P}, free before {free_before}", flush=True)
        assert _call(mit2, fresh, "mit2cfm_condition_device_noalloc", s_infer, codes, prompt, P, got,
                     mit2.FLAG_SYNC) == gen
        torch.cuda.synchronize()
        free_after, _ = torch.cuda.mem_get_info()
        assert free_after == free_before, f"free memory moved by {free_before - free_after} bytes"
        assert torch.equal(got, ref)
    finally:
        fresh.close()


def test_noalloc_call_captured_into_a_graph_replays_the_same_bits(mit2, ctx_na):
    """The no-alloc call captured on the context's stream into a HIP graph
    (without FLAG_SYNC): three replays, with the allocating entry point run
    eagerly between them on other inputs, each give the allocating entry
    point's condition bit for bit."""
    torch = pytest.importorskip("torch")
    hip = ctypes.CDLL("libamdhip64.so.7")
    codes, P = 200, 100
    gen, s_infer, prompt = _inputs(mit2, codes, P, 71)
    _, s_other, p_other = _inputs(mit2, 300, 50, 81)
    ref = torch.full((P + gen, 512), float("nan"), dtype=torch.float32, device=s_infer.device)
    got = torch.full_like(ref, float("nan"))
    other = torch.full((50 + mit2.generated_frames(300), 512), float("nan"), dtype=torch.float32,
                       device=s_infer.device)
    torch.cuda.synchronize()
    _call(mit2, ctx_na, "mit2cfm_condition_device", s_infer, codes, prompt, P, ref, mit2.FLAG_SYNC)
    stream = ctypes.c_void_p(ctx_na.stream)
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    print(f"no-alloc graph capture: codes={codes} P={P}", flush=True)
    assert hip.hipStreamBeginCapture(stream, 1) == 0  # hipStreamCaptureModeThreadLocal
    try:
        _call(mit2, ctx_na, "mit2cfm_condition_device_noalloc", s_infer, codes, prompt, P, got, 0)
    finally:
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
    try:
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        for rep in range(3):
            got.fill_(float("nan"))
            torch.cuda.synchronize()
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            assert torch.equal(got, ref), f"replay {rep}"
            _call(mit2, ctx_na, "mit2cfm_condition_device", s_other, 300, p_other, 50, other, mit2.FLAG_SYNC)
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
