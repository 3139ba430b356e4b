#!/usr/bin/env python3
"""Benchmark: DiT-CFM mel decode on one MI355X.

Workload (one bench "step" = one full decode): T = 860 mel frames (258 prompt
+ 602 generated), 25 Euler steps, CFG rate 0.7 with the cond/null pair
batched as B = 2, hidden 512, 13 AdaRMSNorm blocks (8 heads x 64), 8-layer
WaveNet (k=5, 512 ch); synthetic f16 weights N(0, 0.02) from seed 20240605;
x0, content, style ~ N(0,1), prompt mel ~ N(-5, 2).  Inputs are resident in
HBM before the timed region; the decode runs on the library's stream through
the C ABI (mit2cfm_decode_device) and is timed with host wall clock around
`--steps` decodes, bracketed by device synchronisation.

Prints ONE JSON line.  Extra fields:
  roofline      the dominant kernel's algorithmic TFLOP/s (flops per launch /
                average launch time from HIP events on the library stream)
                against the f16 dense MFMA peak; traffic from committed
                rocprofv3 FETCH_SIZE / WRITE_SIZE runs when present.
  cpu_baseline  the CPU restatement of the reference path on this host:
                one Euler step (cond + null forward) at T = 860, extrapolated
                to the 25-step decode.
  condition_producer
                the step before the decode, on the GPU: the length regulator
                on the semantic codes that make this decode's T - P frames,
                merged with the P prompt rows (mit2cfm_condition_device); time
                per call from HIP events on the library stream, its
                algorithmic TFLOP/s, and the oracle's time for one call on
                the host cores.
  vocoder       the step after the decode, on the GPU: the BigVGAN vocoder on
                this decode's mel (T frames -> 256 T samples,
                mit2cfm_bigvgan_device) with synthetic weights (seed
                20240607); time per call from HIP events on the library
                stream, output samples/s, algorithmic conv TFLOP/s, and the
                oracle on the host cores over a bounded sample (two mel
                frames).
  context_create_s
                creating the context from the host tensors (f16 -> weight
                preparation -> upload) and from a device image of the same
                prepared weights (mit2cfm_create_from_image).
  acoustic_stage
                the whole acoustic stage of one synthesis segment on the GPU
                (mit2cfm_acoustic_device: condition, seeded noise, CFG decode,
                vocoder), at the reference's published steady-state segment:
                553 semantic codes -> 951 generated frames after a 629-frame
                voice prompt (T = 1580), 16 steps, CFG 0.7, 11.0 s of audio;
                time per call from HIP events, its real-time factor, and the
                reference's published time for that segment on its own
                hardware (a different machine and the real weights).
  configs       every other workload of the benchmark set on the same
                context, inputs resident in HBM, median of the timed
                decodes: one estimator forward at T=256 (B=2 CFG pair),
                T=128 with 12 steps (launch-bound), T=3000 with 25 steps
                (O(T^2) attention), and 8 right-padded requests (B=16) with 16
                steps; each with frames/s, CFM steps/s and whole-decode MFMA
                utilisation on valid rows and keys only.
  pcie_inclusive
                the headline decode through the host-pointer entry point
                (upload, decode, readback), median of 10 -- reported beside
                `value`, never as it.
  first_call_ms the first decode of a length the context has not seen:
                graph capture and instantiation included, beside the
                replay time of the same shape.
  gpt_decode    the GPT mel-code decoder (the stage that makes the semantic
                codes) on the GPU: greedy decode of 553 codes after a
                150-row prefix with the 24-layer synthetic model (seed
                20240608); device time of the prefill and the decode loop,
                ms per code, the weight stream it implies, the reference's
                published 5.5 ms per code, its dominant GEMV's bandwidth
                (c_fc, cycling the layers' weights, HIP events) against HBM
                peak, and the oracle's decode step on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "index-tts2-metal_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "DiT-CFM mel frames/sec at 25 steps, B=2 CFG, T=860; MFMA util %"
PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16 MFMA
PEAK_HBM_GBS = 8000.0
# Algorithmic FLOPs per estimator forward: 148,373,504 per valid row + 26,624 * sum_b T_b^2.
FLOPS_PER_ROW = 148_373_504
FLOPS_PER_T2 = 26_624
KERNEL_IDS = {"w13": 0, "conv": 1, "qkv": 2, "w2": 3, "attention": 4, "adarms": 5}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10, help="timed decodes")
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--tokens", type=int, default=860)
    p.add_argument("--prompt", type=int, default=258)
    p.add_argument("--cfm-steps", type=int, default=25)
    p.add_argument("--cfg", type=float, default=0.7)
    p.add_argument("--kernel", default="conv", choices=sorted(KERNEL_IDS),
                   help="kernel reported in `roofline`")
    p.add_argument("--kernel-launches", type=int, default=200)
    p.add_argument("--cpu-threads", type=int, default=0, help="0 = min(16, available cores)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cond-calls", type=int, default=50, help="timed condition-producer calls")
    p.add_argument("--voc-calls", type=int, default=10, help="timed vocoder calls (0 = skip)")
    p.add_argument("--acoustic-calls", type=int, default=5,
                   help="timed acoustic-stage calls (0 = skip; needs the vocoder)")
    p.add_argument("--gpt-codes", type=int, default=553,
                   help="mel codes of the timed GPT greedy decode (0 = skip)")
    p.add_argument("--gpt-prefix", type=int, default=150, help="prefix rows of the GPT decode")
    p.add_argument("--pcie-reps", type=int, default=10, help="host-pointer decodes (median)")
    p.add_argument("--no-configs", dest="configs", action="store_false",
                   help="skip the other workloads of the benchmark set")
    p.add_argument("--no-cpu-1thread", dest="cpu_1thread", action="store_false",
                   help="skip the one-thread CPU baseline")
    p.add_argument("--calib-mib", type=int, default=256,
                   help="size of the counter-calibration copy (0 = skip)")
    return p.parse_args()


def traffic_from_profiles(kernel_name: str, tokens: int):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE),
    committed under profiles/ as JSON; None when not measured."""
    f = ROOT / "profiles" / f"traffic_{kernel_name}_T{tokens}.json"
    if not f.exists():
        return None
    try:
        return float(json.loads(f.read_text())["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def cpu_baseline(tensors, T, P, cfm_steps, cfg, threads):
    import numpy as np
    import mit2cfm
    from oracle import oracle

    oracle.set_threads(threads)
    model = oracle.Model(tensors)
    x0 = mit2cfm.normal_noise(T, 80, 1)
    cond = mit2cfm.normal_noise(T, 512, 2)
    style = mit2cfm.normal_noise(1, 192, 3)[0]
    prompt = mit2cfm.normal_noise(P, 80, 4, 2.0) - 5.0
    x = x0.copy()
    x[:P] = 0
    px = np.zeros((T, 80), np.float32)
    px[:P] = prompt
    mask = np.ones(T, np.uint32)
    t0 = time.perf_counter()
    model.estimator_step(x, px, cond, style, 0.0, mask)
    if cfg > 0:
        model.estimator_step(x, np.zeros_like(px), np.zeros_like(cond), np.zeros_like(style), 0.0, mask)
    step_s = time.perf_counter() - t0
    model.close()
    decode_s = step_s * cfm_steps
    return {
        "value": T / decode_s,
        "unit": "mel frames/s",
        "cores": threads,
        "kind": "port",
        "sample": f"1 of {cfm_steps} Euler steps (cond + null estimator forwards) at T={T}, "
                  f"{step_s:.1f} s measured, decode time extrapolated x{cfm_steps}",
    }


def cpu_baseline_1thread(tensors, T=256, P=96):
    """The reference CPU path is single-threaded (cpu_linear, tokenizer_tests.cpp:3026):
    the oracle on one thread for one estimator forward pair at T=256 (the
    benchmark set's CPU-runnable case), scaled to the T=860 decode by
    algorithmic FLOPs."""
    import numpy as np
    import mit2cfm
    from oracle import oracle

    oracle.set_threads(1)
    model = oracle.Model(tensors)
    x = mit2cfm.normal_noise(T, 80, 1)
    cond = mit2cfm.normal_noise(T, 512, 2)
    style = mit2cfm.normal_noise(1, 192, 3)[0]
    px = np.zeros((T, 80), np.float32)
    px[:P] = mit2cfm.normal_noise(P, 80, 4, 2.0) - 5.0
    mask = np.ones(T, np.uint32)
    t0 = time.perf_counter()
    model.estimator_step(x, px, cond, style, 0.5, mask)
    model.estimator_step(x, np.zeros_like(px), np.zeros_like(cond), np.zeros_like(style), 0.5, mask)
    sec = time.perf_counter() - t0
    model.close()
    f_sample = FLOPS_PER_ROW * 2 * T + FLOPS_PER_T2 * 2 * T * T
    f_decode = 25 * (FLOPS_PER_ROW * 2 * 860 + FLOPS_PER_T2 * 2 * 860 * 860)
    return {"value": round(860 / (sec * f_decode / f_sample), 4), "unit": "mel frames/s", "cores": 1,
            "kind": "port", "gflop_per_s": round(f_sample / sec / 1e9, 2),
            "sample": f"one estimator forward pair (cond + null) at T={T}, {sec:.1f} s on one thread, "
                      "scaled to the 25-step T=860 decode by algorithmic FLOPs"}


def request_lengths(n: int, lo: int, hi: int, seed: int) -> list[int]:
    """Target lengths of the padded-batch workload: uniform in [lo, hi] from one
    seed by splitmix64 modulo (the same draw as the test fixtures)."""
    out, st = [], seed
    for _ in range(n):
        st = (st + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = st
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        out.append(lo + (z ^ (z >> 31)) % (hi - lo + 1))
    return out


def decode_flops(valid_T, steps):
    """Algorithmic FLOPs of a CFG decode: each request is a cond + null branch
    pair; valid rows and keys only."""
    rows = sum(2 * t for t in valid_T)
    keys2 = sum(2 * t * t for t in valid_T)
    return steps * (FLOPS_PER_ROW * rows + FLOPS_PER_T2 * keys2)


def timed_median(fn, sync, reps):
    """Median wall time (ms) of `reps` calls, each bracketed by device synchronisation."""
    ts = []
    for _ in range(reps):
        sync()
        t0 = time.perf_counter()
        fn()
        sync()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    return ts[len(ts) // 2], ts


def configs_section(a, mit2cfm, ctx, torch, dev):
    """The benchmark set's other workloads on resident inputs."""
    import numpy as np

    def sync():
        ctx.synchronize()
        torch.cuda.synchronize()

    out = {}
    singles = [("config1_forward_T256", 256, 96, 1, 20), ("config3_T128_S12", 128, 48, 12, 20),
               ("config4_T3000_S25", 3000, 258, 25, 5)]
    for name, T, P, S, reps in singles:
        x0 = torch.from_numpy(mit2cfm.normal_noise(T, 80, 1)).to(dev)
        cond = torch.from_numpy(mit2cfm.normal_noise(T, 512, 2)).to(dev)
        style = torch.from_numpy(mit2cfm.normal_noise(1, 192, 3)[0]).to(dev)
        prompt = torch.from_numpy(np.ascontiguousarray(mit2cfm.normal_noise(P, 80, 4, 2.0) - 5.0)).to(dev)
        o = torch.empty((T, 80), dtype=torch.float32, device=dev)
        sync()

        def run():
            ctx.decode_device(x0.data_ptr(), prompt.data_ptr(), cond.data_ptr(), style.data_ptr(), T, P, S,
                              a.cfg, o.data_ptr())

        for _ in range(2):
            run()
        med, _ = timed_median(run, sync, reps)
        fl = decode_flops([T], S)
        r = {"tokens": T, "prompt_tokens": P, "cfm_steps": S, "cfg_rate": a.cfg, "branches": 2,
             "ms_per_decode": round(med, 3), "frames_per_s": round(T / (med / 1e3), 1),
             "cfm_steps_per_s": round(S / (med / 1e3), 1),
             "algorithmic_tflop": round(fl / 1e12, 4),
             "decode_mfma_util": round(fl / (med / 1e3) / 1e12 / PEAK_F16_TFLOPS, 4), "timed": reps}
        if S == 1:
            r["note"] = "one CFG Euler step: the estimator forward pair (B=2) plus the fused conv2/CFG/Euler update"
        out[name] = r
    # 8 right-padded requests (B = 16), 16 steps
    P, S, nreq = 258, 16, 8
    toks = [P + L for L in request_lengths(nreq, 300, 1500, 5)]
    tmax = max(toks)
    x0 = np.zeros((nreq, tmax, 80), np.float32)
    pr = np.zeros((nreq, tmax, 80), np.float32)
    co = np.zeros((nreq, tmax, 512), np.float32)
    st = np.zeros((nreq, 192), np.float32)
    for r_, T in enumerate(toks):
        x0[r_, :T] = mit2cfm.normal_noise(T, 80, 100 + 10 * r_)
        co[r_, :T] = mit2cfm.normal_noise(T, 512, 101 + 10 * r_)
        st[r_] = mit2cfm.normal_noise(1, 192, 102 + 10 * r_)[0]
        pr[r_, :P] = mit2cfm.normal_noise(P, 80, 103 + 10 * r_, 2.0) - 5.0
    d = [torch.from_numpy(v).to(dev) for v in (x0, pr, co, st)]
    o = torch.empty((nreq, tmax, 80), dtype=torch.float32, device=dev)
    sync()

    def runb():
        ctx.decode_batched_device(toks, [P] * nreq, d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr(),
                                  d[3].data_ptr(), tmax, S, a.cfg, o.data_ptr())

    fl = decode_flops(toks, S)
    for key, padding in (("config5_8req_padded_B16_S16", "compute"),
                         ("config5_8req_padded_B16_S16_skip_padding", "skip")):
        ctx.set_padding(padding)
        try:
            for _ in range(2):
                runb()
            med, _ = timed_median(runb, sync, 5)
        finally:
            ctx.set_padding("compute")
        out[key] = {
            "requests": nreq, "tokens": toks, "t_max": tmax, "prompt_tokens": P, "cfm_steps": S,
            "cfg_rate": a.cfg, "branches": 2 * nreq, "padding": padding, "ms_per_decode": round(med, 3),
            "frames_per_s": round(sum(toks) / (med / 1e3), 1),
            "padded_frames_per_s": round(nreq * tmax / (med / 1e3), 1),
            "cfm_steps_per_s": round(S / (med / 1e3), 1), "algorithmic_tflop": round(fl / 1e12, 4),
            "decode_mfma_util": round(fl / (med / 1e3) / 1e12 / PEAK_F16_TFLOPS, 4),
            "note": ("frames/s and utilisation count valid frames, rows and keys only (padding is waste)"
                     + ("; padded rows computed (the masked estimator at the padded length)"
                        if padding == "compute" else
                        "; rows from two past each request's valid length not computed "
                        "(MIT2CFM_PADDING_SKIP: valid rows bit-identical, padded rows unspecified)")),
            "timed": 5}
    return out


def cpu_threads(a) -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return a.cpu_threads or max(1, min(16, n))


def condition_codes(generated: int) -> int:
    """Smallest semantic-token count whose floor(codes * 1.72f) is `generated`
    (0 when none is)."""
    import mit2cfm

    for codes in range(max(1, int(generated / 1.72) - 2), int(generated / 1.72) + 3):
        if mit2cfm.generated_frames(codes) == generated:
            return codes
    return 0


def condition_cpu_baseline(lr_tensors, s_infer, gen, threads):
    from oracle import oracle

    oracle.set_threads(threads)
    t0 = time.perf_counter()
    oracle.length_regulator(lr_tensors, s_infer, gen)
    ms = (time.perf_counter() - t0) * 1e3
    return {"value": round(ms, 1), "unit": "ms per call", "cores": threads, "kind": "port",
            "sample": f"one length-regulator call ({s_infer.shape[0]} codes -> {gen} frames)"}


def vocoder_cpu_baseline(bv_tensors, mel, threads):
    from oracle import oracle

    oracle.set_threads(threads)
    bv = oracle.BigVGAN(bv_tensors)
    frames = 2
    t0 = time.perf_counter()
    bv.vocoder(mel[:frames])
    s = time.perf_counter() - t0
    return {"value": round(256 * frames / s, 1), "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"the vocoder on the first {frames} mel frames ({256 * frames} samples)"}


def gpt_cpu_baseline(gpt_tensors, threads):
    """The oracle's cached decode step (24 layers): the time of 5 greedy steps
    minus the time of 1, after the same 8-row prefix, over 4."""
    import numpy as np
    from oracle import oracle

    oracle.set_threads(threads)
    g = oracle.GPT(gpt_tensors)
    prefix = (np.random.default_rng(3).standard_normal((8, 1280)) * 0.05).astype(np.float32)
    t0 = time.perf_counter()
    g.kv_greedy(prefix, 1)
    t1 = time.perf_counter()
    g.kv_greedy(prefix, 5)
    t2 = time.perf_counter()
    per_token = ((t2 - t1) - (t1 - t0)) / 4
    return {"value": round(1.0 / per_token, 2), "unit": "mel codes/s", "cores": threads, "kind": "port",
            "sample": "the oracle's 24-layer cached decode: (time of 5 greedy steps - time of 1) / 4 "
                      "after an 8-row prefix"}


def gpt_section(a, mit2cfm, tensors, torch):
    """GPT mel-code decoder: greedy decode of a.gpt_codes codes after an
    a.gpt_prefix-row prefix (24 layers, synthetic weights), and its dominant
    GEMV's bandwidth."""
    import numpy as np

    gpt_tensors = mit2cfm.synthetic_gpt_tensors()
    ctx = mit2cfm.Context({**tensors, **gpt_tensors}, device=0)
    prefix = (np.random.default_rng(2).standard_normal((a.gpt_prefix, 1280)) * 0.05).astype(np.float32)
    ctx.gpt_kv_greedy(prefix, 16)  # warm-up (captures the step graphs)
    runs = [ctx.gpt_kv_greedy(prefix, a.gpt_codes) for _ in range(2)]
    r = min(runs, key=lambda q: q["decode_ms"])
    # the production setting: IndexTTS2's do_sample (top_p 0.8, top_k 30, temperature 0.8,
    # repetition penalty 10)
    smp = dict(temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0)
    ctx.gpt_kv_sample(prefix, 16, 1, **smp)
    rs = min((ctx.gpt_kv_sample(prefix, a.gpt_codes, 20240605 + i, **smp) for i in range(2)),
             key=lambda q: q["decode_ms"] / max(len(q["predicted"]), 1))
    n = len(r["predicted"])
    ms_tok = r["decode_ms"] / n
    step_bytes = mit2cfm.gpt_step_bytes(24)
    # the dominant GEMV (c_fc, 5120 x 1280, LayerNorm prologue, gelu_new), cycling the 24 layers' weights
    stream = torch.cuda.ExternalStream(ctx.stream, device=torch.device("cuda:0"))
    name, kbytes = ctx.gpt_profile_launch(2, 24)
    ctx.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    launches = 240
    ctx.gpt_profile_launch(2, launches)  # captures the launch loop into a graph
    ctx.synchronize()
    e0.record(stream)
    ctx.gpt_profile_launch(2, launches)  # replays it: back-to-back kernels, no host launch gaps
    e1.record(stream)
    ctx.synchronize()
    torch.cuda.synchronize()
    k_us = e0.elapsed_time(e1) / launches * 1e3
    achieved = kbytes / (k_us / 1e6) / 1e9
    ctx.close()
    out = {"workload": f"GPT-2 24 x 1280 greedy decode: {a.gpt_prefix}-row prefix, {a.gpt_codes} codes "
                       "(synthetic f16 weights seed 20240608)",
           "codes": n, "first_stop_step": r["first_stop_step"],
           "prefill_ms": round(r["prefill_ms"], 3), "decode_ms": round(r["decode_ms"], 3),
           "ms_per_code": round(ms_tok, 4), "codes_per_s": round(1e3 / ms_tok, 1),
           "sampled": {"settings": smp, "codes": len(rs["predicted"]),
                       "ms_per_code": round(rs["decode_ms"] / max(len(rs["predicted"]), 1), 4)},
           "weight_gb_per_code": round(step_bytes / 1e9, 4),
           "weight_stream_gb_s": round(step_bytes / (ms_tok / 1e3) / 1e9, 1),
           "reference_published": {"ms_per_code": 5.5, "hardware": "Apple M3 Ultra (Metal, ICB greedy decode)",
                                   "source": "docs/evolution.md:77"},
           "speedup_vs_published": round(5.5 / ms_tok, 1),
           "roofline": {"bound": "hbm", "kernel": name, "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                        "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                        "avg_launch_us": round(k_us, 2), "algorithmic_bytes": int(kbytes)}}
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = gpt_cpu_baseline(gpt_tensors, cpu_threads(a))
    return out


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: the library runs on one GPU; --gpus {a.gpus} is not supported "
              "(multi-GPU sharding is design-only).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch  # first: the library then shares torch's HIP runtime
    import mit2cfm

    T, P, S, cfg = a.tokens, a.prompt, a.cfm_steps, a.cfg
    dev = torch.device("cuda:0")
    tensors = mit2cfm.synthetic_tensors(20240605, 0.02)
    lr_tensors = mit2cfm.synthetic_lr_tensors(20240606, 0.02)
    bv_tensors = mit2cfm.synthetic_bigvgan_tensors(20240607) if a.voc_calls else {}
    c0 = time.perf_counter()
    ctx = mit2cfm.Context({**tensors, **lr_tensors, **bv_tensors}, device=0)
    create_s = time.perf_counter() - c0
    # Context creation from the device image of the same weights (no host-side
    # weight preparation): written once, then timed.
    import tempfile
    with tempfile.TemporaryDirectory() as td:
        img = os.path.join(td, "model.mit2hip")
        ctx.write_image(img)
        c0 = time.perf_counter()
        mit2cfm.Context(image=img, device=0).close()
        create_img_s = time.perf_counter() - c0
        img_mb = os.path.getsize(img) / 2**20

    x0 = mit2cfm.normal_noise(T, 80, 1)
    cond = mit2cfm.normal_noise(T, 512, 2)
    style = mit2cfm.normal_noise(1, 192, 3)[0]
    prompt = mit2cfm.normal_noise(P, 80, 4, 2.0) - 5.0
    d_x0 = torch.from_numpy(x0).to(dev)
    d_prompt = torch.from_numpy(np.ascontiguousarray(prompt)).to(dev)
    d_cond = torch.from_numpy(cond).to(dev)
    d_style = torch.from_numpy(style).to(dev)
    d_out = torch.empty((T, 80), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def decode():
        ctx.decode_device(d_x0.data_ptr(), d_prompt.data_ptr(), d_cond.data_ptr(), d_style.data_ptr(),
                          T, P, S, cfg, d_out.data_ptr(), sync=False)

    stream = torch.cuda.ExternalStream(ctx.stream, device=dev)
    for _ in range(a.warmup):
        decode()
    ctx.synchronize()
    torch.cuda.synchronize()

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(a.steps):
        decode()
    ev1.record(stream)
    ctx.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_decode = wall * 1e3 / a.steps
    ev_ms = ev0.elapsed_time(ev1) / a.steps
    out = d_out.cpu().numpy()
    if not np.isfinite(out).all():
        raise RuntimeError("decode produced non-finite values")

    flops_decode = S * (FLOPS_PER_ROW * 2 * T + FLOPS_PER_T2 * 2 * T * T)
    frames_per_s = T / (ms_per_decode / 1e3)

    # Dominant kernel: average launch time from events on the library stream.
    kid = KERNEL_IDS[a.kernel]
    name, kflops, kbytes = ctx.profile_launch(kid, 0)
    ctx.profile_launch(kid, 10)  # warm
    ctx.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    ctx.profile_launch(kid, a.kernel_launches)
    e1.record(stream)
    ctx.synchronize()
    torch.cuda.synchronize()
    k_ms = e0.elapsed_time(e1) / a.kernel_launches
    if kflops > 0:
        achieved = kflops / (k_ms / 1e3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_F16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_F16_TFLOPS, 4)}
    else:
        achieved = kbytes / (k_ms / 1e3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4)}
    roof.update({"traffic": traffic_from_profiles(name, T), "kernel": name,
                 "avg_launch_us": round(k_ms * 1e3, 2), "algorithmic_flops": kflops,
                 "algorithmic_bytes": kbytes})

    # Counter calibration: a plain streaming copy of known size (reads and
    # writes calib_mib MiB once each).  Under rocprofv3 --pmc FETCH_SIZE /
    # WRITE_SIZE its readings give the KiB-per-byte factor that turns the
    # dominant kernel's readings into HBM bytes.
    if a.calib_mib > 0:
        n = a.calib_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst

    # Condition producer (the step before the decode): the length regulator on
    # `codes` semantic tokens plus the merge with the prompt rows, sized so the
    # condition is exactly this decode's T frames.
    codes = condition_codes(T - P)
    cp = None
    if codes and a.cond_calls:
        gen = mit2cfm.generated_frames(codes)
        s_infer = mit2cfm.normal_noise(codes, 1024, 6)
        d_s = torch.from_numpy(s_infer).to(dev)
        d_pc = torch.from_numpy(mit2cfm.normal_noise(P, 512, 7)).to(dev)
        d_c = torch.empty((P + gen, 512), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        def time_condition():
            for _ in range(3):
                ctx.condition_device(d_s.data_ptr(), codes, d_pc.data_ptr(), P, d_c.data_ptr())
            ctx.synchronize()
            c0 = torch.cuda.Event(enable_timing=True)
            c1 = torch.cuda.Event(enable_timing=True)
            c0.record(stream)
            for _ in range(a.cond_calls):
                ctx.condition_device(d_s.data_ptr(), codes, d_pc.data_ptr(), P, d_c.data_ptr())
            c1.record(stream)
            ctx.synchronize()
            torch.cuda.synchronize()
            return c0.elapsed_time(c1) / a.cond_calls

        c_ms = time_condition()  # fp32 mode (split operands), the default
        ctx.set_precision("length_regulator", "f16")
        c16_ms = time_condition()
        ctx.set_precision("length_regulator", "f32")
        lr_flops = 2.0 * codes * 512 * 1024 + 4 * 2.0 * gen * 512 * 1536 + 2.0 * gen * 512 * 512
        cp = {"workload": f"length regulator {codes} codes -> {gen} frames + merge with {P} prompt rows",
              "precision": "f32 (split f16 operand pairs)",
              "us_per_call": round(c_ms * 1e3, 2), "algorithmic_gflop": round(lr_flops / 1e9, 3),
              "tflops": round(lr_flops / (c_ms / 1e3) / 1e12, 2),
              "f16_mode": {"us_per_call": round(c16_ms * 1e3, 2),
                           "tflops": round(lr_flops / (c16_ms / 1e3) / 1e12, 2)}}
        if not a.no_cpu_baseline:
            cp["cpu_baseline"] = condition_cpu_baseline(lr_tensors, s_infer, gen, cpu_threads(a))

    # Vocoder (the step after the decode) on this decode's mel.
    voc = None
    if a.voc_calls:
        d_wav = torch.empty(256 * T, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()

        def time_vocoder():
            for _ in range(2):
                ctx.bigvgan_device(d_out.data_ptr(), T, d_wav.data_ptr())
            ctx.synchronize()
            v0 = torch.cuda.Event(enable_timing=True)
            v1 = torch.cuda.Event(enable_timing=True)
            v0.record(stream)
            for _ in range(a.voc_calls):
                ctx.bigvgan_device(d_out.data_ptr(), T, d_wav.data_ptr())
            v1.record(stream)
            ctx.synchronize()
            torch.cuda.synchronize()
            return v0.elapsed_time(v1) / a.voc_calls

        v_ms = time_vocoder()  # fp32 mode (split operands), the default
        ctx.set_precision("vocoder", "f16")
        v16_ms = time_vocoder()
        ctx.set_precision("vocoder", "f32")
        vflops = mit2cfm.bigvgan_flops(T)
        voc = {"workload": f"BigVGAN v2 256x, {T} mel frames -> {256 * T} samples",
               "precision": "f32 (split f16 activation pairs; weight-norm directions exact in f16 with the g/|v| scale in the epilogue: two matrix-core products per term, three for the transposed convs)",
               "ms_per_call": round(v_ms, 3), "samples_per_s": round(256 * T / (v_ms / 1e3), 1),
               "algorithmic_tflop": round(vflops / 1e12, 4),
               "tflops": round(vflops / (v_ms / 1e3) / 1e12, 1),
               "mfma_util": round(vflops / (v_ms / 1e3) / 1e12 / PEAK_F16_TFLOPS, 4),
               "f16_mode": {"ms_per_call": round(v16_ms, 3),
                            "samples_per_s": round(256 * T / (v16_ms / 1e3), 1),
                            "tflops": round(vflops / (v16_ms / 1e3) / 1e12, 1),
                            "mfma_util": round(vflops / (v16_ms / 1e3) / 1e12 / PEAK_F16_TFLOPS, 4)}}
        if not a.no_cpu_baseline:
            voc["cpu_baseline"] = vocoder_cpu_baseline(bv_tensors, d_out.cpu().numpy(), cpu_threads(a))

    # The whole acoustic stage at the reference's published segment
    # (docs/evolution.md:27: 553 codes, 11.0 s audio, 16 steps, acoustic 5.39 s;
    # the voice prompt is 629 frames, docs/evolution.md:14).
    ac = None
    if a.acoustic_calls and a.voc_calls:
        codes_a, P_a, S_a = 553, 629, 16
        gen_a = mit2cfm.generated_frames(codes_a)
        d_si = torch.from_numpy(mit2cfm.normal_noise(codes_a, 1024, 8)).to(dev)
        d_pc_a = torch.from_numpy(mit2cfm.normal_noise(P_a, 512, 9)).to(dev)
        d_pm_a = torch.from_numpy(mit2cfm.normal_noise(P_a, 80, 10, 2.0) - 5.0).to(dev)
        d_wav_a = torch.empty(256 * gen_a, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()

        def acoustic():
            return ctx.acoustic_device(d_si.data_ptr(), codes_a, d_pc_a.data_ptr(), d_pm_a.data_ptr(), P_a,
                                       d_style.data_ptr(), 20240608, 1.0, S_a, cfg, d_wav_a.data_ptr())

        for _ in range(2):
            acoustic()
        ctx.synchronize()
        a0 = torch.cuda.Event(enable_timing=True)
        a1 = torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        for _ in range(a.acoustic_calls):
            acoustic()
        a1.record(stream)
        ctx.synchronize()
        torch.cuda.synchronize()
        a_ms = a0.elapsed_time(a1) / a.acoustic_calls
        audio_s = 256 * gen_a / 22050.0
        ac = {"workload": f"{codes_a} codes -> {gen_a} frames after a {P_a}-frame prompt (T={P_a + gen_a}), "
                          f"{S_a} steps, cfg {cfg}, vocoder -> {256 * gen_a} samples",
              "ms_per_call": round(a_ms, 3), "audio_s": round(audio_s, 3),
              "rtf": round(a_ms / 1e3 / audio_s, 5),
              "reference_published": {"acoustic_s": 5.39, "hardware": "Apple M3 Ultra (Metal/MPS)",
                                      "source": "docs/evolution.md:27, segment 1"},
              "speedup_vs_published": round(5390.0 / a_ms, 1)}

    # Host-pointer decode (upload, decode, readback): PCIe-inclusive, median of
    # 10, reported beside the headline value, never as it.
    ctx.decode(x0, prompt, cond, style, S, cfg)
    pcie_ms, pcie_all = timed_median(lambda: ctx.decode(x0, prompt, cond, style, S, cfg),
                                     lambda: None, a.pcie_reps)

    # First decode of a length this context has not seen: graph capture and
    # instantiation, then the replay of the same shape.
    Tn = T + 1
    d_x0n = torch.from_numpy(mit2cfm.normal_noise(Tn, 80, 11)).to(dev)
    d_cn = torch.from_numpy(mit2cfm.normal_noise(Tn, 512, 12)).to(dev)
    d_on = torch.empty((Tn, 80), dtype=torch.float32, device=dev)

    def new_t():
        ctx.decode_device(d_x0n.data_ptr(), d_prompt.data_ptr(), d_cn.data_ptr(), d_style.data_ptr(), Tn, P, S,
                          cfg, d_on.data_ptr())

    def sync_all():
        ctx.synchronize()
        torch.cuda.synchronize()

    first_ms, _ = timed_median(new_t, sync_all, 1)
    replay_ms, _ = timed_median(new_t, sync_all, 3)
    first_call = {"tokens": Tn, "first_call_ms": round(first_ms, 3), "replay_ms": round(replay_ms, 3),
                  "capture_and_instantiate_ms": round(first_ms - replay_ms, 3),
                  "graph_cache": dict(zip(("held", "capacity"), ctx.graph_count()))}
    ctx.set_graph(False)
    first_call["no_graph_ms"] = round(timed_median(new_t, sync_all, 3)[0], 3)
    ctx.set_graph(True)

    configs = configs_section(a, mit2cfm, ctx, torch, dev) if a.configs else None
    ctx.close()

    result = {
        "metric": METRIC,
        "value": round(frames_per_s, 1),
        "unit": "mel frames/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_decode, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"cfm_decode_T{T}_P{P}_S{S}_cfg{cfg}_B2", "tokens": T,
                   "prompt_tokens": P, "cfm_steps": S, "cfg_rate": cfg, "branches": 2,
                   "weights": "synthetic f16 N(0,0.02) seed 20240605",
                   "step": "one full decode"},
        "cfm_steps_per_s": round(S / (ms_per_decode / 1e3), 1),
        "generated_frames_per_s": round((T - P) / (ms_per_decode / 1e3), 1),
        "event_ms_per_decode": round(ev_ms, 4),
        "decode_mfma_util": round(flops_decode / (ms_per_decode / 1e3) / 1e12 / PEAK_F16_TFLOPS, 4),
        "algorithmic_tflop_per_decode": round(flops_decode / 1e12, 4),
        "pcie_inclusive": {"frames_per_s": round(T / (pcie_ms / 1e3), 1), "median_ms": round(pcie_ms, 3),
                           "runs": len(pcie_all), "min_ms": round(pcie_all[0], 3),
                           "max_ms": round(pcie_all[-1], 3),
                           "what": "host-pointer decode: upload, decode, readback"},
        "first_call": first_call,
        "roofline": roof,
    }
    if configs:
        result["configs"] = configs
    if cp:
        result["condition_producer"] = cp
    if voc:
        result["vocoder"] = voc
    if ac:
        result["acoustic_stage"] = ac
    if a.gpt_codes:
        result["gpt_decode"] = gpt_section(a, mit2cfm, tensors, torch)
    result["context_create_s"] = {"from_host_tensors": round(create_s, 3), "from_device_image": round(create_img_s, 3),
                                  "image_mib": round(img_mb, 1)}
    if not a.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(tensors, T, P, S, cfg, cpu_threads(a))
        result["cpu_baseline"]["nproc"] = os.cpu_count()
        if a.cpu_1thread:
            result["cpu_baseline_1thread"] = cpu_baseline_1thread(tensors)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
