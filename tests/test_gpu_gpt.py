"""GPU parity of the GPT mel-code decoder (runtime/impl/gpt.cpp) through the C
ABI against the CPU oracle on identical inputs and weights.

The reference holds its Metal decode to max-abs 3e-3 on the last logits and
identical tokens against its CPU path (run_gpt_kv_greedy_test,
gpt.cpp:2305-2371), and to 2e-3 on the cached single-row decode
(run_gpt_kv_decode_test, :1469-1504).  Here the weights are f16 on both
sides (the checkpoint's precision) and everything else fp32, so the only
difference is the order of fp32 sums; the bars below are the reference's.

The cached attention splits its keys into blocks of 256 (the GPT_ATTN_KEYS
build knob): each split writes its max, exp-sum and unnormalised output, and
a combine launch merges the splits eight at a time, rescaling the running
sums when a later group raises the max.  Prefixes of a few rows, of 509 / 511
(a split boundary), 600 (three splits), 2,100 (nine splits: the combine's
second pass) and 2,303 (the cache ends exactly on a split boundary) exercise
one split, the boundary and the rescaling; prefill chunks hold 8 rows.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import sincos_series

pytestmark = pytest.mark.gpu

W = 1280
LOGITS_TOL = 3e-3   # run_gpt_kv_greedy_test's bar on the last logits (max-abs)
DECODE_TOL = 2e-3   # run_gpt_kv_decode_test's bar (max-abs)


@pytest.fixture(scope="module")
def gpt24_t(mit2):
    return mit2.synthetic_gpt_tensors()


@pytest.fixture(scope="module")
def ctx24(mit2, tensors, gpt24_t):
    c = mit2.Context({**tensors, **gpt24_t}, device=0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def orc24(orc, gpt24_t):
    return orc.GPT(gpt24_t)


@pytest.fixture(scope="module")
def gpt2_t(mit2):
    return mit2.synthetic_gpt_tensors(layers=2)


@pytest.fixture(scope="module")
def ctx2(mit2, tensors, gpt2_t):
    c = mit2.Context({**tensors, **gpt2_t}, device=0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def orc2(orc, gpt2_t):
    return orc.GPT(gpt2_t)


def _prefix(n, seed=None):
    if seed is None:  # run_gpt_kv_greedy_test's conditioning series (gpt.cpp:2313-2316)
        return sincos_series(n * W, 0.007, 0.011, 0.045, 0.018, 251).reshape(n, W)
    return (np.random.default_rng(seed).standard_normal((n, W)) * 0.05).astype(np.float32)


def _compare(got, ref, label):
    err = float(np.abs(got["last_logits"] - ref["last_logits"]).max()) if ref["last_logits"] is not None else 0.0
    print(f"{label}: tokens {got['predicted'].tolist()[:12]} stop {got['first_stop_step']} "
          f"logits max-abs {err:.2e} prefill {got['prefill_ms']:.2f} ms decode {got['decode_ms']:.2f} ms",
          flush=True)
    assert got["predicted"].tolist() == ref["predicted"].tolist()
    assert got["input_tokens"].tolist() == ref["input_tokens"].tolist()
    assert got["first_stop_step"] == ref["first_stop_step"]
    assert err <= LOGITS_TOL


def test_layers(ctx24, ctx2, mit2, tensors):
    assert ctx24.gpt_layers() == 24 and ctx2.gpt_layers() == 2
    c = mit2.Context(tensors, device=0)
    try:
        assert c.gpt_layers() == 0
        with pytest.raises(mit2.Mit2CfmError) as e:
            c.gpt_kv_greedy(_prefix(2), 1)
        assert e.value.status == mit2.E_MODEL
    finally:
        c.close()


def test_cached_decode_reference_input(ctx24, orc24):
    """run_gpt_kv_decode_test (gpt.cpp:1469-1504): 3 prefix rows + 1, its series."""
    x = sincos_series(4 * W, 0.009, 0.013, 0.065, 0.021, 307).reshape(4, W)
    ln_f, fn, logits, am = ctx24.gpt_cached_decode(x, 3)
    r_ln_f, r_fn, r_logits, r_am = orc24.cached_decode(x, 3)
    errs = [float(np.abs(a - b).max()) for a, b in ((ln_f, r_ln_f), (fn, r_fn), (logits, r_logits))]
    print(f"cached decode: ln_f {errs[0]:.2e} final_norm {errs[1]:.2e} logits {errs[2]:.2e} argmax {am}/{r_am}",
          flush=True)
    assert max(errs) <= DECODE_TOL and am == r_am


@pytest.mark.parametrize("P,steps,hf", [(10, 3, False), (20, 12, True), (100, 8, False)])
def test_kv_greedy_matches_oracle_24_layers(ctx24, orc24, P, steps, hf):
    prefix = _prefix(P)
    print(f"kv greedy 24 layers P={P} steps={steps} hf={hf}", flush=True)
    _compare(ctx24.gpt_kv_greedy(prefix, steps, hf), orc24.kv_greedy(prefix, steps, hf), "  24 layers")


@pytest.mark.parametrize("P,steps", [(0, 3), (1, 2), (63, 3), (300, 10), (509, 5), (511, 3), (600, 4),
                                     (2100, 4), (2303, 2)])
def test_kv_greedy_attention_chunks(ctx2, orc2, P, steps):
    prefix = _prefix(P, seed=P)
    print(f"kv greedy 2 layers P={P} steps={steps}", flush=True)
    _compare(ctx2.gpt_kv_greedy(prefix, steps), orc2.kv_greedy(prefix, steps), "  2 layers")


def test_zero_steps(ctx2):
    r = ctx2.gpt_kv_greedy(_prefix(5), 0)
    assert r["predicted"].size == 0 and r["input_tokens"].tolist() == [8192]
    assert r["first_stop_step"] == -1 and r["last_logits"] is None


def test_repeatable_and_independent_of_earlier_calls(ctx2):
    prefix = _prefix(40, seed=9)
    a = ctx2.gpt_kv_greedy(prefix, 9)
    ctx2.gpt_kv_greedy(_prefix(500, seed=10), 30)  # a longer call in between grows the caches
    b = ctx2.gpt_kv_greedy(prefix, 9)
    assert a["predicted"].tolist() == b["predicted"].tolist()
    assert np.array_equal(a["last_logits"], b["last_logits"])


def test_greedy_last_step_equals_cached_decode(ctx24, gpt24_t):
    """The decode loop's last logits equal a cached decode of the same sequence
    (prefix rows, then each input token's embedding at its position)."""
    prefix = _prefix(150, seed=11)
    r = ctx24.gpt_kv_greedy(prefix, 40)
    toks = r["input_tokens"]
    emb = np.asarray(gpt24_t["gpt.mel_embedding.weight"], np.float32)
    pos = np.asarray(gpt24_t["gpt.mel_pos_embedding.emb.weight"], np.float32)
    n = len(r["predicted"])
    rows = np.concatenate([prefix, np.stack([emb[toks[t]] + pos[t] for t in range(n)])])
    _, _, logits, am = ctx24.gpt_cached_decode(rows, len(rows) - 1)
    err = float(np.abs(logits - r["last_logits"]).max())
    print(f"greedy ({n} steps, {r['decode_ms']:.2f} ms) vs cached decode: logits max-abs {err:.2e}", flush=True)
    assert am == r["predicted"][-1] and err <= 1e-4


def _with_stop_bias(t, delta):
    t = dict(t)
    b = np.asarray(t["gpt.mel_head.bias"], np.float32).copy()
    b[8193] += np.float32(delta)
    t["gpt.mel_head.bias"] = b
    return t


def _mid_run_stop(g, steps):
    """A prefix and a stop-token bias increase under which the stop token wins
    at a step s in 1..steps-1 and at no earlier step (None when no seed tried
    offers a margin of 0.02 either way)."""
    for seed in range(12, 40):
        prefix = _prefix(12, seed=seed)
        gaps = []  # per step: best other token's logit minus the stop token's
        for s in range(1, steps + 1):
            lg = g.kv_greedy(prefix, s)["last_logits"]
            gaps.append(float(np.delete(lg, 8193).max() - lg[8193]))
        for s in range(1, steps):
            earlier = min(gaps[:s])
            if 0 < gaps[s] < earlier - 0.04:
                return prefix, s, 0.5 * (gaps[s] + earlier)
    return None


def test_stop_token(mit2, orc, tensors, gpt2_t):
    """A stop at step 0, and one in the middle of a run (inside a group of
    steps between the host's stop-flag checks): the bias of the stop token is
    raised just enough that it wins at one later step and at no earlier one."""
    found = _mid_run_stop(orc.GPT(gpt2_t), 7)
    assert found is not None, "no seed offers a clean mid-run stop"
    prefix, step, delta = found
    for delta, expect in ((100.0, 0), (delta, step)):
        t = _with_stop_bias(gpt2_t, delta)
        ref = orc.GPT(t).kv_greedy(prefix, 12)
        assert ref["first_stop_step"] == expect
        c = mit2.Context({**tensors, **t}, device=0)
        try:
            _compare(c.gpt_kv_greedy(prefix, 12), ref, f"  stop at {expect}")
        finally:
            c.close()


def test_position_table_bound(ctx2, mit2):
    with pytest.raises(mit2.Mit2CfmError) as e:
        ctx2.gpt_kv_greedy(_prefix(2), 1818, hf_generate_positions=True)
    assert e.value.status == mit2.E_ARG


@pytest.mark.parametrize("P", [1, 7, 8, 9, 100])
def test_chunked_prefill_equals_row_prefill(ctx2, monkeypatch, P):
    """The prefill's chunks of 8 rows give the values of prefilling one row at a
    time through the decode step's kernels (same sums in the same order)."""
    prefix = _prefix(P, seed=20 + P)
    chunked = ctx2.gpt_kv_greedy(prefix, 4)
    monkeypatch.setenv("MIT2CFM_GPT_ROW_PREFILL", "1")
    rows = ctx2.gpt_kv_greedy(prefix, 4)
    err = float(np.abs(chunked["last_logits"] - rows["last_logits"]).max())
    print(f"P={P}: chunked prefill {chunked['prefill_ms']:.2f} ms, row prefill {rows['prefill_ms']:.2f} ms, "
          f"logits max-abs {err:.2e}", flush=True)
    assert chunked["predicted"].tolist() == rows["predicted"].tolist()
    assert err <= 1e-5


# IndexTTS2's generation settings (do_sample, top_p 0.8, top_k 30, temperature
# 0.8, repetition_penalty 10.0) and settings that take the sampler's other paths.
SAMPLING_CASES = [
    dict(temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0),
    dict(temperature=1.0, top_k=4, top_p=0.95, repetition_penalty=2.0),
    dict(temperature=0.7, top_k=0, top_p=0.9, repetition_penalty=1.0),   # top-p over every token
    dict(temperature=1.3, top_k=0, top_p=1.0, repetition_penalty=1.0),   # no filter
    dict(temperature=1.0, top_k=1, top_p=1.0, repetition_penalty=1.0),   # = greedy
]


def _compare_sampled(got, ref, label):
    _compare(got, ref, label)
    a, b = got["last_processed_logits"], ref["last_processed_logits"]
    assert np.array_equal(np.isfinite(a), np.isfinite(b))
    fin = np.isfinite(b)
    assert np.abs(a[fin] - b[fin]).max() <= LOGITS_TOL * 10  # temperature / penalty scale the logits


def test_sampled_decode_matches_oracle_24_layers(ctx24, orc24):
    prefix = _prefix(20)
    cfg = SAMPLING_CASES[0]
    print(f"sampled 24 layers {cfg}", flush=True)
    _compare_sampled(ctx24.gpt_kv_sample(prefix, 10, 20240605, **cfg),
                     orc24.kv_sample(prefix, 10, 20240605, **cfg), "  24 layers sampled")


@pytest.mark.parametrize("case", range(len(SAMPLING_CASES)))
def test_sampled_decode_paths(ctx2, orc2, case):
    prefix = _prefix(30, seed=40 + case)
    cfg = SAMPLING_CASES[case]
    print(f"sampled 2 layers {cfg}", flush=True)
    got = ctx2.gpt_kv_sample(prefix, 12, 7 + case, **cfg)
    _compare_sampled(got, orc2.kv_sample(prefix, 12, 7 + case, **cfg), "  2 layers sampled")
    if cfg["top_k"] == 1:
        assert got["predicted"].tolist() == ctx2.gpt_kv_greedy(prefix, 12)["predicted"].tolist()


def test_sampled_decode_with_fake_inputs_history_24_layers(ctx24, orc24):
    """The synthesis path's sampled call (synthesis_pipeline.cpp:795-802) passes
    the prefix's fake_inputs, [1] x P + [8192] (gpt.cpp:66-67), as the
    repetition-history prefix, so token 1 is penalised from the first step;
    IndexTTS2's settings, tokens and logits against the oracle."""
    P = 20
    prefix = _prefix(P, seed=77)
    hist = [1] * P + [8192]
    cfg = SAMPLING_CASES[0]
    got = ctx24.gpt_kv_sample(prefix, 10, 20240609, history=hist, **cfg)
    ref = orc24.kv_sample(prefix, 10, 20240609, history=hist, **cfg)
    _compare_sampled(got, ref, "  24 layers sampled, fake_inputs history")


def test_history_prefix_penalises_its_tokens(ctx2, orc2):
    """With no temperature or filtering the processed logits are the raw ones
    except the history's tokens, scaled by the penalty (divided when positive,
    multiplied when negative): token 1 from a fake_inputs history; a history of
    [8192] alone is the default."""
    prefix = _prefix(12, seed=78)
    cfg = dict(temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=2.0)
    with_h = ctx2.gpt_kv_sample(prefix, 1, 5, history=[1] * 12 + [8192], **cfg)
    without = ctx2.gpt_kv_sample(prefix, 1, 5, **cfg)
    start_only = ctx2.gpt_kv_sample(prefix, 1, 5, history=[8192], **cfg)
    raw = with_h["last_logits"]
    want = raw.copy()
    for t in (1, 8192):
        want[t] = raw[t] / 2.0 if raw[t] >= 0 else raw[t] * 2.0
    assert np.array_equal(with_h["last_processed_logits"], want.astype(np.float32))
    assert without["last_processed_logits"][1] == raw[1]
    assert np.array_equal(start_only["last_processed_logits"], without["last_processed_logits"])
    _compare_sampled(with_h, orc2.kv_sample(prefix, 1, 5, history=[1] * 12 + [8192], **cfg), "  2 layers history")
    # An empty prefix (non-NULL, count 0) replaces the start token, as the
    # reference's empty vector does: nothing is penalised at the first step,
    # and later steps penalise the predictions alone.
    empty = ctx2.gpt_kv_sample(prefix, 1, 5, history=[], **cfg)
    assert np.array_equal(empty["last_processed_logits"], empty["last_logits"])
    _compare_sampled(ctx2.gpt_kv_sample(prefix, 6, 5, history=[], **cfg),
                     orc2.kv_sample(prefix, 6, 5, history=[], **cfg), "  2 layers empty history")


def test_sampling_settings_rejected(ctx2, mit2):
    for bad in (dict(temperature=0.0), dict(repetition_penalty=0.0), dict(top_p=0.0), dict(top_p=1.5)):
        with pytest.raises(mit2.Mit2CfmError) as e:
            ctx2.gpt_kv_sample(_prefix(3), 2, 1, **bad)
        assert e.value.status == mit2.E_ARG
