"""Pins the GPT decoder oracle (oracle/gpt_oracle.c, a restatement of
runtime/impl/gpt.cpp's fp32 CPU path) on the CPU.

The reference ships no GPT golden files (its golden tests read directories
produced by generator scripts that need the real checkpoint), so the oracle
is pinned by independent computations of the same mathematics:

* gelu_new and the two attention forms against closed forms and torch;
* the whole stack (blocks, ln_f, final_norm, mel_head) against Hugging Face
  transformers' GPT2Model -- the published implementation IndexTTS2's
  UnifiedVoice wraps -- with the same weights (checkpoint layouts: Conv1D
  matrices [in][out]) and the position table zeroed, so a transposed
  operand, a wrong LayerNorm or a missing residual fails;
* the cached decode against GPT2Model's own key/value cache;
* the reference's own consistency tests: cached greedy == uncached greedy
  (run_gpt_kv_greedy_test, gpt.cpp:2305) and cached decode == the last row
  of the full logits (run_gpt_kv_decode_test, gpt.cpp:1469);
* the position rule of gpt_cached_generate_position against an explicit
  re-run of the sequence with those positions, and the stop rule.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import sincos_series

W = 1280


@pytest.fixture(scope="module")
def gpt_t(mit2):
    return mit2.synthetic_gpt_tensors(layers=2)


@pytest.fixture(scope="module")
def gpt(orc, gpt_t):
    return orc.GPT(gpt_t)


@pytest.fixture(scope="module")
def hf(gpt_t):
    """GPT2Model with the same two layers; wpe zeroed (the reference adds
    positions to the inputs itself)."""
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    cfg = transformers.GPT2Config(n_embd=W, n_layer=2, n_head=20, n_inner=5120, activation_function="gelu_new",
                                  layer_norm_epsilon=1e-5, n_positions=256, vocab_size=16, resid_pdrop=0.0,
                                  embd_pdrop=0.0, attn_pdrop=0.0, bos_token_id=0, eos_token_id=0)
    cfg._attn_implementation = "eager"
    m = transformers.GPT2Model(cfg).eval()
    sd = {k: torch.zeros_like(v) for k, v in m.state_dict().items()}
    for name, v in gpt_t.items():
        if name.startswith("gpt.gpt."):
            sd[name[len("gpt.gpt."):]] = torch.from_numpy(np.asarray(v, np.float32))
    m.load_state_dict(sd)
    return m


def _head(gpt_t, hidden_ln_f):
    """final_norm + mel_head of HF's last_hidden_state (= ln_f output), float64."""
    x = np.asarray(hidden_ln_f, np.float64)
    g = np.asarray(gpt_t["gpt.final_norm.weight"], np.float64)
    b = np.asarray(gpt_t["gpt.final_norm.bias"], np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    fn = (x - mu) / np.sqrt(var + 1e-5) * g + b
    hw = np.asarray(gpt_t["gpt.mel_head.weight"], np.float64)
    hb = np.asarray(gpt_t["gpt.mel_head.bias"], np.float64)
    return fn, fn @ hw.T + hb


def _rows(n, seed=0, scale=0.05):
    return (np.random.default_rng(seed).standard_normal((n, W)) * scale).astype(np.float32)


def test_gelu_new_closed_form(orc):
    x = np.concatenate([np.linspace(-12, 12, 4001), [-10.0, 10.0, -10.0001, 10.0001]]).astype(np.float32)
    got = orc.gelu_new(x)
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(0.7978845608028654 * (xd + 0.044715 * xd ** 3)))
    ref = np.where(xd > 10, xd, np.where(xd < -10, 0.0, ref))
    assert np.abs(got - ref).max() <= 2e-6 * np.maximum(1, np.abs(ref)).max()
    assert got[-1] == np.float32(10.0001) and got[-2] == 0.0  # the saturation branches


def test_gelu_new_matches_torch_tanh_gelu(orc):
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(1).standard_normal(5000).astype(np.float32) * 4
    ref = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    assert np.abs(orc.gelu_new(x) - ref).max() <= 1e-5


def test_attention_single_query_closed_form(orc):
    rng = np.random.default_rng(2)
    q, k, v = rng.standard_normal(64), rng.standard_normal((37, 64)), rng.standard_normal((37, 64))
    s = k @ q / 8.0
    p = np.exp(s - s.max())
    ref = (p / p.sum()) @ v
    assert np.abs(orc.attention_single_query(q, k, v) - ref).max() <= 1e-5
    # one key: the output is that key's value
    assert np.allclose(orc.attention_single_query(q, k[:1], v[:1]), v[0].astype(np.float32), atol=1e-7)


def test_attention_causal_matches_torch(orc):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((23, 64)).astype(np.float32) for _ in range(3))
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[None], torch.from_numpy(k)[None], torch.from_numpy(v)[None], is_causal=True)[0]
    assert np.abs(orc.attention_causal(q, k, v) - ref.numpy()).max() <= 1e-5
    # row t is the single-query form over keys 0..t
    assert np.array_equal(orc.attention_causal(q, k, v)[7], orc.attention_single_query(q[7], k[:8], v[:8]))


def test_stack_matches_hf_gpt2(gpt, gpt_t, hf):
    torch = pytest.importorskip("torch")
    x = sincos_series(9 * W, 0.009, 0.013, 0.065, 0.021, 307).reshape(9, W)
    fn, logits, am = gpt.logits(x)
    with torch.no_grad():
        h = hf(inputs_embeds=torch.from_numpy(x)[None]).last_hidden_state[0].double().numpy()
    ref_fn, ref_logits = _head(gpt_t, h)
    assert np.abs(fn - ref_fn).max() <= 2e-4
    err = np.abs(logits - ref_logits).max() / np.abs(ref_logits).max()
    assert err <= 2e-5, err
    assert am == int(np.argmax(ref_logits[-1]))


def test_block_matches_hf_gpt2(gpt, hf):
    """Block 0's output against GPT2Model's first hidden state (the last one
    is after ln_f, so the stack test above covers block 1)."""
    torch = pytest.importorskip("torch")
    x = _rows(6, 4, 0.5)
    with torch.no_grad():
        hs = hf(inputs_embeds=torch.from_numpy(x)[None], output_hidden_states=True).hidden_states
    ref = hs[1][0].numpy()
    assert np.abs(gpt.block(x, 0) - ref).max() / np.abs(ref).max() <= 2e-5


def test_cached_decode_matches_hf_kv_cache(gpt, gpt_t, hf):
    torch = pytest.importorskip("torch")
    rows = _rows(6, 5, 0.3)
    ln_f, fn, logits, am = gpt.cached_decode(rows, 5)
    with torch.no_grad():
        out = hf(inputs_embeds=torch.from_numpy(rows[:5])[None], use_cache=True)
        out2 = hf(inputs_embeds=torch.from_numpy(rows[5:])[None], past_key_values=out.past_key_values)
        h = out2.last_hidden_state[0, -1].double().numpy()
    assert np.abs(ln_f - h).max() <= 2e-4
    _, ref_logits = _head(gpt_t, h)
    assert np.abs(logits - ref_logits).max() / np.abs(ref_logits).max() <= 2e-5
    assert am == int(np.argmax(ref_logits))


def test_cached_decode_equals_full_last_row(gpt):
    """run_gpt_kv_decode_test (gpt.cpp:1469-1504): 3 prefix rows + 1, its input series."""
    x = sincos_series(4 * W, 0.009, 0.013, 0.065, 0.021, 307).reshape(4, W)
    fn_full, logits_full, am_full = gpt.logits(x)
    _, fn, logits, am = gpt.cached_decode(x, 3)
    assert np.abs(logits - logits_full[-1]).max() <= 2e-3  # the reference's bar; here exact
    assert np.array_equal(logits, logits_full[-1]) and np.array_equal(fn, fn_full[-1])
    assert am == am_full


def test_kv_greedy_equals_uncached_greedy(gpt):
    """run_gpt_kv_greedy_test (gpt.cpp:2305-2371): cached and uncached greedy
    loops give the same tokens and last logits."""
    prefix = sincos_series(10 * W, 0.007, 0.011, 0.045, 0.018, 251).reshape(10, W)
    a = gpt.kv_greedy(prefix, 5)
    b = gpt.greedy_full(prefix, 5)
    assert np.array_equal(a["predicted"], b["predicted"])
    assert np.array_equal(a["input_tokens"], b["input_tokens"])
    assert a["first_stop_step"] == b["first_stop_step"] == -1
    assert np.abs(a["last_logits"] - b["last_logits"]).max() <= 3e-3
    assert a["input_tokens"][0] == 8192 and len(a["input_tokens"]) == 6


def test_hf_positions_follow_generate_rule(gpt, gpt_t):
    """gpt_cached_generate_position (gpt.cpp:1873): step s > 0 embeds its token at
    position s + 1.  Re-running the whole sequence with those positions gives
    the cached loop's last logits."""
    prefix = _rows(4, 6)
    r = gpt.kv_greedy(prefix, 4, hf_generate_positions=True)
    toks = r["input_tokens"]
    emb = np.asarray(gpt_t["gpt.mel_embedding.weight"], np.float32)
    pos = np.asarray(gpt_t["gpt.mel_pos_embedding.emb.weight"], np.float32)
    positions = [0] + [s + 1 for s in range(1, len(toks))]
    seq = np.concatenate([prefix, np.stack([emb[t] + pos[p] for t, p in zip(toks[:4], positions[:4])])])
    _, logits, am = gpt.logits(seq)
    assert np.array_equal(logits[-1], r["last_logits"])
    assert am == r["predicted"][-1]
    plain = gpt.kv_greedy(prefix, 4)
    assert plain["predicted"][0] == r["predicted"][0]  # step 0 uses position 0 either way
    assert not np.array_equal(plain["last_logits"], r["last_logits"])


def test_stop_token_ends_the_cached_loop(orc, gpt_t):
    t = dict(gpt_t)
    b = np.asarray(t["gpt.mel_head.bias"], np.float32).copy()
    b[8193] = 100.0
    t["gpt.mel_head.bias"] = b
    g = orc.GPT(t)
    r = g.kv_greedy(_rows(3, 7), 6)
    assert r["first_stop_step"] == 0
    assert r["predicted"].tolist() == [8193] and r["input_tokens"].tolist() == [8192]
    full = g.greedy_full(_rows(3, 7), 3)  # the uncached loop records the stop but goes on
    assert full["first_stop_step"] == 0 and len(full["predicted"]) == 3


def test_position_table_bound(gpt):
    with pytest.raises(ValueError):
        gpt.kv_greedy(_rows(1, 8), 1819)


def test_planted_mistake_is_caught(orc, gpt_t, hf):
    """A transposed c_proj (the Conv1D layout taken as [out][in]) is caught by the
    transformers pin above."""
    torch = pytest.importorskip("torch")
    t = dict(gpt_t)
    w = np.asarray(t["gpt.gpt.h.0.attn.c_proj.weight"], np.float32)
    t["gpt.gpt.h.0.attn.c_proj.weight"] = np.ascontiguousarray(w.T)
    x = sincos_series(5 * W, 0.009, 0.013, 0.065, 0.021, 307).reshape(5, W)
    _, logits, _ = orc.GPT(t).logits(x)
    with torch.no_grad():
        h = hf(inputs_embeds=torch.from_numpy(x)[None]).last_hidden_state[0].double().numpy()
    _, ref_logits = _head(gpt_t, h)
    assert np.abs(logits - ref_logits).max() / np.abs(ref_logits).max() > 1e-3


def test_sampling_processors_reference_vector(orc):
    """run_gpt_sampling_processors_test (gpt.cpp:1757-1800): its logits, history
    and settings; its expected filtering, values and sampled token."""
    logits = np.arange(-2, 8, dtype=np.float32)
    processed = orc.gpt_sampling_processors(logits, [2, 7, 3, 7], temperature=0.5, top_k=4, top_p=0.95,
                                            repetition_penalty=2.0)
    assert not np.isfinite(processed[[0, 5, 6]]).any()
    assert np.isfinite(processed[[8, 9]]).all()
    assert abs(processed[8] - 12.0) <= 1e-6 and abs(processed[9] - 14.0) <= 1e-6
    rng = np.array([20240605], np.uint64)
    assert orc.gpt_sample_token(processed, rng) == 9


def test_sampling_processors_closed_forms(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal(300).astype(np.float32) * 3
    # temperature alone divides; top_k keeps the k largest (ties kept); top_p keeps the
    # smallest set of largest scores whose mass exceeds top_p
    assert np.array_equal(orc.gpt_sampling_processors(x, [], temperature=0.7), x / np.float32(0.7))
    k = orc.gpt_sampling_processors(x, [], top_k=17)
    assert np.isfinite(k).sum() == 17 and np.array_equal(np.sort(np.where(np.isfinite(k))[0]),
                                                         np.sort(np.argsort(-x)[:17]))
    p = orc.gpt_sampling_processors(x, [], top_p=0.6)
    order = np.argsort(-x.astype(np.float64), kind="stable")
    prob = np.exp(x[order].astype(np.float64) - x.max())
    prob /= prob.sum()
    keep = np.searchsorted(np.cumsum(prob), 0.6) + 1  # the head whose mass first passes 0.6
    assert set(np.where(np.isfinite(p))[0]) == set(order[:keep].tolist())
    # repetition penalty: once per distinct token, divide positives, multiply negatives
    h = [3, 3, 9, 250]
    r = orc.gpt_sampling_processors(x, h, repetition_penalty=1.3)
    ref = x.copy()
    for t in set(h):
        ref[t] = ref[t] / np.float32(1.3) if ref[t] >= 0 else ref[t] * np.float32(1.3)
    assert np.array_equal(r, ref)


def test_sample_token_follows_the_distribution(orc):
    x = np.log(np.array([0.1, 0.2, 0.3, 0.4], np.float32))
    rng = np.array([7], np.uint64)
    draws = [orc.gpt_sample_token(x, rng) for _ in range(4000)]
    freq = np.bincount(draws, minlength=4) / 4000
    assert np.abs(freq - [0.1, 0.2, 0.3, 0.4]).max() < 0.03


def test_kv_sample_with_greedy_settings_equals_greedy(gpt):
    """top_k = 1 leaves only the maximum, so sampling picks the greedy token."""
    prefix = _rows(6, 12)
    s = gpt.kv_sample(prefix, 4, seed=5, top_k=1)
    g = gpt.kv_greedy(prefix, 4)
    assert s["predicted"].tolist() == g["predicted"].tolist()


def test_kv_sample_history_prefix(gpt):
    """repetition_history_prefix (gpt.cpp:2224-2229): a prefix of [8192] alone is
    the default history; a fake_inputs-shaped prefix ([1] x n + [8192],
    gpt.cpp:66-67) additionally penalises token 1 from the first step, and
    nothing else (no temperature or filter: the other scores stay raw)."""
    prefix = _rows(6, seed=31)
    cfg = dict(temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=3.0)
    default = gpt.kv_sample(prefix, 1, 9, **cfg)
    start = gpt.kv_sample(prefix, 1, 9, history=[8192], **cfg)
    fake = gpt.kv_sample(prefix, 1, 9, history=[1] * 6 + [8192], **cfg)
    assert np.array_equal(default["last_processed_logits"], start["last_processed_logits"])
    raw = fake["last_logits"]
    want = raw.copy()
    for t in (1, 8192):
        want[t] = raw[t] / np.float32(3.0) if raw[t] >= 0 else raw[t] * np.float32(3.0)
    assert np.array_equal(fake["last_processed_logits"], want)
    # an empty prefix (the reference's empty vector) replaces the start token:
    # nothing is penalised at the first step
    empty = gpt.kv_sample(prefix, 1, 9, history=[], **cfg)
    assert np.array_equal(empty["last_processed_logits"], empty["last_logits"])
    assert not np.array_equal(empty["last_processed_logits"], default["last_processed_logits"])
    # later steps: the predictions join the prefix in the history
    long = gpt.kv_sample(prefix, 4, 9, history=[1] * 6 + [8192], **cfg)
    again = gpt.kv_sample(prefix, 4, 9, history=[1] * 6 + [8192] + [8192], **cfg)
    assert long["predicted"].tolist() == again["predicted"].tolist()  # duplicates count once
