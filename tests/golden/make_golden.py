"""Writes the oracle fixtures used by the GPU parity tests at full size.

The reference holds no golden vectors for this path (its PyTorch golden
generators need the upstream checkpoints), so these fixtures are the
oracle's outputs on seeded synthetic weights and inputs; the oracle itself is
pinned by tests/test_oracle_*.py.  Inputs are regenerated from their seeds
where the tests run, so only outputs (and the oracle states the per-step velocity
check starts from) are stored.

    python tests/golden/make_golden.py [config1|config2|config3 ...]

Configs (benchmark workloads):
  config1  one estimator forward, B=2 CFG pair, T=256 (P=96), t=0.5
  config2  full decode T=860 (P=258), 25 steps, cfg 0.7  (~15 min on 8 threads)
  config3  full decode T=128 (P=48), 12 steps, cfg 0.7
  config4  T=3000 (P=258): the CFG-pair velocity at three Euler states, t=0 on x0
           and steps 12 and 24 of 25 on blends of x0 and a mel-like state (~9 min on
           8 threads)
  config5  8 requests, P=258, target lengths U{300..1500} from one seed, right-padded
           (B=16 rows): the masked CFG-pair velocity at t=0 of the shortest and the
           longest request at the padded length (~4 min on 8 threads)
  config5t the same batch decoded for 2 Euler steps: the final mel of the shortest and of
           the longest request from the masked oracle decode at the padded length (~4 min
           on 8 threads)
  config4t T=3000 (P=258): the first 2 Euler steps of the 25-step schedule -- the guided
           velocity of each step and the state after them (~4 min on 8 threads)
"""
from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "index-tts2-metal_amd"))

import mit2cfm  # noqa: E402  (seeded generator + synthetic inventory only)
from oracle import oracle  # noqa: E402

WEIGHT_SEED = 20240605
WEIGHT_STD = 0.02

CONFIGS = {
    "config1": dict(kind="forward", T=256, P=96, t=0.5, seed=1),
    "config2": dict(kind="decode", T=860, P=258, steps=25, cfg=0.7, seed=1, keep_steps=[0, 12, 24]),
    "config3": dict(kind="decode", T=128, P=48, steps=12, cfg=0.7, seed=1, keep_steps=[0, 11]),
    "config4": dict(kind="states", T=3000, P=258, steps=25, cfg=0.7, seed=1, mid_step=12,
                    late_step=24),
    "config5": dict(kind="padded", nreq=8, P=258, lo=300, hi=1500, len_seed=5, steps=16, cfg=0.7,
                    seed=100),
    "config5t": dict(kind="padded_decode", nreq=8, P=258, lo=300, hi=1500, len_seed=5, steps=2,
                     cfg=0.7, seed=100),
    "config4t": dict(kind="partial", T=3000, P=258, steps=25, run_steps=2, cfg=0.7, seed=1),
}


def splitmix64(state: int):
    """One splitmix64 step (the generator of the seeded inputs); returns (value, state)."""
    state = (state + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
    return z ^ (z >> 31), state


def request_lengths(n: int, lo: int, hi: int, seed: int) -> list[int]:
    """Target lengths uniform in [lo, hi] from one seed (splitmix64 modulo)."""
    out, st = [], seed
    for _ in range(n):
        v, st = splitmix64(st)
        out.append(lo + v % (hi - lo + 1))
    return out


def padded_requests(c):
    """Config-5 batch: per-request totals T_r = P + L_r, right-padded to T_max.
    Request r uses input seeds seed + 10 r .. + 3 at its own length."""
    L = request_lengths(c["nreq"], c["lo"], c["hi"], c["len_seed"])
    toks = [c["P"] + l for l in L]
    tmax = max(toks)
    n = c["nreq"]
    X0 = np.zeros((n, tmax, 80), np.float32)
    PR = np.zeros((n, tmax, 80), np.float32)
    CO = np.zeros((n, tmax, 512), np.float32)
    ST = np.zeros((n, 192), np.float32)
    for r, t in enumerate(toks):
        a, b, cc, s = inputs(t, c["P"], c["seed"] + 10 * r)
        X0[r, :t] = a
        PR[r, :c["P"]] = b
        CO[r, :t] = cc
        ST[r] = s
    return toks, tmax, X0, PR, CO, ST


def step_time(s: int, steps: int) -> float:
    """t of Euler step s, accumulated in fp32 by dt = 1/steps."""
    t = np.float32(0.0)
    dt = np.float32(1.0 / steps)
    for _ in range(s):
        t = np.float32(t + dt)
    return float(t)


def mid_state(x0, T, P, seed, t):
    """(1 - t) x0 + t m with m a mel-like N(-5, 2) field; prompt rows zero."""
    m = mit2cfm.normal_noise(T, 80, seed + 7, 2.0) - 5.0
    x = (np.float32(1.0 - t) * x0 + np.float32(t) * m).astype(np.float32)
    x[:P] = 0
    return x


def pair_velocity(model, x, prompt, cond, style, T, P, t, cfg, mask):
    """v = (1+cfg) est(x, prompt_x, cond, style) - cfg est(x, 0, 0, 0) at flow time t."""
    px = np.zeros((T, 80), np.float32)
    px[:P] = prompt[:P]
    d_c = model.estimator_step(x, px, cond, style, t, mask)
    d_u = model.estimator_step(x, np.zeros_like(px), np.zeros_like(cond), np.zeros_like(style), t, mask)
    return (np.float32(1 + cfg) * d_c - np.float32(cfg) * d_u).astype(np.float32)


def inputs(T: int, P: int, seed: int):
    """x0, content, style ~ N(0,1); prompt mel ~ N(-5, 2) (seeds seed..seed+3)."""
    x0 = mit2cfm.normal_noise(T, 80, seed)
    cond = mit2cfm.normal_noise(T, 512, seed + 1)
    style = mit2cfm.normal_noise(1, 192, seed + 2)[0]
    prompt = mit2cfm.normal_noise(max(P, 1), 80, seed + 3, 2.0)[:P] - 5.0
    return x0, prompt, cond, style


def weights_digest(tensors: dict) -> str:
    h = hashlib.sha256()
    for name in sorted(tensors):
        h.update(name.encode())
        h.update(np.ascontiguousarray(tensors[name]).tobytes())
    return h.hexdigest()


def make(name: str, model, digest: str) -> None:
    c = CONFIGS[name]
    if "T" in c:
        T, P = c["T"], c["P"]
        x0, prompt, cond, style = inputs(T, P, c["seed"])
    t0 = time.time()
    out = {}
    if c["kind"] == "forward":
        x = x0.copy()
        x[:P] = 0
        px = np.zeros((T, 80), np.float32)
        px[:P] = prompt
        mask = np.ones(T, np.uint32)
        out["dphi_cond"] = model.estimator_step(x, px, cond, style, c["t"], mask)
        out["dphi_null"] = model.estimator_step(x, np.zeros_like(px), np.zeros_like(cond),
                                                np.zeros_like(style), c["t"], mask)
    elif c["kind"] == "states":
        mask = np.ones(T, np.uint32)
        x = x0.copy()
        x[:P] = 0
        out["v_t0"] = pair_velocity(model, x, prompt, cond, style, T, P, 0.0, c["cfg"], mask)
        tm = step_time(c["mid_step"], c["steps"])
        out["v_mid"] = pair_velocity(model, mid_state(x0, T, P, c["seed"], tm), prompt, cond, style,
                                     T, P, tm, c["cfg"], mask)
        tl = step_time(c["late_step"], c["steps"])
        out["v_late"] = pair_velocity(model, mid_state(x0, T, P, c["seed"], tl), prompt, cond, style,
                                      T, P, tl, c["cfg"], mask)
    elif c["kind"] == "padded":
        toks, tmax, X0, PR, CO, ST = padded_requests(c)
        picks = [int(np.argmin(toks)), int(np.argmax(toks))]
        for r in picks:
            mask = (np.arange(tmax) < toks[r]).astype(np.uint32)
            x = X0[r].copy()
            x[:c["P"]] = 0
            v = pair_velocity(model, x, PR[r], CO[r], ST[r], tmax, c["P"], 0.0, c["cfg"], mask)
            out[f"v_t0_req{r}"] = v[:toks[r]]
        c = dict(c, tokens=toks, t_max=tmax, picked=picks)
    elif c["kind"] == "padded_decode":
        toks, tmax, X0, PR, CO, ST = padded_requests(c)
        picks = [int(np.argmin(toks)), int(np.argmax(toks))]
        for r in picks:
            mask = (np.arange(tmax) < toks[r]).astype(np.uint32)
            final = model.cfm_euler_masked(X0[r], PR[r][:c["P"]], CO[r], ST[r], mask, c["steps"],
                                           c["cfg"])
            out[f"final_req{r}"] = final[:toks[r]]
        c = dict(c, tokens=toks, t_max=tmax, picked=picks)
    elif c["kind"] == "partial":
        x_after, xt, vt = model.cfm_euler_partial(x0, prompt, cond, style, c["steps"], c["run_steps"],
                                                  c["cfg"])
        out["x_after"] = x_after
        for s in range(c["run_steps"]):
            out[f"v_step{s}"] = vt[s]
    else:
        final, xt, vt = model.cfm_euler(x0, prompt, cond, style, c["steps"], c["cfg"], trace=True)
        out["final"] = final
        for s in c["keep_steps"]:
            out[f"x_step{s}"] = xt[s]
            out[f"v_step{s}"] = vt[s]
    meta = dict(c, weight_seed=WEIGHT_SEED, weight_std=WEIGHT_STD, weights_sha256=digest,
                oracle_seconds=round(time.time() - t0, 1), threads=oracle.lib().orc_get_threads())
    np.savez_compressed(HERE / f"{name}.npz", **out)
    (HERE / f"{name}.json").write_text(json.dumps(meta, indent=1) + "\n")
    print(f"{name}: {meta['oracle_seconds']} s", flush=True)


def main(argv):
    names = argv or list(CONFIGS)
    tensors = mit2cfm.synthetic_tensors(WEIGHT_SEED, WEIGHT_STD)
    digest = weights_digest(tensors)
    oracle.set_threads(oracle.default_threads())
    model = oracle.Model(tensors)
    for n in names:
        make(n, model, digest)


if __name__ == "__main__":
    main(sys.argv[1:])
