"""Writes the oracle fixtures used by the GPU parity tests at full size.

The reference holds no golden vectors for this path (its PyTorch golden
generators need the upstream checkpoints), so these fixtures are the
oracle's outputs on seeded synthetic weights and inputs; the oracle itself is
pinned by tests/test_oracle_*.py.  Inputs are regenerated from their seeds on
the GPU box, so only outputs (and the oracle states the per-step velocity
check starts from) are stored.

    python tests/golden/make_golden.py [config1|config2|config3 ...]

Configs (benchmark workloads):
  config1  one estimator forward, B=2 CFG pair, T=256 (P=96), t=0.5
  config2  full decode T=860 (P=258), 25 steps, cfg 0.7  (~15 min on 8 threads)
  config3  full decode T=128 (P=48), 12 steps, cfg 0.7
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
}


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
