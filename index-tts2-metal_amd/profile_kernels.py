"""Kernel-profiling driver for rocprofv3 runs of the decoder's hot kernels.

Builds a context on the synthetic weights, runs one CFG decode at the given
length (so every workspace buffer holds real activations), then enqueues
`launches` back-to-back launches of each hot kernel in turn through
mit2cfm_profile_launch, in this order:

    0 w13 (FFN w1|w3 + SwiGLU)   1 WaveNet k=5 conv + gate   2 QKV + RoPE
    3 w2 + residual               4 attention                  5 AdaRMSNorm
    6 wo + residual + norm        7 WaveNet res/skip

Under `rocprofv3 --pmc ...` or `--kernel-trace` the last 8 * launches
dispatches are these launches, kernel by kernel.

    python3 index-tts2-metal_amd/profile_kernels.py [--tokens 860] [--prompt 258]
        [--cfm-steps 25] [--launches 20] [--decodes 1]
"""
from __future__ import annotations

import argparse
import sys
import time
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))

import mit2cfm  # noqa: E402

KERNELS = ["w13", "conv", "qkv", "w2", "attention", "adarms", "wo", "resskip"]


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--tokens", type=int, default=860)
    p.add_argument("--prompt", type=int, default=258)
    p.add_argument("--cfm-steps", type=int, default=25)
    p.add_argument("--launches", type=int, default=20)
    p.add_argument("--decodes", type=int, default=1)
    a = p.parse_args()
    T, P = a.tokens, a.prompt
    with mit2cfm.Context(mit2cfm.synthetic_tensors(20240605, 0.02), device=0) as ctx:
        x0 = mit2cfm.normal_noise(T, 80, 1)
        cond = mit2cfm.normal_noise(T, 512, 2)
        style = mit2cfm.normal_noise(1, 192, 3)[0]
        prompt = mit2cfm.normal_noise(P, 80, 4, 2.0) - 5.0
        for _ in range(a.decodes):
            t0 = time.perf_counter()
            ctx.decode(x0, prompt, cond, style, a.cfm_steps, 0.7)
            print(f"decode T={T} steps={a.cfm_steps}: {1e3 * (time.perf_counter() - t0):.2f} ms", flush=True)
        for kid, short in enumerate(KERNELS):
            name, flops, nbytes = ctx.profile_launch(kid, a.launches)
            ctx.synchronize()
            print(f"kernel {kid} {short} ({name}) x{a.launches}: {flops:.4g} FLOP, {nbytes:.4g} B per launch",
                  flush=True)
    print("done", flush=True)


if __name__ == "__main__":
    main()
