"""Independent float64 restatement of the DiT-CFM estimator from PyTorch library ops.

Used only to pin the oracle: every operator here is a torch library routine
(F.linear, F.rms_norm, F.layer_norm, F.scaled_dot_product_attention,
F.conv1d on an F.pad(mode="reflect") input, torch._weight_norm, complex
multiplication for RoPE), so a mistake in the oracle's hand-written loops
(a dropped term, a transposed operand, a wrong index or sign) shows up as a
mismatch.  Only the wiring between the ops follows the reference
(runtime/impl/dit_cfm_bigvgan.cpp:1-1788, 2908-2937).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

PFX = "s2mel.net.cfm.estimator."


class TorchEstimator:
    def __init__(self, tensors: dict[str, np.ndarray]):
        self.w = {k[len(PFX):]: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in tensors.items()}

    def W(self, name: str) -> torch.Tensor:
        return self.w[name]

    # gpt.cpp:5404 (cos first, scale 1000)
    def timestep_embedder(self, t: float, which: int) -> torch.Tensor:
        p = "t_embedder" if which == 1 else "t_embedder2"
        args = 1000.0 * t * self.W(p + ".freqs")
        e = torch.cat([torch.cos(args), torch.sin(args)])
        h = F.silu(F.linear(e, self.W(p + ".mlp.0.weight"), self.W(p + ".mlp.0.bias")))
        return F.linear(h, self.W(p + ".mlp.2.weight"), self.W(p + ".mlp.2.bias"))

    def adaptive_norm(self, x, t1, prefix: str) -> torch.Tensor:
        wb = F.linear(t1, self.W(prefix + ".project_layer.weight"), self.W(prefix + ".project_layer.bias"))
        n = F.rms_norm(x, (512,), weight=self.W(prefix + ".norm.weight"), eps=1e-5)
        return wb[:512] * n + wb[512:]

    @staticmethod
    def rope(x: torch.Tensor) -> torch.Tensor:
        """Pairs (2i, 2i+1) of each 64-wide head rotated by t / 10000^(2i/64)."""
        T = x.shape[0]
        xc = torch.view_as_complex(x.reshape(T, 8, 32, 2).contiguous())
        pos = torch.arange(T, dtype=torch.float64)[:, None]
        inv = 10000.0 ** (-(2.0 * torch.arange(32, dtype=torch.float64)) / 64.0)
        rot = torch.polar(torch.ones(T, 32, dtype=torch.float64), pos * inv)
        return torch.view_as_real(xc * rot[:, None, :]).reshape(T, 512)

    def attention_core(self, x, mask, layer: int) -> torch.Tensor:
        b = f"transformer.layers.{layer}.attention"
        T = x.shape[0]
        q, k, v = F.linear(x, self.W(b + ".wqkv.weight")).split(512, dim=-1)
        q, k = self.rope(q), self.rope(k)
        heads = lambda z: z.reshape(T, 8, 64).transpose(0, 1)
        keep = torch.as_tensor(np.asarray(mask) != 0)
        o = F.scaled_dot_product_attention(heads(q), heads(k), heads(v), attn_mask=keep[None, None, :])
        return F.linear(o.transpose(0, 1).reshape(T, 512), self.W(b + ".wo.weight"))

    def feed_forward(self, x, layer: int) -> torch.Tensor:
        b = f"transformer.layers.{layer}.feed_forward"
        h = F.silu(F.linear(x, self.W(b + ".w1.weight"))) * F.linear(x, self.W(b + ".w3.weight"))
        return F.linear(h, self.W(b + ".w2.weight"))

    def block(self, x, t1, mask, layer: int, skip=None) -> torch.Tensor:
        b = f"transformer.layers.{layer}"
        if skip is not None:
            x = F.linear(torch.cat([x, skip], -1), self.W(b + ".skip_in_linear.weight"),
                         self.W(b + ".skip_in_linear.bias"))
        h = x + self.attention_core(self.adaptive_norm(x, t1, b + ".attention_norm"), mask, layer)
        return h + self.feed_forward(self.adaptive_norm(h, t1, b + ".ffn_norm"), layer)

    def stack(self, x, t1, mask) -> torch.Tensor:
        saved = []
        for layer in range(13):
            skip = saved.pop() if layer > 6 else None
            x = self.block(x, t1, mask, layer, skip)
            if layer < 6:
                saved.append(x)
        return self.adaptive_norm(x, t1, "transformer.norm")

    def input_merge(self, x, prompt_x, cond, style) -> torch.Tensor:
        cp = F.linear(cond, self.W("cond_projection.weight"), self.W("cond_projection.bias"))
        T = x.shape[0]
        row = torch.cat([x, prompt_x, cp, style.expand(T, 192)], -1)
        return F.linear(row, self.W("cond_x_merge_linear.weight"), self.W("cond_x_merge_linear.bias"))

    def post(self, xres, xmel):
        ls = F.linear(torch.cat([xres, xmel], -1), self.W("skip_linear.weight"), self.W("skip_linear.bias"))
        c1 = F.linear(ls, self.W("conv1.weight"), self.W("conv1.bias"))
        rp = F.linear(ls, self.W("res_projection.weight"), self.W("res_projection.bias"))
        return ls, c1, rp

    def _wn(self, prefix: str) -> torch.Tensor:
        return torch._weight_norm(self.W(prefix + ".weight_v"), self.W(prefix + ".weight_g"), 0)

    def wavenet(self, x, t2, mask) -> torch.Tensor:
        m = torch.as_tensor(np.asarray(mask) != 0, dtype=torch.float64)[:, None]
        cp = "wavenet.cond_layer.conv.conv"
        cond = F.conv1d(t2[None, :, None], self._wn(cp), self.W(cp + ".bias"))[0, :, 0]
        out = torch.zeros_like(x)
        for layer in range(8):
            ip = f"wavenet.in_layers.{layer}.conv.conv"
            xin = F.pad(x.T[None], (2, 2), mode="reflect")
            y = F.conv1d(xin, self._wn(ip), self.W(ip + ".bias"))[0].T
            c = cond[layer * 1024:(layer + 1) * 1024]
            g = torch.tanh(y[:, :512] + c[:512]) * torch.sigmoid(y[:, 512:] + c[512:])
            rp = f"wavenet.res_skip_layers.{layer}.conv.conv"
            rs = F.conv1d(g.T[None], self._wn(rp), self.W(rp + ".bias"))[0].T
            if layer < 7:
                x = (x + rs[:, :512]) * m
                out = out + rs[:, 512:]
            else:
                out = out + rs
        return out * m

    def final_layer(self, x, t1) -> torch.Tensor:
        ss = F.linear(F.silu(t1), self.W("final_layer.adaLN_modulation.1.weight"),
                      self.W("final_layer.adaLN_modulation.1.bias"))
        y = F.layer_norm(x, (512,), eps=1e-6) * (1.0 + ss[512:]) + ss[:512]
        w = torch._weight_norm(self.W("final_layer.linear.weight_v"), self.W("final_layer.linear.weight_g"), 0)
        return F.linear(y, w, self.W("final_layer.linear.bias"))

    def estimator_step(self, x, prompt_x, cond, style, t: float, mask) -> torch.Tensor:
        t1 = self.timestep_embedder(t, 1)
        t2 = self.timestep_embedder(t, 2)
        xin = self.input_merge(x, prompt_x, cond, style)
        xres = self.stack(xin, t1, mask)
        _, c1, rp = self.post(xres, x)
        fin = self.wavenet(c1, t2, mask) + rp
        h = self.final_layer(fin, t1)
        return F.conv1d(h.T[None], self.W("conv2.weight"), self.W("conv2.bias"))[0].T

    def cfm_euler(self, x0, prompt, cond, style, steps: int, cfg: float) -> torch.Tensor:
        x = x0.clone()
        T = x.shape[0]
        P = prompt.shape[0]
        px = torch.zeros(T, 80, dtype=torch.float64)
        px[:P] = prompt
        x[:P] = 0
        mask = np.ones(T, np.uint32)
        zeros80 = torch.zeros(T, 80, dtype=torch.float64)
        zeros512 = torch.zeros(T, 512, dtype=torch.float64)
        zeros192 = torch.zeros(192, dtype=torch.float64)
        for s in range(steps):
            t = s / steps
            d = self.estimator_step(x, px, cond, style, t, mask)
            if cfg > 0:
                dn = self.estimator_step(x, zeros80, zeros512, zeros192, t, mask)
                d = (1 + cfg) * d - cfg * dn
            x = x + d / steps
            x[:P] = 0
        return x


def t64(a) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, dtype=np.float64))
