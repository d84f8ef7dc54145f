"""Small helpers shared by the tests (tensor <-> numpy for the oracle)."""
from __future__ import annotations

import numpy as np
import torch

BF16_TOL = dict(atol=1e-2, rtol=1e-2)  # attention outputs vs the fp64 oracle


def to_np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit patterns of a 2-byte tensor (bit-exact comparisons)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def assert_close_bf16(actual: torch.Tensor, expected: np.ndarray, atol=1e-2, rtol=1e-2):
    a = to_np64(actual)
    np.testing.assert_allclose(a, expected, atol=atol, rtol=rtol)


class TorchOps:
    """The decoder op set (aios_amd.layers.HipOps interface) as plain torch
    math: the reference formulas of layers/norm.py:18-40 (fp32),
    models/qwen3.py:65-66 + layers/attention.py:11-16 (bf16 RoPE products
    when the input is bf16) and layers/activation.py:9-12.  Test helper."""

    @staticmethod
    def _norm(x, weight, eps):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)

    def rmsnorm(self, x, weight, eps):
        return self._norm(x, weight, eps)

    def fused_add_rmsnorm(self, x, residual, weight, eps):
        r = x.float() + residual.float()
        y = r * torch.rsqrt(r.pow(2).mean(-1, keepdim=True) + eps) * weight.float()
        residual.copy_(r.to(residual.dtype))
        x.copy_(y.to(x.dtype))
        return x, residual

    def qk_norm_rope(self, qkv, q_weight, k_weight, cos, sin, positions, hq, hkv, d, eps):
        t = qkv.shape[0]
        q = self._norm(qkv[:, : hq * d].reshape(t, hq, d), q_weight, eps)
        k = self._norm(qkv[:, hq * d : (hq + hkv) * d].reshape(t, hkv, d), k_weight, eps)
        c = cos[positions.long()].unsqueeze(1).to(q.dtype)
        s = sin[positions.long()].unsqueeze(1).to(q.dtype)

        def rot(x):
            x1, x2 = x.chunk(2, dim=-1)
            return torch.cat((-x2, x1), dim=-1)

        return q * c + rot(q) * s, k * c + rot(k) * s

    def attnres_mix(self, bank, partial, weighted_query, eps):
        """kernel/attnres.py:8-127: fp32 RMS scores, fp32 softmax, weights
        rounded to the bank dtype, fp32 weighted sum."""
        src = bank if partial is None else torch.cat((bank, partial[None]), 0)
        x = src.float()
        sc = (x * weighted_query.float()).sum(-1) * torch.rsqrt(x.pow(2).mean(-1) + eps)
        w = sc.softmax(0).to(bank.dtype).float()
        return (w[:, :, None] * x).sum(0).to(bank.dtype)

    def attnres_mix_step(self, bank, partial, delta, weighted_query, eps, partial_out):
        partial_out.copy_(delta if partial is None else partial + delta)
        return self.attnres_mix(bank, partial_out, weighted_query, eps)

    def silu_and_mul(self, x):
        g, u = x.chunk(2, dim=-1)
        return torch.nn.functional.silu(g) * u

    def linear(self, x, weight):
        return torch.nn.functional.linear(x, weight)

    def add_rmsnorm_linear(self, h, residual, norm_weight, eps, weight, silu=False):
        if residual is None:
            x = self.rmsnorm(h, norm_weight, eps)
            residual = h
        else:
            x, residual = self.fused_add_rmsnorm(h.clone(), residual.clone(), norm_weight, eps)
        y = self.linear(x, weight)
        return (self.silu_and_mul(y) if silu else y), residual
